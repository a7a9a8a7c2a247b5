"""CPU oracle for the PrunePath sparse-MoE MLP path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker / CPU baseline. The product
package never imports it and has no CPU fallback.

Contents and the reference lines each function restates (paths relative to the
reference repository root):

* ``softmax``, ``select`` -- ``softmax_thresholding``
  (src/MoEBlock_origin.py:50-97). Bit-level torch-CPU recipe in
  ``oracle/route_oracle.c`` (C, strict IEEE, explicit fma).
* ``bucket`` -- canonical layout derived from ``moe_local_scan_kernel`` /
  ``moe_global_scan_kernel`` / ``moe_dispatch_kernel``
  (src/tl_kernel_optimized_Ultimate_PanGU.py:133-266): experts ascending,
  tokens ascending inside each expert.
* ``pack_permutation`` -- ``physical_reorder_for_inference``
  (src/openpangu_moe.py:228-243); stable order inside an expert (the reference
  uses an unstable argsort, so its in-expert order is unspecified and the MLP
  output does not depend on it).
* ``masked_moe_mlp`` -- the dense masked MoE-MLP layer
  ``IntegratedOpenPanguMoEMLP.forward`` (src/openpangu_moe_origin.py:96-118)
  with ``MoELayer.forward`` (src/MoEBlock_origin.py:188-212): dense SwiGLU over
  all neurons, router, tau mask, ``intermediate * (gates @ experts_masks)``,
  down projection.
* ``sparse_moe_from_selection`` -- the same layer evaluated sparsely from a
  given selection, in float64, on caller-given (e.g. bf16-rounded) weights;
  optionally with the acts rounded to bf16 before the down projection, the
  rounding point of the reference's fused expert kernel
  (src/tl_kernel_optimized_Ultimate_PanGU.py:318).
* ``bf16_rne`` -- float32 to bfloat16, round to nearest even (torch's conversion).

Pinning (tests/test_oracle.py): softmax/select bits against torch CPU ops in the
container (same torch 2.10 the reference pins, requirements.txt:3) and against
committed golden fixtures; bucket against brute force; masked MLP against the
sparse form and against a float64 direct sum; bf16_rne against torch's conversion
(ties, subnormals, overflow, NaN) and the bf16-act form against the exact one within
the half-ulp bound; the permutation against the
reference-held cluster maps (src/Pangu_Clusters/*.txt).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile oracle/liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        ip = ctypes.POINTER(ctypes.c_int32)
        bp = ctypes.POINTER(ctypes.c_uint8)
        lib.oracle_expf_u10.argtypes = [ctypes.c_float]
        lib.oracle_expf_u10.restype = ctypes.c_float
        lib.oracle_sigmoid.argtypes = [ctypes.c_float]
        lib.oracle_sigmoid.restype = ctypes.c_float
        lib.oracle_softmax_rows.argtypes = [fp, ctypes.c_int64, ctypes.c_int32, fp]
        lib.oracle_softmax_rows.restype = None
        lib.oracle_select_rows.argtypes = [fp, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
                                           fp, fp, bp, ip, ip]
        lib.oracle_select_rows.restype = None
        lib.oracle_bucket.argtypes = [bp, fp, ctypes.c_int64, ctypes.c_int32, ip, ip, fp, ip]
        lib.oracle_bucket.restype = None
        lib.oracle_sort_desc.argtypes = [fp, ctypes.c_int32, ip]
        lib.oracle_sort_desc.restype = None
        _lib = lib
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def expf_u10(x) -> np.ndarray:
    lib = _load()
    x = np.asarray(x, dtype=np.float32)
    out = np.empty_like(x)
    flat, oflat = x.reshape(-1), out.reshape(-1)
    for i in range(flat.size):
        oflat[i] = lib.oracle_expf_u10(float(flat[i]))
    return out


def softmax(logits: np.ndarray) -> np.ndarray:
    """torch.softmax(logits, -1) on CPU fp32, bit for bit."""
    lib = _load()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    E = x.shape[-1]
    n = x.size // E if E else 0
    out = np.empty_like(x)
    if n:
        lib.oracle_softmax_rows(_ptr(x, ctypes.c_float), n, E, _ptr(out, ctypes.c_float))
    return out


def sort_desc(p: np.ndarray) -> np.ndarray:
    """Index order of torch.sort(p, descending=True) on CPU for each row of p
    (libstdc++ introsort tie order; stable for rows of at most 16)."""
    lib = _load()
    x = np.ascontiguousarray(p, dtype=np.float32)
    E = x.shape[-1]
    x2 = x.reshape(-1, E)
    out = np.empty(x2.shape, np.int32)
    for r in range(x2.shape[0]):
        lib.oracle_sort_desc(_ptr(x2[r], ctypes.c_float), E, _ptr(out[r], ctypes.c_int32))
    return out.reshape(x.shape)


class Selection:
    """Result of tau selection for n tokens over E experts."""

    def __init__(self, probs, gates, mask, ranked, count):
        self.probs = probs      # [n, E] fp32 softmax
        self.gates = gates      # [n, E] fp32, sigmoid(logit) on selected experts, else 0
        self.mask = mask        # [n, E] uint8
        self.ranked = ranked    # [n, E] int32, expert ids by descending probability
        self.count = count      # [n] int32, selected experts per token


def select(logits: np.ndarray, tau: float) -> Selection:
    """softmax_thresholding(logits, tau) (src/MoEBlock_origin.py:50-97) on [n, E] fp32 logits."""
    lib = _load()
    x = np.ascontiguousarray(logits, dtype=np.float32)
    E = x.shape[-1]
    x2 = x.reshape(-1, E)
    n = x2.shape[0]
    probs = np.empty((n, E), np.float32)
    gates = np.empty((n, E), np.float32)
    mask = np.empty((n, E), np.uint8)
    ranked = np.empty((n, E), np.int32)
    count = np.empty((n,), np.int32)
    if n:
        lib.oracle_select_rows(_ptr(x2, ctypes.c_float), n, E, float(np.float32(tau)),
                               _ptr(probs, ctypes.c_float), _ptr(gates, ctypes.c_float),
                               _ptr(mask, ctypes.c_uint8), _ptr(ranked, ctypes.c_int32),
                               _ptr(count, ctypes.c_int32))
    return Selection(probs, gates, mask, ranked, count)


class Buckets:
    def __init__(self, offsets, token_ids, pair_gates, token_pairs):
        self.offsets = offsets          # [E+1] int32
        self.token_ids = token_ids      # [P] int32
        self.pair_gates = pair_gates    # [P] fp32
        self.token_pairs = token_pairs  # [n, E] int32, -1 padded


def bucket(mask: np.ndarray, gates: np.ndarray | None = None) -> Buckets:
    """Canonical token->expert CSR layout (experts ascending, tokens ascending)."""
    lib = _load()
    m = np.ascontiguousarray(mask, dtype=np.uint8)
    n, E = m.shape
    g = np.ascontiguousarray(gates if gates is not None else np.zeros((n, E)), dtype=np.float32)
    P = int(m.astype(np.int64).sum())
    offsets = np.empty((E + 1,), np.int32)
    token_ids = np.empty((max(P, 1),), np.int32)
    pair_gates = np.empty((max(P, 1),), np.float32)
    token_pairs = np.empty((n, E), np.int32)
    lib.oracle_bucket(_ptr(m, ctypes.c_uint8), _ptr(g, ctypes.c_float), n, E,
                      _ptr(offsets, ctypes.c_int32), _ptr(token_ids, ctypes.c_int32),
                      _ptr(pair_gates, ctypes.c_float), _ptr(token_pairs, ctypes.c_int32))
    return Buckets(offsets, token_ids[:P], pair_gates[:P], token_pairs)


def pack_permutation(expert_ids: np.ndarray) -> np.ndarray:
    """Neuron order after rearrangement: stable argsort of neuron->expert ids
    (src/openpangu_moe.py:230-231). Rearranged neuron j is original neuron perm[j]."""
    ids = np.asarray(expert_ids, dtype=np.int64)
    return np.argsort(ids, kind="stable")


def _silu64(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def masked_moe_mlp(x, w_gate, w_up, w_down, w_router, expert_ids, tau, bias=None,
                   logits=None):
    """Dense masked MoE-MLP layer (src/openpangu_moe_origin.py:96-118 with
    src/MoEBlock_origin.py:188-212), evaluated in float64 from fp32 inputs.

    x [n,H]; w_gate/w_up [I,H] (nn.Linear layout); w_down [H,I]; w_router [E,H];
    expert_ids [I] neuron->expert. Routing uses fp32 logits ``x @ w_router.T (+bias)``
    unless ``logits`` is given. Returns (out [n,H] float64, Selection).
    """
    x = np.asarray(x, np.float32)
    if logits is None:
        logits = (x.astype(np.float64) @ np.asarray(w_router, np.float64).T)
        if bias is not None:
            logits = logits + np.asarray(bias, np.float64)
        logits = logits.astype(np.float32)
    sel = select(logits, tau)
    E = sel.gates.shape[1]
    x64 = x.astype(np.float64)
    gate = _silu64(x64 @ np.asarray(w_gate, np.float64).T)
    up = x64 @ np.asarray(w_up, np.float64).T
    inter = gate * up
    onehot = (np.asarray(expert_ids)[None, :] == np.arange(E)[:, None]).astype(np.float64)
    moe_mask = sel.gates.astype(np.float64) @ onehot
    out = (inter * moe_mask) @ np.asarray(w_down, np.float64).T
    return out, sel


def bf16_rne(a) -> np.ndarray:
    """float32 values rounded to bfloat16 (round to nearest, ties to even; NaN stays a
    quiet NaN), returned as float32 -- torch's ``.to(torch.bfloat16)``."""
    f = np.ascontiguousarray(a, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(np.isnan(f), np.uint32(0x7FC00000), r)
    return r.view(np.float32)


def sparse_moe_from_selection(x, gate_rows, up_rows, down_cols, gates, G, act_bf16=False):
    """Sparse evaluation of the same layer in float64 from a given selection.

    x [n,H]; gate_rows/up_rows [I,H] rearranged (expert e owns rows e*G:(e+1)*G);
    down_cols [I,H] rearranged down weights (row j = column j of down_proj);
    gates [n,E] (0 where not selected). Returns out [n,H] float64.
    act_bf16: round each act = silu(g) * u * gate to bfloat16 before the down projection,
    as the reference's fused expert kernel does (``acc_gate.to(tl.bfloat16)``,
    src/tl_kernel_optimized_Ultimate_PanGU.py:318).
    """
    x64 = np.asarray(x, np.float64)
    g = np.asarray(gates, np.float64)
    n, E = g.shape
    H = x64.shape[1]
    out = np.zeros((n, H), np.float64)
    Wg = np.asarray(gate_rows, np.float64)
    Wu = np.asarray(up_rows, np.float64)
    Wd = np.asarray(down_cols, np.float64)
    for e in range(E):
        toks = np.nonzero(g[:, e] != 0)[0]
        if toks.size == 0:
            continue
        sl = slice(e * G, (e + 1) * G)
        xe = x64[toks]
        act = _silu64(xe @ Wg[sl].T) * (xe @ Wu[sl].T) * g[toks, e][:, None]
        if act_bf16:
            act = bf16_rne(act.astype(np.float32)).astype(np.float64)
        out[toks] += act @ Wd[sl]
    return out
