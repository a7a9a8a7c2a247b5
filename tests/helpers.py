"""Shared helpers for the GPU parity tests (no GPU work at import time)."""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden")
for p in (ROOT, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)

import inputs as gi  # noqa: E402
from oracle import oracle  # noqa: E402

# bf16 outputs vs the fp32 reference
RTOL, ATOL = 2e-2, 2e-3


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (round to nearest even) and return them as fp32."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def dev():
    return torch.device("cuda:0")


def to_gpu(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev())


def make_module(pkg, w: dict, tau: float, bias=None):
    """TauSparseMoE on cuda:0 loaded from masked-layout weights (load_from_masked)."""
    I, H = w["w_gate"].shape
    E = w["w_router"].shape[0]
    G = I // E
    m = pkg.TauSparseMoE(H, I, E, G, tau,
                         router_bias=None if bias is None else torch.as_tensor(bias, dtype=torch.float32))
    m = m.to(dev())
    m.load_from_masked(to_gpu(w["w_gate"]), to_gpu(w["w_up"]), to_gpu(w["w_down"]), to_gpu(w["w_router"]),
                       to_gpu(w["expert_ids"]))
    return m


def sparse_expected(x: np.ndarray, w: dict, gates: np.ndarray, act_bf16: bool = False) -> np.ndarray:
    """float64 layer output from a given selection, on bf16-rounded x and weights
    (what the kernels consume); act_bf16 rounds the acts to bf16 before the down
    projection, as the reference's fused expert kernel does."""
    E = w["w_router"].shape[0]
    I = w["w_gate"].shape[0]
    G = I // E
    perm = oracle.pack_permutation(w["expert_ids"])
    return oracle.sparse_moe_from_selection(bf16_round(x), bf16_round(w["w_gate"])[perm],
                                            bf16_round(w["w_up"])[perm], bf16_round(w["w_down"])[:, perm].T,
                                            gates, G, act_bf16=act_bf16)


def sparse_expected_gpu(x: np.ndarray, w: dict, gates: np.ndarray, act_bf16: bool = False) -> np.ndarray:
    """sparse_expected in torch float64 on cuda:0, for sizes where the numpy restatement
    is slow (e.g. 8200 tokens): every expert's SwiGLU on every token, times the gate
    (0 for unselected experts, so those terms vanish exactly), down projection. Same
    operands as sparse_expected (bf16-rounded x and weights, rearranged neurons);
    test_prefill_full_rows pins it against sparse_expected on a slice. act_bf16 rounds
    the acts to bf16 before the down projection, as the reference's fused expert kernel
    does (src/tl_kernel_optimized_Ultimate_PanGU.py:321)."""
    E = w["w_router"].shape[0]
    I = w["w_gate"].shape[0]
    G = I // E
    perm = oracle.pack_permutation(w["expert_ids"])
    d = dev()

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(d, torch.float64)

    xr = t(bf16_round(x))
    WgT = t(bf16_round(w["w_gate"])[perm].T)        # [H, I], contiguous right operands
    WuT = t(bf16_round(w["w_up"])[perm].T)
    WdT = t(bf16_round(w["w_down"])[:, perm].T)     # [I, H]
    g = xr @ WgT
    a = g / (1.0 + torch.exp(-g)) * (xr @ WuT) * t(gates).repeat_interleave(G, dim=1)
    if act_bf16:
        a = a.to(torch.float32).to(torch.bfloat16).to(torch.float64)
    return (a @ WdT).cpu().numpy()


def assert_close_fp32(got: np.ndarray, ref32: np.ndarray, ref_q: np.ndarray, what=""):
    """bf16 output vs the fp32 reference (original fp32 weights and x).

    Casting the weights and x to bf16 (BASELINE: bf16 weights) moves the exact result
    by |ref_q - ref32| per element, where ref_q is the float64 result on the bf16
    operands; on the config-1 layer that alone exceeds rtol 2e-2 / atol 2e-3 on ~0.4%
    of the elements. The bound is therefore rtol/atol plus that measured quantization
    term, and the normwise relative error must stay below 1e-2."""
    got = np.asarray(got, np.float64)
    ref32 = np.asarray(ref32, np.float64)
    q = np.abs(np.asarray(ref_q, np.float64) - ref32)
    err = np.abs(got - ref32)
    bad = err > ATOL + RTOL * np.abs(ref32) + q
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} outside rtol/atol + bf16 quantization; first at "
                             f"{tuple(i)}: got {got[tuple(i)]} ref {ref32[tuple(i)]} q {q[tuple(i)]}")
    rel = np.linalg.norm(got - ref32) / max(np.linalg.norm(ref32), 1e-30)
    assert rel < 1e-2, f"{what}: normwise relative error {rel:.3e}"


def assert_close(got: np.ndarray, ref: np.ndarray, rtol=RTOL, atol=ATOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} outside rtol={rtol} atol={atol}; "
                             f"first at {tuple(i)}: got {got[tuple(i)]} ref {ref[tuple(i)]}; "
                             f"max abs err {err.max():.3e}")


def abi_prefill(pkg, m, xs, E, G, tau=0.7, routed=True):
    """pp_moe_prefill_routed through the C ABI on the module's buffers: (out bf16 [n,H],
    logits fp32 [n,E], mask uint8 [n,E]) -- the routing the call itself used (routed=False:
    no routing outputs requested)."""
    import ctypes
    n, H = xs.shape
    y = torch.empty(n, H, dtype=torch.bfloat16, device=xs.device)
    lg = torch.empty(n, E, dtype=torch.float32, device=xs.device)
    mk = torch.empty(n, E, dtype=torch.uint8, device=xs.device)
    ws = torch.empty(pkg.ops.prefill_workspace_bytes(n, H, E, G), dtype=torch.uint8, device=xs.device)
    vp = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    lib = pkg._lib.lib()
    xc = 0 if xs.dtype == torch.float32 else 1
    pkg._lib.check(lib.pp_moe_prefill_routed(vp(xs), xc, n, H, vp(m.router_packed), vp(m.router_bias), E, G,
                                             ctypes.c_float(tau), vp(m.packed_experts), vp(y), vp(ws),
                                             vp(lg if routed else None), vp(mk if routed else None),
                                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                   "moe_prefill_routed")
    return y, lg, mk
