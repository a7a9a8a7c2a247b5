"""Torch-level entry points over the C ABI (include/prunepath_moe.h).

PyTorch only provides device memory and the current HIP stream here. The hot-path
ops -- ``route``, ``route_logits``, ``bucket``, ``pack_experts``, ``pack_router``,
``decode_workspace_init``, ``moe_decode``, ``moe_prefill`` -- are ``torch.library``
ops of the C++ extension ``libprunepath_torch.so`` (csrc/torch_ops.cpp, namespace
``prunepath``: ``torch.ops.prunepath.route`` etc.), which checks arguments, allocates
outputs and calls the C ABI; the functions below only adapt their results to
dicts / defaults. The test-level stage entry points (``expert_gateup``,
``expert_down``, ``combine``) and the masked-gate training kernels call the C ABI
through ctypes. All work is enqueued on ``torch.cuda.current_stream()``; nothing
synchronises with the host, so the calls can be captured in a CUDA (HIP) graph.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib as L


def _vp(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need_gpu(name: str, *ts: Optional[torch.Tensor]) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"prunepath.{name}: tensors must be on the GPU (got {t.device}); "
                               "there is no CPU implementation")
        if not t.is_contiguous():
            raise RuntimeError(f"prunepath.{name}: tensors must be contiguous")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"prunepath.{name}: tensors on different devices ({dev}, {t.device})")


# ----------------------------------------------------------------------------- rearrangement
def packed_expert_numel(H: int, E: int, G: int) -> int:
    return int(L.lib().pp_packed_expert_bytes(H, E, G)) // 2


def pack_experts(w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor, E: int, G: int,
                 perm: Optional[torch.Tensor] = None, layout: str = "linear") -> torch.Tensor:
    """One-time physical rearrangement (physical_reorder_for_inference,
    src/openpangu_moe.py:212-256) into the packed bf16 expert buffer
    (``torch.ops.prunepath.pack_experts``).

    layout="linear": nn.Linear weights, gate/up [I,H], down [H,I].
    layout="tau":    TauSparseMoE buffers, W_gate/W_up [H,I], W_down [I,H].
    perm[j] (int32, device) = source neuron of rearranged neuron j (None = identity).
    """
    return L.torch_ops().pack_experts(w_gate, w_up, w_down, E, G, perm, layout)


def pack_router(w_router: torch.Tensor, layout: str = "linear") -> torch.Tensor:
    """Router weights to fp32 [Epad, H] (Epad = E rounded up to 16, zero rows).
    layout="linear": MoELayer router weight [E,H]; layout="tau": TauSparseMoE.router [H,E]."""
    return L.torch_ops().pack_router(w_router, layout)


# ----------------------------------------------------------------------------- routing
def route(x: torch.Tensor, router_packed: torch.Tensor, E: int, tau: float,
          bias: Optional[torch.Tensor] = None, want_logits: bool = True, want_probs: bool = False):
    """fp32 router + tau selection for x [N,H] (``torch.ops.prunepath.route``). Returns dict
    with gates [N,E] fp32, mask [N,E] uint8, count [N] int32, logits and probs [N,E] fp32
    (None unless asked for)."""
    if x.dtype not in (torch.float32, torch.bfloat16) and x.is_floating_point():
        x = x.float()
    logits, probs, gates, mask, count = L.torch_ops().route(x, router_packed, bias, E, float(tau))
    return {"gates": gates, "mask": mask, "count": count, "logits": logits if want_logits else None,
            "probs": probs if want_probs else None}


def route_logits(logits: torch.Tensor, tau: float):
    """Tau selection from given fp32 logits [N,E] (bit-exact with torch CPU
    softmax_thresholding, src/MoEBlock_origin.py:50-97; ``torch.ops.prunepath.route_logits``).
    Returns (probs, gates, mask, count)."""
    return L.torch_ops().route_logits(logits, float(tau))


# ----------------------------------------------------------------------------- bucketing
def gemm_tile_m() -> int:
    return int(L.lib().pp_gemm_tile_m())


def max_tiles(N: int, E: int, tile_m: Optional[int] = None) -> int:
    return int(L.lib().pp_max_tiles(N, E, tile_m or gemm_tile_m()))


def bucket(mask: torch.Tensor, gates: torch.Tensor, tile_m: Optional[int] = None):
    """Token -> expert CSR layout, experts ascending, tokens ascending inside an expert
    (``torch.ops.prunepath.bucket``). Returns dict: offsets [E+1], token_ids [N*E],
    pair_gates [N*E], token_pairs [N,E], tiles [max_tiles,4], meta [4] (all int32 except
    pair_gates fp32) and max_tiles. Only the first offsets[E] entries of token_ids /
    pair_gates and the first meta[0] tiles are valid."""
    off, tok, pg, tp, tiles, meta = L.torch_ops().bucket(mask, gates, int(tile_m or 0))
    return {"offsets": off, "token_ids": tok, "pair_gates": pg, "token_pairs": tp, "tiles": tiles, "meta": meta,
            "max_tiles": max_tiles(mask.shape[0], mask.shape[1], tile_m)}


# ----------------------------------------------------------------------------- decode
def decode_workspace(H: int, E: int, device) -> torch.Tensor:
    """Allocate and zero (with a kernel, once) a decode workspace."""
    n = int(L.lib().pp_decode_workspace_bytes(H, E))
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    return decode_workspace_init(ws, H, E)


def decode_workspace_init(ws: torch.Tensor, H: int, E: int) -> torch.Tensor:
    """Zero a decode workspace in place (first use, or to clear its error flag)."""
    L.torch_ops().decode_workspace_init(ws, H, E)
    return ws


def decode_state(ws: torch.Tensor, E: int) -> dict:
    """Read the pp_decode_state header of a decode workspace (synchronises)."""
    hdr = ws[:16 + 16 + 3 * 4 * 256].cpu()
    u32 = hdr[:32].view(torch.int32)
    k = int(u32[4])
    body = hdr[32:]
    logits = body[:1024].view(torch.float32)[:E].clone()
    ids = body[1024:2048].view(torch.int32)[:k].clone()
    gts = body[2048:3072].view(torch.float32)[:k].clone()
    return {"error": int(u32[3]), "k": k, "logits": logits, "sel_ids": ids, "sel_gates": gts,
            "router_ticket": int(u32[0]), "epoch16": int(u32[1]), "epochb": int(u32[2]),
            "layout": int(u32[6]) & 0xffffffff}


def moe_decode(x: torch.Tensor, router_packed: torch.Tensor, bias: Optional[torch.Tensor], E: int, G: int,
               tau: float, packed: torch.Tensor, workspace: torch.Tensor, grid: int = 0,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused single-token MoE-MLP layer (``torch.ops.prunepath.moe_decode``, or
    ``moe_decode_into`` writing ``out``). x [H] or [1,H]; returns bf16 [1,H]."""
    x = x.reshape(1, -1)
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    if out is None:
        return L.torch_ops().moe_decode(x, router_packed, bias, E, G, float(tau), packed, workspace, int(grid))
    L.torch_ops().moe_decode_into(x, router_packed, bias, E, G, float(tau), packed, workspace, out, int(grid))
    return out


# ----------------------------------------------------------------------------- small-batch decode
DECODE_BATCH_MAX = 64


def decode_batch_workspace_bytes(H: int, E: int, G: int) -> int:
    return int(L.lib().pp_decode_batch_workspace_bytes(H, E, G))


def decode_batch_supported(N: int, H: int, E: int, G: int) -> bool:
    """Shapes the one-launch small-batch kernel takes (the rest go through prefill)."""
    return 1 <= N <= DECODE_BATCH_MAX and E == 16 and H % 512 == 0 and 512 <= H <= 4096 and G % 32 == 0 and G <= 512


def moe_decode_batch(x: torch.Tensor, router_packed: torch.Tensor, bias: Optional[torch.Tensor], E: int, G: int,
                     tau: float, packed: torch.Tensor, workspace: torch.Tensor, batch_workspace: torch.Tensor,
                     grid: int = 0, out: Optional[torch.Tensor] = None, logits_out: Optional[torch.Tensor] = None,
                     mask_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Small-batch MoE-MLP layer in one launch (``torch.ops.prunepath.moe_decode_batch``,
    or ``moe_decode_batch_into`` writing ``out`` and, when given, the routing: logits
    [N,E] fp32 and mask [N,E] uint8). x [N,H] with N <= 64; ``workspace`` a decode
    workspace (``decode_workspace``), ``batch_workspace`` of
    ``decode_batch_workspace_bytes(H, E, G)`` bytes. Returns bf16 [N,H]."""
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    ops = L.torch_ops()
    if out is None and logits_out is None and mask_out is None:
        return ops.moe_decode_batch(x, router_packed, bias, E, G, float(tau), packed, workspace, batch_workspace,
                                    int(grid))
    if out is None:
        out = torch.empty(x.shape[0], x.shape[1], dtype=torch.bfloat16, device=x.device)
    ops.moe_decode_batch_into(x, router_packed, bias, E, G, float(tau), packed, workspace, batch_workspace, out,
                              logits_out, mask_out, int(grid))
    return out


# ----------------------------------------------------------------------------- prefill
def prefill_workspace_bytes(N: int, H: int, E: int, G: int) -> int:
    return int(L.lib().pp_prefill_workspace_bytes(N, H, E, G))


def moe_prefill(x: torch.Tensor, router_packed: torch.Tensor, bias: Optional[torch.Tensor], E: int, G: int,
                tau: float, packed: torch.Tensor, workspace: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, logits_out: Optional[torch.Tensor] = None,
                mask_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The prefill layer: x [N,H] -> bf16 [N,H]. G % 64 == 0: route -> bucket -> grouped
    gate/up GEMM (SwiGLU) -> grouped down GEMM -> combine; otherwise the dense form (router
    logits, selection, dense gate/up with the gate 0 for unselected experts, dense down).
    ``torch.ops.prunepath.moe_prefill`` (workspace from the caching allocator), or
    ``moe_prefill_into`` when a workspace, output or routing output (logits_out fp32 [N,E],
    mask_out uint8 [N,E]: the routing the call used) is given."""
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.float()
    ops = L.torch_ops()
    if workspace is None and out is None and logits_out is None and mask_out is None:
        return ops.moe_prefill(x, router_packed, bias, E, G, float(tau), packed)
    N, H = x.shape
    if workspace is None or workspace.numel() < prefill_workspace_bytes(N, H, E, G):
        workspace = torch.empty(prefill_workspace_bytes(N, H, E, G), dtype=torch.uint8, device=x.device)
    if out is None:
        out = torch.empty(N, H, dtype=torch.bfloat16, device=x.device)
    ops.moe_prefill_into(x, router_packed, bias, E, G, float(tau), packed, workspace, out, logits_out, mask_out)
    return out


def moe_prefill_routed(x: torch.Tensor, router_packed: torch.Tensor, bias: Optional[torch.Tensor], E: int, G: int,
                       tau: float, packed: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(out bf16 [N,H], logits fp32 [N,E], mask uint8 [N,E]): the prefill and the routing it used."""
    N = x.shape[0]
    logits = torch.empty(N, E, dtype=torch.float32, device=x.device)
    mask = torch.empty(N, E, dtype=torch.uint8, device=x.device)
    out = moe_prefill(x, router_packed, bias, E, G, tau, packed, logits_out=logits, mask_out=mask)
    return out, logits, mask


def expert_gateup(x_bf16: torch.Tensor, packed: torch.Tensor, E: int, G: int, bk: dict) -> torch.Tensor:
    """act [N*E, G] bf16 (rows = pairs in bucket order) from a bucket() layout."""
    N, H = x_bf16.shape
    _need_gpu("expert_gateup", x_bf16, packed)
    act = torch.empty(max(N * E, 1), G, dtype=torch.bfloat16, device=x_bf16.device)
    rc = L.lib().pp_expert_gateup(_vp(x_bf16), H, G, _vp(packed), E, _vp(bk["token_ids"]), _vp(bk["pair_gates"]),
                                  _vp(bk["tiles"]), _vp(bk["meta"]), bk["max_tiles"], _vp(act), _stream(x_bf16))
    L.check(rc, "expert_gateup")
    return act


def expert_down(act: torch.Tensor, packed: torch.Tensor, H: int, E: int, G: int, bk: dict) -> torch.Tensor:
    _need_gpu("expert_down", act, packed)
    y = torch.empty(act.shape[0], H, dtype=torch.float32, device=act.device)
    rc = L.lib().pp_expert_down(_vp(act), H, G, _vp(packed), E, _vp(bk["tiles"]), _vp(bk["meta"]),
                                bk["max_tiles"], _vp(y), _stream(act))
    L.check(rc, "expert_down")
    return y


def combine(y: torch.Tensor, token_pairs: torch.Tensor, count: torch.Tensor, H: int, E: int) -> torch.Tensor:
    N = token_pairs.shape[0]
    _need_gpu("combine", y, token_pairs, count)
    out = torch.empty(N, H, dtype=torch.bfloat16, device=y.device)
    rc = L.lib().pp_combine(_vp(y), _vp(token_pairs), _vp(count), N, H, E, _vp(out), _stream(y))
    L.check(rc, "combine")
    return out


# ----------------------------------------------------------------------------- masked gating
def masked_gate_layout(expert_ids: torch.Tensor, E: int):
    """(expert_ids int32, perm, seg) for the masked-gate kernels: perm = neurons sorted by
    expert id (stable), seg [E+1] = expert segment offsets in perm."""
    eid = expert_ids.to(torch.int32).contiguous()
    if eid.numel() and (int(eid.min()) < 0 or int(eid.max()) >= E):
        raise RuntimeError(f"prunepath.masked_gate_layout: expert ids outside [0, {E})")
    perm = torch.argsort(eid, stable=True).to(torch.int32)
    seg = torch.zeros(E + 1, dtype=torch.int32, device=eid.device)
    seg[1:] = torch.cumsum(torch.bincount(eid.long(), minlength=E), 0).to(torch.int32)
    return eid, perm, seg


def _mg_rows(t: torch.Tensor, last: int):
    return t.reshape(-1, last).contiguous()


def _mg_dtype(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return L.PP_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return L.PP_DTYPE_BF16
    raise RuntimeError(f"prunepath.masked_gate: activations must be float32 or bfloat16 (got {t.dtype})")


def masked_gate_fwd(inter: torch.Tensor, gates: torch.Tensor, eid: torch.Tensor, perm=None, seg=None) -> torch.Tensor:
    """inter [..., I] * gates[..., expert_ids] (MoELayer.forward's mask matmul and multiply,
    src/MoEBlock_origin.py:205-212), same dtype and shape as inter
    (``torch.ops.prunepath.masked_gate``; no autograd here: see ``masked_gate``)."""
    if perm is None or seg is None:
        perm = seg = torch.empty(0, dtype=torch.int32, device=eid.device)
    x = inter.contiguous()
    _mg_dtype(x)
    with torch.no_grad():
        return L.torch_ops().masked_gate(x, gates.float().contiguous(), eid, perm, seg)


def masked_gate_bwd(d_out: torch.Tensor, inter: torch.Tensor, gates: torch.Tensor, eid: torch.Tensor,
                    perm: torch.Tensor, seg: torch.Tensor, need_d_inter: bool = True):
    """(d_inter or None, d_gates fp32) of masked_gate_fwd (``torch.ops.prunepath.masked_gate_bwd``)."""
    x = inter.contiguous()
    _mg_dtype(x)
    d_inter, d_gates = L.torch_ops().masked_gate_bwd(d_out.to(x.dtype).contiguous(), x, gates.float().contiguous(),
                                                     eid, perm, seg, need_d_inter)
    return (d_inter if need_d_inter else None), d_gates


def _mg_setup_context(ctx, inputs, output):
    inter, gates, eid, perm, seg = inputs
    ctx.save_for_backward(inter, gates, eid, perm, seg)


def _mg_backward(ctx, d_out):
    inter, gates, eid, perm, seg = ctx.saved_tensors
    d_inter, d_gates = L.torch_ops().masked_gate_bwd(d_out.contiguous(), inter, gates, eid, perm, seg,
                                                     bool(ctx.needs_input_grad[0]))
    return (d_inter if ctx.needs_input_grad[0] else None), d_gates, None, None, None


_MG_AUTOGRAD = False


def _register_masked_gate_autograd() -> None:
    global _MG_AUTOGRAD
    if not _MG_AUTOGRAD:
        L.torch_ops()  # loads the extension (defines prunepath::masked_gate)
        torch.library.register_autograd("prunepath::masked_gate", _mg_backward, setup_context=_mg_setup_context)
        _MG_AUTOGRAD = True


def masked_gate(inter: torch.Tensor, gates: torch.Tensor, layout) -> torch.Tensor:
    """Differentiable masked gating: inter * (gates @ experts_masks) with the HIP forward
    and backward kernels (``torch.ops.prunepath.masked_gate``, autograd registered on the
    op); ``layout`` from masked_gate_layout. gates of any float dtype (computed in fp32)."""
    eid, perm, seg = layout
    _register_masked_gate_autograd()
    x = inter.contiguous()
    _mg_dtype(x)
    return L.torch_ops().masked_gate(x, gates.float().contiguous(), eid, perm, seg)
