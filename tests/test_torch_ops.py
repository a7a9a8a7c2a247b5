"""The torch.library surface (C++ extension libprunepath_torch.so, namespace prunepath).

CPU: every op is registered with its schema, the Meta (fake-tensor) implementations give
the output shapes and dtypes of the GPU ones (also under symbolic sizes), and CPU tensors
are refused with a clear error -- there is no host implementation.
GPU: torch.library.opcheck on each op (schema / mutation annotations, autograd
registration, fake-tensor agreement with the real kernels, tracing with dynamic shapes),
and each op's results equal the C ABI's through ctypes on the same inputs.
"""
import ctypes

import pytest
import torch

from conftest import import_pkg

OPS = ["route", "route_logits", "bucket", "pack_experts", "pack_router", "decode_workspace_init", "moe_decode",
       "moe_decode_into", "moe_decode_batch", "moe_decode_batch_into", "moe_prefill", "moe_prefill_into",
       "masked_gate", "masked_gate_bwd"]


@pytest.fixture(scope="module")
def P():
    return import_pkg()._lib.torch_ops()


def test_ops_registered(P):
    for name in OPS:
        op = getattr(P, name)
        assert op.default._schema.name == f"prunepath::{name}"
    # mutation annotations: the workspace (and out) of decode / the *_into ops
    assert "Tensor(a!) workspace" in str(P.moe_decode.default._schema)
    assert "Tensor(b!) out" in str(P.moe_prefill_into.default._schema)


def test_meta_shapes(P):
    m = torch.device("meta")
    N, H, E, G = 37, 256, 16, 64
    x = torch.empty(N, H, device=m)
    rp = torch.empty(16, H, device=m)
    logits, probs, gates, mask, count = P.route(x, rp, None, E, 0.7)
    assert logits.shape == (N, E) and mask.dtype == torch.uint8 and count.shape == (N,) and count.dtype == torch.int32
    off, tok, pg, tp, tiles, meta = P.bucket(mask, gates)
    lib = import_pkg()._lib.lib()
    assert off.shape == (E + 1,) and tok.shape == (N * E + 1,) and pg.dtype == torch.float32
    assert tiles.shape == (lib.pp_max_tiles(N, E, 128), 4) and meta.shape == (4,)
    wg = torch.empty(E * G, H, device=m)
    wd = torch.empty(H, E * G, device=m)
    packed = P.pack_experts(wg, wg, wd, E, G)
    assert packed.shape == (lib.pp_packed_expert_bytes(H, E, G) // 2,) and packed.dtype == torch.bfloat16
    assert P.pack_experts(wg.t(), wg.t(), wd.t(), E, G, None, "tau").shape == packed.shape
    assert P.pack_router(torch.empty(24, H, device=m)).shape == (32, H)
    assert P.pack_router(torch.empty(H, 24, device=m), "tau").shape == (32, H)
    ws = torch.empty(lib.pp_decode_workspace_bytes(H, E), dtype=torch.uint8, device=m)
    assert P.moe_decode(x[0], rp, None, E, G, 0.7, packed, ws).shape == (1, H)
    y = P.moe_prefill(x, rp, None, E, G, 0.7, packed)
    assert y.shape == (N, H) and y.dtype == torch.bfloat16
    bws = torch.empty(lib.pp_decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=m)
    yb = P.moe_decode_batch(x, rp, None, E, G, 0.7, packed, ws, bws)
    assert yb.shape == (N, H) and yb.dtype == torch.bfloat16
    inter = torch.empty(2, N, 1024, dtype=torch.bfloat16, device=m)
    gts = torch.empty(2, N, E, device=m)
    eid = torch.empty(1024, dtype=torch.int32, device=m)
    seg = torch.empty(E + 1, dtype=torch.int32, device=m)
    mg = P.masked_gate(inter, gts, eid, eid, seg)
    assert mg.shape == inter.shape and mg.dtype == torch.bfloat16
    di, dg = P.masked_gate_bwd(inter, inter, gts, eid, eid, seg, True)
    assert di.shape == inter.shape and dg.shape == gts.shape and dg.dtype == torch.float32
    di, _ = P.masked_gate_bwd(inter, inter, gts, eid, eid, seg, False)
    assert di.numel() == 0


def test_meta_symbolic_sizes(P):
    """The fake implementations trace with a symbolic token count (make_fx, symbolic mode)."""
    from torch.fx.experimental.proxy_tensor import make_fx

    def f(lg):
        probs, gates, mask, count = P.route_logits(lg, 0.5)
        return P.bucket(mask, gates, 0)

    gm = make_fx(f, tracing_mode="symbolic")(torch.empty(50, 16))
    shapes = {n.target.__name__ if hasattr(n.target, "__name__") else str(n.target): n.meta.get("val")
              for n in gm.graph.nodes if n.op == "call_function"}
    bk = [v for k, v in shapes.items() if "bucket" in k][0]
    tok = bk[1]
    n_sym, e_sym = str(bk[3].shape[0]), str(bk[3].shape[1])  # token_pairs [N, E]
    assert not isinstance(tok.shape[0], int)
    assert str(tok.shape[0]).replace(" ", "") in (f"{n_sym}*{e_sym}+1", f"{e_sym}*{n_sym}+1")


def test_cpu_tensors_refused(P):
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        P.route_logits(torch.zeros(3, 16), 0.7)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        P.moe_prefill(torch.zeros(3, 128), torch.zeros(16, 128), None, 16, 32, 0.7, torch.zeros(16))


# ----------------------------------------------------------------------------- GPU
def _inputs(N=40, H=512, E=16, G=64, seed=3):
    from helpers import gi, to_gpu
    w = gi.layer_weights(seed, H=H, I=E * G, E=E)
    x = to_gpu(gi.tokens(seed + 1, N, H=H))
    return w, x, to_gpu


@pytest.mark.gpu
def test_opcheck_all_ops(P):
    from torch.library import opcheck
    pkg = import_pkg()
    H, E, G = 512, 16, 64
    w, x, to_gpu = _inputs(H=H, E=E, G=G)
    wg, wu, wd, wr = (to_gpu(w[k]) for k in ("w_gate", "w_up", "w_down", "w_router"))
    perm = torch.randperm(E * G, device="cuda:0").to(torch.int32)
    rp = P.pack_router(wr)
    packed = P.pack_experts(wg, wu, wd, E, G, perm, "linear")
    logits, probs, gates, mask, count = P.route(x, rp, None, E, 0.7)
    ws = pkg.ops.decode_workspace(H, E, x.device)
    out1 = torch.empty(1, H, dtype=torch.bfloat16, device=x.device)
    wsp = torch.empty(pkg.ops.prefill_workspace_bytes(x.shape[0], H, E, G), dtype=torch.uint8, device=x.device)
    outp = torch.empty(x.shape[0], H, dtype=torch.bfloat16, device=x.device)
    bws = torch.empty(pkg.ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=x.device)
    outb = torch.empty(x.shape[0], H, dtype=torch.bfloat16, device=x.device)
    lgb = torch.empty(x.shape[0], E, dtype=torch.float32, device=x.device)
    mkb = torch.empty(x.shape[0], E, dtype=torch.uint8, device=x.device)
    cases = [
        (P.route, (x, rp, None, E, 0.7)),
        (P.route_logits, (logits, 0.7)),
        (P.bucket, (mask, gates, 0)),
        (P.pack_experts, (wg, wu, wd, E, G, perm, "linear")),
        (P.pack_router, (wr, "linear")),
        (P.decode_workspace_init, (ws, H, E)),
        (P.moe_decode, (x[0], rp, None, E, G, 0.7, packed, ws, 0)),
        (P.moe_decode_into, (x[0], rp, None, E, G, 0.7, packed, ws, out1, 0)),
        (P.moe_decode_batch, (x, rp, None, E, G, 0.7, packed, ws, bws, 0)),
        (P.moe_decode_batch_into, (x, rp, None, E, G, 0.7, packed, ws, bws, outb, lgb, mkb, 0)),
        (P.moe_prefill, (x, rp, None, E, G, 0.7, packed)),
        (P.moe_prefill_into, (x, rp, None, E, G, 0.7, packed, wsp, outp)),
    ]
    # the masked training gating (autograd registered on masked_gate from ops.py)
    I = 1024
    lay = pkg.ops.masked_gate_layout(torch.randperm(I, device=x.device) % E, E)
    pkg.ops._register_masked_gate_autograd()
    inter = torch.randn(x.shape[0], I, device=x.device, requires_grad=True)
    gts = torch.rand(x.shape[0], E, device=x.device, requires_grad=True)
    cases += [(P.masked_gate, (inter, gts, *lay)),
              (P.masked_gate, (inter.detach().bfloat16(), gts.detach(), *lay)),
              (P.masked_gate_bwd, (inter.detach(), inter.detach(), gts.detach(), *lay, True))]
    for op, args in cases:
        print(f"opcheck {op}", flush=True)
        opcheck(op, args)


@pytest.mark.gpu
def test_ops_equal_the_c_abi(P):
    """The op results are the C ABI's results on the same inputs (selection and bucket
    layout bit-exact, prefill output bit-exact: it is deterministic)."""
    pkg = import_pkg()
    lib = pkg._lib.lib()
    H, E, G, N = 512, 16, 64, 40
    w, x, to_gpu = _inputs(N=N, H=H, E=E, G=G, seed=11)
    rp = P.pack_router(to_gpu(w["w_router"]))
    packed = P.pack_experts(to_gpu(w["w_gate"]), to_gpu(w["w_up"]), to_gpu(w["w_down"]), E, G, None, "linear")
    logits, probs, gates, mask, count = P.route(x, rp, None, E, 0.7)
    vp = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g2, m2 = torch.empty_like(gates), torch.empty_like(mask)
    c2, l2, p2 = torch.empty_like(count), torch.empty_like(logits), torch.empty_like(probs)
    pkg._lib.check(lib.pp_route(vp(x), 0, N, H, vp(rp), vp(None), E, ctypes.c_float(0.7), vp(l2), vp(p2), vp(g2),
                                vp(m2), vp(c2), s), "route")
    for a, b in ((logits, l2), (probs, p2), (gates, g2), (mask, m2), (count, c2)):
        assert torch.equal(a, b)
    y = P.moe_prefill(x, rp, None, E, G, 0.7, packed)
    ws = torch.empty(pkg.ops.prefill_workspace_bytes(N, H, E, G), dtype=torch.uint8, device=x.device)
    y2 = torch.empty_like(y)
    pkg._lib.check(lib.pp_moe_prefill(vp(x), 0, N, H, vp(rp), vp(None), E, G, ctypes.c_float(0.7), vp(packed),
                                      vp(y2), vp(ws), s), "moe_prefill")
    assert torch.equal(y, y2)
    torch.cuda.synchronize()
