"""GPU parity of the one-launch small-batch decode (pp_moe_decode_batch, decodeb_kernel).

Each case routes N tokens through the kernel and checks, against the CPU oracle:
* the selection bit-exact (mask_out against oracle.select on the kernel's own logits,
  which are checked against the oracle's fp64 router within fp32 rounding);
* every output row against the float64 sparse restatement on the same bf16 operands
  with the acts rounded to bf16 before the down projection -- the rounding point of the
  reference's fused expert kernel (src/tl_kernel_optimized_Ultimate_PanGU.py:318) and of
  both of this library's paths (rtol 2e-2 / atol 2e-3, the north-star tolerance; with
  unrounded acts, ~1000 acts per output at H = 4096 leave a 1e-3 spread that prefill
  shows alike);
* the output against pp_moe_prefill on the same tokens (same tolerance; both compute the
  same layer with bf16 acts and fp32 sums, in different orders);
* determinism: a second call gives the same bits, and the call epoch advances by one.
Shapes cover both token-block widths (N <= 32 and N > 32), CPL 1 / 3 / 8, G = 32 and
512, fp32 and bf16 x, a router bias, and grids small enough that a row group spans
several LDS passes of down rows.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, gi, make_module, oracle, sparse_expected, to_gpu

pytestmark = pytest.mark.gpu


def _run(pkg, m, xg, grid=0):
    N, H = xg.shape
    E, G = m.num_experts, m.group_size
    bws = torch.empty(pkg.ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=xg.device)
    logits = torch.empty(N, E, dtype=torch.float32, device=xg.device)
    mask = torch.empty(N, E, dtype=torch.uint8, device=xg.device)
    out = pkg.ops.moe_decode_batch(xg, m.router_packed, m.router_bias, E, G, m.tau, m.packed_experts,
                                   m.decode_workspace, bws, grid=grid, logits_out=logits, mask_out=mask)
    return out, logits, mask, bws


# (H, E, G, N, tau, x dtype, router bias, grid)
CASES = [
    (1536, 16, 384, 16, 0.95, torch.float32, True, 0),     # config 3, bs 16
    (1536, 16, 384, 64, 0.95, torch.float32, True, 0),     # config 3, bs 64 (two token blocks)
    (1536, 16, 384, 2, 0.70, torch.bfloat16, False, 0),    # two tokens, bf16 x
    (1536, 16, 384, 33, 0.70, torch.float32, False, 0),    # ragged second token block
    (512, 16, 32, 1, 0.70, torch.float32, False, 0),       # CPL 1, G = 32, one token
    (512, 16, 512, 20, 0.90, torch.bfloat16, True, 0),     # G = 512 (the kernel's limit)
    (4096, 16, 128, 64, 0.70, torch.float32, False, 0),    # CPL 8, two token blocks
    (4096, 16, 128, 17, 0.70, torch.float32, False, 32),   # 32 workgroups: rows in several LDS passes
    (2048, 16, 256, 16, 0.50, torch.bfloat16, False, 16),  # one row group (16 workgroups)
]


@pytest.mark.parametrize("H,E,G,N,tau,xdt,with_bias,grid", CASES,
                         ids=[f"H{c[0]}-G{c[2]}-N{c[3]}-tau{c[4]}-{str(c[5])[6:]}{'-bias' if c[6] else ''}"
                              f"{'-grid' + str(c[7]) if c[7] else ''}" for c in CASES])
def test_decode_batch_vs_oracle(pkg, H, E, G, N, tau, xdt, with_bias, grid):
    seed = 11 * H + 5 * G + N
    w = gi.layer_weights(seed, H=H, I=E * G, E=E)
    m = make_module(pkg, w, tau, bias=gi.zipf_bias(E) if with_bias else None)
    x = gi.tokens(seed + 1, N, H=H)
    xg = to_gpu(x, xdt)
    e0 = pkg.ops.decode_state(m.decode_workspace, E)["epochb"]
    out, logits, mask, _ = _run(pkg, m, xg, grid)
    torch.cuda.synchronize()
    st = pkg.ops.decode_state(m.decode_workspace, E)
    assert st["error"] == 0 and st["epochb"] == e0 + 1
    lg = logits.cpu().numpy()
    xr = xg.float().cpu().numpy()
    # the kernel's logits: the router in fp32 (fixed order) -- close to the fp64 product
    ref_logits = xr.astype(np.float64) @ w["w_router"].astype(np.float64).T
    if with_bias:
        ref_logits = ref_logits + gi.zipf_bias(E)
    np.testing.assert_allclose(lg, ref_logits, rtol=1e-4, atol=1e-4)
    sel = oracle.select(lg, tau)
    np.testing.assert_array_equal(mask.cpu().numpy(), sel.mask)
    o = out.float().cpu().numpy()
    assert_close(o, sparse_expected(xr, w, sel.gates, act_bf16=True), what=f"decode batch H={H} G={G} N={N}")
    # the prefill path on the same tokens (the same roundings: equal within a few bf16 ulps)
    pf = pkg.ops.moe_prefill(xg, m.router_packed, m.router_bias, E, G, tau, m.packed_experts).float().cpu().numpy()
    assert_close(o, pf, rtol=1e-2, atol=1e-3, what="decode batch vs prefill")
    # bitwise reproducible, call after call; the epoch advances once per call
    for rep in range(5):
        out2, _, mask2, _ = _run(pkg, m, xg, grid)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out2.float().cpu().numpy(), o, err_msg=f"repeat {rep}")
        np.testing.assert_array_equal(mask2.cpu().numpy(), sel.mask)
    assert pkg.ops.decode_state(m.decode_workspace, E)["epochb"] == e0 + 6


def test_decode_batch_interleaved_with_decode(pkg):
    """Batch calls and single-token decode calls alternate on one decode workspace (each
    kernel family keeps its own epoch); every result matches its stand-alone value."""
    H, E, G = 1536, 16, 384
    w = gi.layer_weights(77, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.8)
    xb = to_gpu(gi.tokens(78, 24, H=H), torch.float32)
    x1 = to_gpu(gi.tokens(79, 1, H=H), torch.float32)
    ref_b, _, _, bws = _run(pkg, m, xb)
    ref_1 = pkg.ops.moe_decode(x1, m.router_packed, m.router_bias, E, G, 0.8, m.packed_experts, m.decode_workspace)
    torch.cuda.synchronize()
    for i in range(6):
        ob = pkg.ops.moe_decode_batch(xb, m.router_packed, m.router_bias, E, G, 0.8, m.packed_experts,
                                      m.decode_workspace, bws)
        o1 = pkg.ops.moe_decode(x1, m.router_packed, m.router_bias, E, G, 0.8, m.packed_experts, m.decode_workspace)
        torch.cuda.synchronize()
        assert torch.equal(ob, ref_b), f"batch call {i}"
        assert torch.equal(o1, ref_1), f"decode call {i}"
    assert pkg.ops.decode_state(m.decode_workspace, E)["error"] == 0


@pytest.mark.parametrize("xdt,with_bias", [(torch.float32, False), (torch.bfloat16, True)])
def test_decode_batch_routing_equals_decode_kernel(pkg, xdt, with_bias):
    """The batch kernel's logits and selection of each token are the single-token decode
    kernel's bits (both run dec16_logits and sel16_wave): the bench takes each timed
    decode step's k from one untimed batch call. 40 tokens at tau 0.7, one decode call
    per token."""
    H, E, G = 1536, 16, 384
    w = gi.layer_weights(81, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.7, bias=gi.zipf_bias(E) if with_bias else None)
    xb = to_gpu(gi.tokens(82, 40, H=H), xdt)
    _, logits, mask, _ = _run(pkg, m, xb)
    lg = logits.cpu().numpy()
    mk = mask.cpu().numpy()
    for t in range(xb.shape[0]):
        pkg.ops.moe_decode(xb[t], m.router_packed, m.router_bias, E, G, 0.7, m.packed_experts, m.decode_workspace)
        st = pkg.ops.decode_state(m.decode_workspace, E)
        np.testing.assert_array_equal(st["logits"].numpy().view(np.uint32), lg[t].view(np.uint32), err_msg=f"token {t}")
        sel = np.zeros(E, np.uint8)
        sel[st["sel_ids"].numpy()] = 1
        np.testing.assert_array_equal(sel, mk[t], err_msg=f"token {t}")
        assert st["k"] == int(mk[t].sum())


def test_decode_batch_graph_replays(pkg):
    """A call captured in a hipGraph (as the bench runs it): every replay, with eager calls on
    the same workspaces and host synchronisations between replays, gives the eager result
    bit for bit; the epoch and the tags advance per call whichever way the call is launched."""
    H, E, G, N = 1536, 16, 384, 16
    w = gi.layer_weights(61, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.95, bias=gi.zipf_bias(E))
    dev = torch.device("cuda:0")
    xs = [to_gpu(gi.tokens(62 + i, N, H=H), torch.float32) for i in range(3)]
    bws = torch.empty(pkg.ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=dev)

    def call(x, out=None):
        return pkg.ops.moe_decode_batch(x, m.router_packed, m.router_bias, E, G, 0.95, m.packed_experts,
                                        m.decode_workspace, bws, out=out)

    refs = [call(x) for x in xs]
    torch.cuda.synchronize()
    xin = xs[0].clone()
    out = torch.empty(N, H, dtype=torch.bfloat16, device=dev)
    call(xin, out)  # warm-up on the capture buffers
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            call(xin, out)
    torch.cuda.current_stream().wait_stream(s)
    e0 = pkg.ops.decode_state(m.decode_workspace, E)["epochb"]
    for rep in range(6):
        i = rep % 3
        xin.copy_(xs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, refs[i]), f"replay {rep}"
        o = call(xs[(i + 1) % 3])  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.equal(o, refs[(i + 1) % 3]), f"eager call after replay {rep}"
    st = pkg.ops.decode_state(m.decode_workspace, E)
    assert st["error"] == 0 and st["epochb"] == e0 + 12


def test_decode_batch_module_dispatch(pkg):
    """TauSparseMoE.forward takes the batch kernel for 2 <= N <= batch_max at the
    supported shapes and prefill beyond; both agree with the float64 restatement."""
    H, E, G = 1536, 16, 384
    w = gi.layer_weights(91, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.95, bias=gi.zipf_bias(E))
    for N, bmax in ((8, 32), (64, 32), (64, 64), (65, 64)):
        m.batch_max = bmax
        x = gi.tokens(92 + N, N, H=H)
        xg = to_gpu(x, torch.float32)
        o = m(xg[None]).float().cpu().numpy()[0]
        res = pkg.ops.route(xg, m.router_packed, E, 0.95, bias=m.router_bias)
        sel = oracle.select(res["logits"].cpu().numpy(), 0.95)
        assert_close(o, sparse_expected(x, w, sel.gates), what=f"module N={N}")
    assert m.decode_error() == 0


def test_decode_batch_unsupported_shapes(pkg):
    """Shapes outside the batch kernel's family are refused (the module falls back to
    prefill): E != 16, H % 512 != 0, G > 512, N > 64."""
    dev = torch.device("cuda:0")
    for (H, E, G, N) in ((1536, 8, 384, 4), (640, 16, 64, 4), (1536, 16, 1024, 4), (1536, 16, 384, 65)):
        assert not pkg.ops.decode_batch_supported(N, H, E, G)
        w = gi.layer_weights(5, H=H, I=E * G, E=E)
        m = make_module(pkg, w, 0.7)
        xg = to_gpu(gi.tokens(6, N, H=H), torch.float32)
        bws = torch.empty(pkg.ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=dev)
        with pytest.raises(RuntimeError, match="unsupported"):
            pkg.ops.moe_decode_batch(xg, m.router_packed, m.router_bias, E, G, 0.7, m.packed_experts,
                                     m.decode_workspace, bws)
