"""GPU parity of the whole layer across the supported shape range.

Every kernel variant the library dispatches by shape gets at least one case, each
checked against the float64 sparse restatement on the same bf16 operands (rtol 2e-2 /
atol 2e-3) with the selection bit-exact against the oracle on the kernel's own logits:

* decode: decode16_kernel (E = 16, H % 512 == 0, G <= 512; CPL 1, 3 and 8, G = 512 at
  its limit), decode2p_kernel (any other shape with E * G <= 8192 and G <= 512: local
  and published logits, E from 8 to 256, the workgroup selection's rank merge over one
  to four 64-key runs, with and without a padded last run) and decode_kernel (the rest:
  G > 512 or E * G > 8192; local and published logits, eight waves for H <= 2560 and
  four above);
* prefill routing: route16_few_kernel (E = 16, N <= 64, H % 512 == 0, H <= 2048),
  route16_kernel (other E = 16 cases), and for E != 16 route_logits_kernel (the LDS-staged
  logits pass, one to three 16-expert tiles per workgroup) with the selection from its
  logits: route_kernel for E <= 64, route_select_wg_kernel above;
* prefill GEMMs: gemm_s_kernel (N <= 64, G % 64 == 0, H >= 384), gemm_v3_kernel
  (G % 64 == 0 otherwise); at G % 64 != 0 the dense form (dense_gemm_kernel, gate/up and
  down), the same implementation behind the torch op and the C ABI (same bits);
* the limits: H = 128 and 4096, E = 1 and 256, G = 32 and 8192, tau above 1 (every
  expert selected) and 0 (rank 0 only), bf16 and fp32 x; a router bias (log Zipf) on
  every router variant;
* for N > 1 the prefill pipeline is called explicitly, and where the one-launch batch
  kernel supports the shape (E = 16, H % 512 == 0, G <= 512, N <= 64) the module's output
  (that kernel) is checked too.
"""
import numpy as np
import pytest
import torch

from helpers import abi_prefill as _abi_prefill, assert_close, gi, make_module, oracle, sparse_expected, to_gpu

pytestmark = pytest.mark.gpu

# (H, E, G, N, tau, x dtype, router bias)
CASES = [
    (128, 16, 32, 3, 0.7, torch.float32, False),       # smallest H; G % 64 == 32 GEMMs; route16_few
    (640, 16, 64, 1, 0.7, torch.float32, False),       # E = 16 but H % 512 != 0: decode2p (local logits)
    (640, 16, 64, 70, 0.7, torch.float32, True),       # route16 with H % 512 != 0 and a bias; gemm_v3 at N = 70
    (4096, 16, 128, 1, 0.7, torch.float32, False),     # decode16 at CPL = 8 (two passes of output rows per workgroup)
    (512, 16, 512, 1, 0.9, torch.bfloat16, False),     # decode16 at CPL = 1 and its G limit (512)
    (2048, 16, 1024, 1, 0.7, torch.float32, True),     # E = 16 with G > 512: decode_kernel (local logits)
    (4096, 16, 128, 40, 0.5, torch.bfloat16, False),   # H > 2048: route16 at N <= 64; short tiles
    (2048, 16, 64, 64, 0.95, torch.float32, True),     # route16_few at CPL = 4 with a bias; short tiles at N = 64
    (1024, 8, 96, 33, 0.9, torch.float32, False),      # route_kernel (E = 8); dense form / gateup/down kernels (G = 96)
    (512, 96, 32, 20, 0.7, torch.bfloat16, True),      # E = 96: split logits (a partial second group) and the
                                                       # workgroup selection; dense form with bf16 x; bias
    (1024, 8, 96, 1, 0.9, torch.bfloat16, True),       # decode2p with local logits, E = 8, bf16 x, bias
    (512, 256, 32, 5, 0.7, torch.float32, False),      # E = 256
    (512, 256, 32, 1, 0.7, torch.float32, True),       # decode2p with E = 256 (published logits, E * G at 8192), bias
    (768, 4, 8192, 2, 1.05, torch.float32, False),     # G = 8192; tau > 1 selects every expert
    (768, 4, 8192, 1, 0.0, torch.float32, False),      # decode_kernel (G > 512), tau = 0: rank 0 only
    (1536, 1, 64, 17, 0.7, torch.float32, False),      # E = 1
    (1536, 16, 384, 129, 0.7, torch.bfloat16, False),  # bf16 x, ragged N past two 64-token blocks
    (1536, 16, 384, 1, 0.7, torch.bfloat16, False),    # decode16 at the configured shape, bf16 x
    (1536, 16, 384, 1, 0.95, torch.float32, True),     # decode16 with the config-3 router bias
    (4096, 192, 32, 1, 0.7, torch.float32, False),     # decode2p at CPL 8, three key runs
    (3072, 100, 32, 1, 0.7, torch.bfloat16, False),    # decode2p at CPL 6; two key runs, the last padded
    (1536, 200, 32, 1, 0.95, torch.float32, True),     # decode2p: four key runs, the last padded; bias
    (3072, 48, 256, 1, 0.7, torch.bfloat16, False),    # decode_kernel (E * G > 8192): published logits, four waves
    (1536, 200, 64, 1, 0.95, torch.float32, True),     # decode_kernel: eight waves, four key runs, the last padded; bias
    (2560, 8, 64, 1, 0.8, torch.float32, True),        # decode2p, E <= 16 with a router too large to read per
                                                       # workgroup: published logits, the wave selection
]


@pytest.mark.parametrize("H,E,G,N,tau,xdt,with_bias", CASES,
                         ids=[f"H{c[0]}-E{c[1]}-G{c[2]}-N{c[3]}-tau{c[4]}-{str(c[5])[6:]}{'-bias' if c[6] else ''}"
                              for c in CASES])
def test_layer_shape_vs_oracle(pkg, H, E, G, N, tau, xdt, with_bias):
    seed = H * 7 + E * 3 + G + N
    w = gi.layer_weights(seed, H=H, I=E * G, E=E)
    m = make_module(pkg, w, tau, bias=gi.zipf_bias(E) if with_bias else None)
    x = gi.tokens(seed + 1, N, H=H)
    xg = to_gpu(x, xdt)
    out = m(xg[None]).float().cpu().numpy()[0] if N == 1 else None
    if N == 1:
        st = pkg.ops.decode_state(m.decode_workspace, m.num_experts)
        logits = st["logits"].numpy()[None]
        sel = oracle.select(logits, tau)
        k = int(sel.count[0])
        assert st["error"] == 0 and st["k"] == k
        # selected experts in rank order (descending probability, ties by index)
        np.testing.assert_array_equal(st["sel_ids"].numpy(), sel.ranked[0][:k])
        np.testing.assert_array_equal(st["sel_gates"].numpy(), sel.gates[0][sel.ranked[0][:k]])
    else:
        res = pkg.ops.route(xg, m.router_packed, E, tau, bias=m.router_bias)
        logits = res["logits"].cpu().numpy()
        sel = oracle.select(logits, tau)
        np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
    xr = xg.float().cpu().numpy()
    expected = sparse_expected(xr, w, sel.gates)
    if N > 1:  # the prefill pipeline explicitly (the module takes the batch kernel where it can)
        pf = lambda: pkg.ops.moe_prefill(xg, m.router_packed, m.router_bias, E, G, tau,
                                         m.packed_experts).float().cpu().numpy()
        out = pf()
    assert_close(out, expected, what=f"layer H={H} E={E} G={G} N={N}")
    if N > 1:  # the C ABI: the same implementation as the torch op, and the routing it used
        y, lg, mk = _abi_prefill(pkg, m, xg, E, G, tau)
        np.testing.assert_array_equal(y.float().cpu().numpy(), out)
        np.testing.assert_array_equal(mk.cpu().numpy(), oracle.select(lg.cpu().numpy(), tau).mask)
        np.testing.assert_array_equal(lg.cpu().numpy(), logits)
    out2 = m(xg[None]).float().cpu().numpy()[0] if N == 1 else pf()
    np.testing.assert_array_equal(out2, out)  # prefill and decode are deterministic bit for bit
    if N > 1 and pkg.ops.decode_batch_supported(N, H, E, G):  # the one-launch batch kernel (module path)
        ob = m(xg[None]).float().cpu().numpy()[0]
        assert_close(ob, expected, what=f"batch kernel H={H} E={E} G={G} N={N}")
