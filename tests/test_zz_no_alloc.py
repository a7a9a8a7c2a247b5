"""GPU check of pp_moe_decode_noalloc (the allocation-free decode entry point) through
the C ABI: each call's output equals pp_moe_decode's on the same inputs within
rtol 2e-2 / atol 2e-3, and both equal the float64 sparse restatement on the selection
the workspace entry point reports (bit-exact against the oracle). Calls run back to back
on the shared scratch with shapes that change between calls -- larger first, then
smaller, then larger again -- which is what the fixed-stride scratch layout is for."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close, gi, make_module, oracle, sparse_expected, to_gpu

pytestmark = pytest.mark.gpu

# (H, E, G, tau, x dtype): the generic kernel with published logits, decode16 at the
# configured shape, the generic kernel with local logits, then decode16 again
SEQ = [(2048, 32, 64, 0.7, torch.float32),
       (1536, 16, 384, 0.7, torch.float32),
       (512, 8, 32, 0.9, torch.bfloat16),
       (1536, 16, 384, 0.95, torch.bfloat16),
       (4096, 16, 128, 0.7, torch.float32)]


def _noalloc(pkg, x, m, out):
    lib = pkg._lib.lib()
    xd = pkg._lib.PP_DTYPE_BF16 if x.dtype == torch.bfloat16 else pkg._lib.PP_DTYPE_F32
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.pp_moe_decode_noalloc(ctypes.c_void_p(x.data_ptr()), xd, m.hidden_size,
                                   ctypes.c_void_p(m.router_packed.data_ptr()), ctypes.c_void_p(0),
                                   m.num_experts, m.group_size, ctypes.c_float(m.tau),
                                   ctypes.c_void_p(m.packed_experts.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                   0, s)
    pkg._lib.check(rc, "pp_moe_decode_noalloc")


def test_noalloc_decode_matches_workspace_entry(pkg):
    mods = []
    for i, (H, E, G, tau, xdt) in enumerate(SEQ):
        w = gi.layer_weights(900 + i, H=H, I=E * G, E=E)
        mods.append((w, make_module(pkg, w, tau)))
    for rep in range(2):  # twice through the sequence: every shape follows a different one
        for i, (H, E, G, tau, xdt) in enumerate(SEQ):
            w, m = mods[i]
            x = gi.tokens(950 + 10 * rep + i, 1, H=H)
            xg = to_gpu(x, xdt)
            out_na = torch.full((1, H), float("nan"), dtype=torch.bfloat16, device="cuda:0")
            print(f"noalloc rep={rep} H={H} E={E} G={G} tau={tau} x={xdt}", flush=True)
            _noalloc(pkg, xg, m, out_na)
            out_ws = m(xg.view(1, 1, H)).view(1, H)
            st = pkg.ops.decode_state(m.decode_workspace, E)
            assert st["error"] == 0
            a = out_na.float().cpu().numpy()[0]
            b = out_ws.float().cpu().numpy()[0]
            assert np.isfinite(a).all()
            assert_close(a, b, what=f"noalloc vs workspace entry H={H} E={E}")
            sel = oracle.select(st["logits"].numpy()[None], tau)
            np.testing.assert_array_equal(st["sel_ids"].numpy(), sel.ranked[0, :sel.count[0]])
            exp = sparse_expected(xg.float().cpu().numpy(), w, sel.gates)[0]
            assert_close(a, exp, what=f"noalloc vs fp64 sparse H={H} E={E}")


def test_noalloc_rejects_sizes_beyond_the_scratch(pkg):
    lib = pkg._lib.lib()
    z = ctypes.c_void_p(0)
    rc = lib.pp_moe_decode_noalloc(z, 0, 8192, z, z, 16, 384, ctypes.c_float(0.7), z, z, 0, z)
    assert rc != 0
    rc = lib.pp_moe_decode_noalloc(ctypes.c_void_p(16), 0, 1536, ctypes.c_void_p(16), z, 300, 384,
                                   ctypes.c_float(0.7), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, z)
    assert rc != 0 and b"300" in lib.pp_last_error()
