"""GPU check of pp_moe_decode_noalloc (the allocation-free decode entry point) through
the C ABI: each call's output equals pp_moe_decode's on the same inputs within
rtol 2e-2 / atol 2e-3, and both equal the float64 sparse restatement on the selection
the workspace entry point reports (bit-exact against the oracle). Calls run back to back
on the shared scratch with shapes -- and kernels -- that change from call to call,
larger and smaller in turn: the scratch keeps one layout for every shape (accumulator
stride 4096), which only decode_kernel uses, so the sequence runs all three kernels.
Then the scratch's error state: a reset that plants error bit 1 makes the next calls
write NaN, a plain reset reports the bit and restores the outputs, and a reset asked for
while the stream is capturing is refused; calls captured in a graph replay to the eager
result."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close, gi, make_module, oracle, sparse_expected, to_gpu

pytestmark = pytest.mark.gpu

# (H, E, G, tau, x dtype) and the kernel pp_moe_decode's dispatch gives each shape:
# decode16_kernel for E == 16, H % 512 == 0, G <= 512; decode2p_kernel for other
# shapes with E*G <= 8192 and G <= 512; decode_kernel for the rest. Logits are computed
# by every workgroup ("local") for E <= 16 and 16*H <= 32768, else published by E router
# workgroups.
SEQ = [(2048, 32, 64, 0.7, torch.float32),     # decode2p_kernel, published logits
       (1536, 16, 384, 0.7, torch.float32),    # decode16_kernel
       (2048, 16, 1024, 0.7, torch.bfloat16),  # decode_kernel, local logits (G > 512)
       (512, 8, 32, 0.9, torch.bfloat16),      # decode2p_kernel, local logits
       (3072, 48, 256, 0.7, torch.float32),    # decode_kernel, published logits (E*G > 8192)
       (1536, 16, 384, 0.95, torch.bfloat16),  # decode16_kernel
       (4096, 16, 128, 0.7, torch.float32)]    # decode16_kernel at the largest H

_mods = {}


def _module(pkg, i):
    if i not in _mods:
        H, E, G, tau, _ = SEQ[i]
        w = gi.layer_weights(900 + i, H=H, I=E * G, E=E)
        _mods[i] = (w, make_module(pkg, w, tau))
    return _mods[i]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _noalloc(pkg, x, m, out):
    lib = pkg._lib.lib()
    xd = pkg._lib.PP_DTYPE_BF16 if x.dtype == torch.bfloat16 else pkg._lib.PP_DTYPE_F32
    rc = lib.pp_moe_decode_noalloc(ctypes.c_void_p(x.data_ptr()), xd, m.hidden_size,
                                   ctypes.c_void_p(m.router_packed.data_ptr()), ctypes.c_void_p(0),
                                   m.num_experts, m.group_size, ctypes.c_float(m.tau),
                                   ctypes.c_void_p(m.packed_experts.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                   0, _stream())
    pkg._lib.check(rc, "pp_moe_decode_noalloc")


def _reset(pkg, error_in=0):
    """pp_decode_noalloc_reset on the current stream; returns the error bits it cleared."""
    lib = pkg._lib.lib()
    err = ctypes.c_uint32(0xdeadbeef)
    pkg._lib.check(lib.pp_decode_noalloc_reset(ctypes.byref(err), error_in, _stream()), "pp_decode_noalloc_reset")
    return err.value


def _nan_out(H):
    return torch.full((1, H), float("nan"), dtype=torch.bfloat16, device="cuda:0")


def test_noalloc_decode_matches_workspace_entry(pkg):
    for rep in range(2):  # twice through the sequence: every shape follows a different one
        for i, (H, E, G, tau, xdt) in enumerate(SEQ):
            w, m = _module(pkg, i)
            x = gi.tokens(950 + 10 * rep + i, 1, H=H)
            xg = to_gpu(x, xdt)
            out_na = _nan_out(H)
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


def test_noalloc_reset_restores_outputs_after_a_sticky_error(pkg):
    """Error bit 1 (a timed-out wait) is sticky: every later call writes NaN. It is planted
    from the host through the reset's error_in; the plain reset then reports it and the
    outputs are finite again, equal to the workspace entry point's. Shapes: the E = 16
    kernel and decode_kernel (each reads the sticky bit its own way)."""
    _reset(pkg)  # a known state, whatever ran before in this process
    for i in (1, 4):
        H, E, G, tau, xdt = SEQ[i]
        w, m = _module(pkg, i)
        xg = to_gpu(gi.tokens(970 + i, 1, H=H), xdt)
        print(f"noalloc reset H={H} E={E} G={G}", flush=True)
        assert _reset(pkg, error_in=1) == 0
        for _ in range(2):  # sticky: not only the first call after the error
            out = torch.zeros((1, H), dtype=torch.bfloat16, device="cuda:0")
            _noalloc(pkg, xg, m, out)
            assert torch.isnan(out.float()).all(), f"H={H} E={E}: outputs not NaN under the sticky error bit"
        assert _reset(pkg) & 1 == 1
        out = _nan_out(H)
        _noalloc(pkg, xg, m, out)
        ref = m(xg.view(1, 1, H)).view(1, H)
        a = out.float().cpu().numpy()[0]
        assert np.isfinite(a).all()
        assert_close(a, ref.float().cpu().numpy()[0], what=f"after reset H={H} E={E}")
        assert _reset(pkg) == 0  # the call after the reset raised nothing


def test_noalloc_in_a_graph_and_reset_refused_while_capturing(pkg):
    """After an eager call has initialised the scratch, a captured pp_moe_decode_noalloc
    replays to the eager output (four replays, eager work and synchronisation between
    them); pp_decode_noalloc_reset while the stream is capturing is refused with
    PP_ERR_INVALID and launches nothing into the graph."""
    lib = pkg._lib.lib()
    H, E, G, tau, xdt = SEQ[1]
    w, m = _module(pkg, 1)
    xg = to_gpu(gi.tokens(990, 1, H=H), xdt)
    eager = _nan_out(H)
    _noalloc(pkg, xg, m, eager)
    torch.cuda.synchronize()
    out = _nan_out(H)
    g = torch.cuda.CUDAGraph()
    rc_reset = None
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    print("noalloc graph capture", flush=True)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            err = ctypes.c_uint32(0)
            rc_reset = lib.pp_decode_noalloc_reset(ctypes.byref(err), 0, _stream())
            _noalloc(pkg, xg, m, out)
    assert rc_reset == 1 and "capturing" in lib.pp_last_error().decode()
    torch.cuda.synchronize()
    for r in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        other = _nan_out(H)
        _noalloc(pkg, xg, m, other)  # an eager call between replays
        torch.cuda.synchronize()
        assert torch.equal(other, eager)
    assert _reset(pkg) == 0


def test_noalloc_rejects_sizes_beyond_the_scratch(pkg):
    lib = pkg._lib.lib()
    z = ctypes.c_void_p(0)
    rc = lib.pp_moe_decode_noalloc(z, 0, 8192, z, z, 16, 384, ctypes.c_float(0.7), z, z, 0, z)
    assert rc != 0
    rc = lib.pp_moe_decode_noalloc(ctypes.c_void_p(16), 0, 1536, ctypes.c_void_p(16), z, 300, 384,
                                   ctypes.c_float(0.7), ctypes.c_void_p(16), ctypes.c_void_p(16), 0, z)
    assert rc != 0 and b"300" in lib.pp_last_error()
