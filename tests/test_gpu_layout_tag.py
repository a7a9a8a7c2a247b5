"""GPU check of the decode workspace's layout tag: a workspace initialised for another
hidden size (so tagged with another layout) is refused by every decode kernel -- NaN
outputs, error bit 8, and not one byte of the workspace written besides the error word
-- and the same workspace initialised for the call's H then gives the module's output.
Every buffer is sized for the larger of the two layouts, so even a kernel that skipped
the check would stay inside it."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import gi, make_module, to_gpu

pytestmark = pytest.mark.gpu

# (H, E, G, H of the foreign tag, N tokens): the kernel pp_moe_decode's dispatch gives
# the shape, or the batch kernel for N > 1
CASES = [(1536, 16, 384, 2048, 1),   # decode16_kernel
         (512, 192, 32, 1024, 1),    # decode2p_kernel (published logits)
         (2048, 16, 1024, 1536, 1),  # decode_kernel (local logits)
         (1024, 48, 256, 2048, 1),   # decode_kernel (published logits)
         (1536, 16, 384, 1024, 8)]   # decodeb_kernel


def _init(pkg, ws, H, E):
    lib = pkg._lib.lib()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    pkg._lib.check(lib.pp_decode_workspace_init(ctypes.c_void_p(ws.data_ptr()), H, E, s), "pp_decode_workspace_init")


def _call(pkg, m, xg, ws):
    N, H = xg.shape
    E, G = m.num_experts, m.group_size
    if N == 1:
        return pkg.ops.moe_decode(xg, m.router_packed, m.router_bias, E, G, m.tau, m.packed_experts, ws)
    bws = torch.zeros(pkg.ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=xg.device)
    return pkg.ops.moe_decode_batch(xg, m.router_packed, m.router_bias, E, G, m.tau, m.packed_experts, ws, bws)


@pytest.mark.parametrize("H,E,G,H_other,N", CASES, ids=[f"H{c[0]}-E{c[1]}-G{c[2]}-N{c[4]}" for c in CASES])
def test_workspace_of_another_layout_is_refused(pkg, H, E, G, H_other, N):
    lib = pkg._lib.lib()
    w = gi.layer_weights(31 * H + E, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.7)
    xg = to_gpu(gi.tokens(7 * H + N, N, H=H))
    nbytes = max(lib.pp_decode_workspace_bytes(H, E), lib.pp_decode_workspace_bytes(H_other, E))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda:0")
    _init(pkg, ws, H_other, E)
    before = ws.clone()
    st0 = pkg.ops.decode_state(ws, E)
    assert st0["layout"] == lib.pp_decode_layout_tag(H_other) != lib.pp_decode_layout_tag(H)
    print(f"layout tag H={H} E={E} G={G} N={N} workspace of H={H_other}", flush=True)
    out = _call(pkg, m, xg, ws)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    st = pkg.ops.decode_state(ws, E)
    assert st["error"] == 8
    changed = torch.nonzero(ws != before).flatten().cpu().numpy()
    assert set(changed.tolist()) <= {12, 13, 14, 15}, f"bytes written: {changed[:16]}"
    # the same buffer initialised for this H: the module's own output
    _init(pkg, ws, H, E)
    out = _call(pkg, m, xg, ws)
    ref = m(xg.view(1, N, H)).view(N, H)
    assert pkg.ops.decode_state(ws, E)["error"] == 0
    np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy(), ref.view(torch.int16).cpu().numpy())
