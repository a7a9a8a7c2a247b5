"""CPU checks of the C ABI: the library loads, exports exactly what
include/prunepath_moe.h declares, sizes are consistent, invalid arguments are
rejected before any launch, and the torch wrappers refuse CPU tensors (there is
no CPU fallback)."""
import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT, import_pkg

HEADER = os.path.join(ROOT, "include", "prunepath_moe.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(pp_[a-z_0-9]+)\s*\(", txt)))


def test_header_symbols_exported():
    pkg = import_pkg()
    lib = pkg._lib.lib()
    names = _declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    # every declared symbol has a ctypes signature in the loader
    assert sorted(pkg._lib.SIGNATURES) == names


def test_exported_symbols_match_header():
    pkg = import_pkg()
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", pkg._lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted({l.split()[-1] for l in out.splitlines() if re.search(r" T pp_", l)})
    assert exported == _declared()


def test_sizes():
    pkg = import_pkg()
    lib = pkg._lib.lib()
    H, E, G = 1536, 16, 384
    assert lib.pp_packed_expert_bytes(H, E, G) == E * G * H * 4 * 2
    assert lib.pp_packed_router_bytes(H, E) == 16 * H * 4
    assert lib.pp_packed_router_bytes(H, 17) == 32 * H * 4
    assert lib.pp_gemm_tile_m() == 128
    # tile bound: sum_e ceil(c_e/128) <= N*E/128 + E
    assert lib.pp_max_tiles(2048, 16, 128) == 2048 * 16 // 128 + 16
    assert lib.pp_decode_workspace_bytes(H, E) >= 32 + 3 * 4 * 256 + 8 * H * 4
    assert lib.pp_prefill_workspace_bytes(2048, H, E, G) > 2048 * 16 * (G + H) * 2
    assert lib.pp_abi_version() == 3


def _state(layout):
    """A host copy of a decode workspace's state header (pp_decode_state) with `layout`
    in its tag word (bytes 24..28)."""
    buf = (ctypes.c_uint8 * (32 + 3 * 4 * 256))()
    ctypes.c_uint32.from_buffer(buf, 24).value = layout
    return buf


def test_decode_workspace_of_another_layout_is_refused():
    """The decode workspace's layout tag: pp_decode_workspace_init writes
    pp_decode_layout_tag(H), and a header whose tag is another H's, another layout
    version's, or zero (never initialised) is refused with both tags named (the kernels
    compare the same word with the same tag before their first workspace write)."""
    pkg = import_pkg()
    lib = pkg._lib.lib()
    tags = {H: lib.pp_decode_layout_tag(H) for H in (128, 1536, 2048, 4096)}
    assert len(set(tags.values())) == 4 and all(t != 0 for t in tags.values())
    assert lib.pp_decode_layout_tag(100) == 0 and lib.pp_decode_layout_tag(8192) == 0
    for H, t in tags.items():
        assert lib.pp_decode_state_check(_state(t), H) == 0
        assert (t >> 13) & 0x7ff == 3  # the layout version this build writes
    t = tags[1536]
    for bad, what in [(tags[2048], "another H"), (t ^ (1 << 13), "another layout version"), (0, "never initialised")]:
        rc = lib.pp_decode_state_check(_state(bad), 1536)
        assert rc == 1, what
        msg = lib.pp_last_error().decode()
        assert f"0x{bad:08x}" in msg and f"0x{t:08x}" in msg, (what, msg)
    assert lib.pp_decode_state_check(None, 1536) == 1


def test_noalloc_reset_without_a_gpu_fails_cleanly():
    """pp_decode_noalloc_reset needs a current device: on a host without one it returns an
    error code, it does not crash."""
    pkg = import_pkg()
    lib = pkg._lib.lib()
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: tests/test_zz_no_alloc.py covers the reset")
    err = ctypes.c_uint32(77)
    assert lib.pp_decode_noalloc_reset(ctypes.byref(err), 0, None) != 0
    assert lib.pp_last_error().decode()


@pytest.mark.parametrize("H,E,G", [(100, 16, 384), (1536, 0, 384), (1536, 300, 32), (1536, 16, 40),
                                   (8192, 16, 384)])
def test_invalid_shapes_rejected(H, E, G):
    pkg = import_pkg()
    lib = pkg._lib.lib()
    p = ctypes.c_void_p(1)
    rc = lib.pp_moe_decode(p, 0, H, p, None, E, G, 0.7, p, p, p, 0, None)
    assert rc == 3
    assert lib.pp_last_error().decode()
    rc = lib.pp_moe_prefill(p, 0, 8, H, p, None, E, G, 0.7, p, p, p, None)
    assert rc == 3


def test_null_pointers_rejected():
    pkg = import_pkg()
    lib = pkg._lib.lib()
    rc = lib.pp_moe_decode(None, 0, 1536, None, None, 16, 384, 0.7, None, None, None, 0, None)
    assert rc == 1 and "null" in lib.pp_last_error().decode()
    rc = lib.pp_route_logits(None, 4, 16, 0.7, None, None, None, None, None)
    assert rc == 1
    rc = lib.pp_bucket(None, None, 4, 16, 128, None, None, None, None, None, None, None, None)
    assert rc == 1
    rc = lib.pp_moe_decode(ctypes.c_void_p(1), 7, 1536, ctypes.c_void_p(1), None, 16, 384, 0.7,
                           ctypes.c_void_p(1), ctypes.c_void_p(1), ctypes.c_void_p(1), 0, None)
    assert rc == 1 and "dtype" in lib.pp_last_error().decode()


def test_zero_tokens_is_a_no_op():
    pkg = import_pkg()
    lib = pkg._lib.lib()
    assert lib.pp_moe_prefill(None, 0, 0, 1536, None, None, 16, 384, 0.7, None, None, None, None) == 0
    assert lib.pp_route_logits(None, 0, 16, 0.7, None, None, None, None, None) == 0


def test_wrappers_refuse_cpu_tensors():
    pkg = import_pkg()
    x = torch.zeros(4, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        pkg.ops.route_logits(x, 0.7)
    m = pkg.TauSparseMoE(128, 512, 16, 32, 0.7)
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.zeros(1, 1, 128))


def test_module_buffers_match_reference_layout():
    pkg = import_pkg()
    m = pkg.TauSparseMoE(1536, 6144, 16, 384, 0.7)
    sd = m.state_dict()
    assert sorted(sd) == ["W_down", "W_gate", "W_up", "router"]
    assert sd["W_gate"].shape == (1536, 6144) and sd["W_gate"].dtype == torch.bfloat16
    assert sd["W_up"].shape == (1536, 6144)
    assert sd["W_down"].shape == (6144, 1536)
    assert sd["router"].shape == (1536, 16)
    assert m.EXPERTS_POWER2 == 16 and m.tau == 0.7
    with pytest.raises(ValueError):
        pkg.TauSparseMoE(1536, 6144, 16, 300, 0.7)
