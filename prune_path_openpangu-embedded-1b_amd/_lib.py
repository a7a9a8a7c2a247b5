"""Loader for libprunepath_moe.so, the C ABI declared in include/prunepath_moe.h.

There is no CPU fallback: if the library is missing or cannot be loaded, every
entry point raises. Build it with ``build()`` (hipcc, gfx950) before use.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libprunepath_moe.so")
# torch.library registration of the ops (csrc/torch_ops.cpp), linked against LIB_PATH
TORCH_LIB_PATH = os.path.join(_HERE, "libprunepath_torch.so")
CSRC = os.path.join(_HERE, "csrc")

PP_OK = 0
PP_DTYPE_F32 = 0
PP_DTYPE_BF16 = 1
PP_MAX_EXPERTS = 256

_lib = None

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_int64 = ctypes.c_int64
c_float = ctypes.c_float
c_size_t = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/prunepath_moe.h
SIGNATURES = {
    "pp_last_error": (ctypes.c_char_p, []),
    "pp_abi_version": (c_int, []),
    "pp_packed_expert_bytes": (c_size_t, [c_int, c_int, c_int]),
    "pp_pack_experts": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int,
                                c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "pp_packed_router_bytes": (c_size_t, [c_int, c_int]),
    "pp_pack_router": (c_int, [c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_void_p, c_void_p]),
    "pp_route": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_void_p, c_int, c_float, c_void_p,
                         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "pp_route_logits": (c_int, [c_void_p, c_int64, c_int, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p]),
    "pp_bucket_workspace_bytes": (c_size_t, [c_int64, c_int]),
    "pp_gemm_tile_m": (c_int, []),
    "pp_max_tiles": (c_int64, [c_int64, c_int, c_int]),
    "pp_bucket": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                          c_void_p, c_void_p, c_void_p, c_void_p]),
    "pp_decode_workspace_bytes": (c_size_t, [c_int, c_int]),
    "pp_decode_workspace_init": (c_int, [c_void_p, c_int, c_int, c_void_p]),
    "pp_decode_layout_tag": (ctypes.c_uint32, [c_int]),
    "pp_decode_state_check": (c_int, [c_void_p, c_int]),
    "pp_moe_decode": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p,
                              c_void_p, c_void_p, c_int, c_void_p]),
    "pp_moe_decode_noalloc": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_float,
                                      c_void_p, c_void_p, c_int, c_void_p]),
    "pp_decode_noalloc_reset": (c_int, [c_void_p, ctypes.c_uint32, c_void_p]),
    "pp_decode_batch_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "pp_moe_decode_batch": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_void_p, c_int, c_int, c_float,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "pp_prefill_workspace_bytes": (c_size_t, [c_int64, c_int, c_int, c_int]),
    "pp_moe_prefill": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_void_p, c_int, c_int, c_float,
                               c_void_p, c_void_p, c_void_p, c_void_p]),
    "pp_moe_prefill_routed": (c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_void_p, c_int, c_int, c_float,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "pp_expert_gateup": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_int64, c_void_p, c_void_p]),
    "pp_expert_down": (c_int, [c_void_p, c_int, c_int, c_void_p, c_int, c_void_p, c_void_p, c_int64,
                               c_void_p, c_void_p]),
    "pp_combine": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p]),
    "pp_masked_gate_fwd": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p,
                                   c_void_p]),
    "pp_masked_gate_bwd": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                   c_int, c_int, c_void_p, c_void_p, c_void_p]),
}


def build(jobs: int = 8) -> str:
    """Compile libprunepath_moe.so (hipcc, gfx950; cross-compiles without a GPU) and the
    torch.library extension libprunepath_torch.so (g++) with csrc/Makefile, recompiling
    what changed."""
    subprocess.run(["make", "-s", "-C", CSRC, f"-j{jobs}"], check=True)
    return LIB_PATH


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"prunepath: {LIB_PATH} is missing -- build it (make -C {CSRC}); there is no CPU fallback")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


_ops = None


def torch_ops():
    """``torch.ops.prunepath`` with the C++ extension loaded; raises if it has not been built."""
    global _ops
    if _ops is None:
        lib()  # the C ABI library first (the extension resolves it by soname)
        if not os.path.exists(TORCH_LIB_PATH):
            raise RuntimeError(f"prunepath: {TORCH_LIB_PATH} is missing -- build it (make -C {CSRC})")
        import torch
        torch.ops.load_library(TORCH_LIB_PATH)
        _ops = torch.ops.prunepath
    return _ops


def check(rc: int, what: str) -> None:
    if rc != PP_OK:
        msg = lib().pp_last_error().decode(errors="replace")
        raise RuntimeError(f"prunepath {what} failed (code {rc}): {msg}")
