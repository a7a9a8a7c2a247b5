"""PrunePath sparse-MoE MLP path for MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (include/prunepath_moe.h,
libprunepath_moe.so), torch-level wrappers in ``ops`` and the drop-in
``TauSparseMoE`` module mirroring src/tl_kernel_optimized_Ultimate_PanGU.py:468-615.
"""
from . import _lib
from ._lib import build
from . import ops
from .tau_sparse_moe import TauSparseMoE

__all__ = ["TauSparseMoE", "ops", "build", "_lib"]
