"""PrunePath sparse-MoE MLP path for MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (include/prunepath_moe.h,
libprunepath_moe.so), torch-level wrappers in ``ops`` and the drop-in
``TauSparseMoE`` module mirroring src/tl_kernel_optimized_Ultimate_PanGU.py:468-615;
``model`` holds the eval-mode MLP wrapper and the one-time reorder of the openPangu
model code (src/openpangu_moe.py:43-130, 212-256).
"""
from . import _lib
from ._lib import build
from . import ops
from .tau_sparse_moe import TauSparseMoE
from .model import (IntegratedOpenPanguMoEMLP, MoELayer, experts_masks_from_ids, load_cluster_ids,
                    penalty_losses, physical_reorder_for_inference)
from . import decoder_stack

__all__ = ["TauSparseMoE", "IntegratedOpenPanguMoEMLP", "MoELayer", "experts_masks_from_ids", "load_cluster_ids",
           "penalty_losses", "physical_reorder_for_inference", "decoder_stack", "ops", "build", "_lib"]
