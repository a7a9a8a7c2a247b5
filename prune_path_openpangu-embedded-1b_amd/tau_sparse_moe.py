"""Drop-in replacement for the reference ``TauSparseMoE`` block
(src/tl_kernel_optimized_Ultimate_PanGU.py:468-615) on MI355X.

Same constructor ``TauSparseMoE(hidden_size, intermediate_size, num_experts,
group_size, tau)``, same persistent buffers and ``state_dict`` keys
(``W_gate`` [H,I], ``W_up`` [H,I], ``W_down`` [I,H] in bf16 -- the rearranged
layout written by ``physical_reorder_for_inference``, src/openpangu_moe.py:234-243 --
and ``router`` [H,E]), same mutable ``tau`` attribute and the same
``forward(x[B,L,H]) -> [B,L,H] bf16`` that takes the decode path for one token
and the prefill path otherwise (:606-615).

Differences by design (each a documented build choice, not an omission):
* ``router`` is kept in fp32 (the reference stores bf16, :486); loading a bf16
  state_dict converts on copy. Routing follows the masked reference
  ``softmax_thresholding`` (src/MoEBlock_origin.py:50-97) bit for bit given the
  fp32 logits.
* The kernels read packed copies of the buffers (``packed_experts``,
  ``router_packed``, non-persistent), rebuilt lazily whenever the reference
  buffers change (``load_state_dict``, ``.data =`` assignment, in-place edits
  through ``mark_weights_changed``). Once packed, ``W_gate``, ``W_up`` and ``W_down``
  are not kept: the packed records hold the same bf16 values, so a layer holds 75.5 MB
  at H=1536, I=6144 instead of 132 MB. Their objects stay registered (so ``.data =``
  mounting works) with no storage; reading one (``m.W_gate``) or ``state_dict()``
  rebuilds it from the packed records, bit for bit, and ``load_state_dict`` gives
  them storage again before copying.
* Outputs are fresh tensors (the reference decode output aliases a persistent
  buffer, :530) and no call synchronises with the host (the reference prefill
  calls ``total_tiles.item()``, :581).
* Every neuron of every selected expert is computed (the reference decode grid
  covers only 64 neurons per expert, :398-399, 515).
* Small batches (2 <= N <= ``batch_max`` tokens, 64 by default and at most 64, at E = 16
  with H % 512 == 0 and G <= 512) run the one-launch batch kernel (``ops.moe_decode_batch``) instead of the prefill pipeline the
  reference uses for every N > 1: same routing and output within the north-star
  tolerance, one kernel instead of five. Its batch workspace is allocated on first use.
* Decode failures are not silent (the reference has no failure reporting): a decode
  call whose selection is inconsistent or whose reduction leaves the fixed-point range
  writes NaN outputs, and one whose cross-workgroup wait times out writes NaN from then
  on; each sets a sticky error bit in the decode workspace.
  ``decode_error()`` reads the bits, ``check_decode()`` raises when one is set, and
  ``checked = True`` runs that check after every decode call (a host sync, so off by
  default; graph-captured serving loops check between replays instead);
  ``reset_decode_error()`` clears it.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _lib, ops


_DECODE_OP = None
# the reference-layout expert buffers, dropped once packed (rebuilt from the records on demand)
_EXPERT_BUFFERS = ("W_gate", "W_up", "W_down")


def _decode_op():
    """torch.ops.prunepath.moe_decode.default, resolved once."""
    global _DECODE_OP
    if _DECODE_OP is None:
        _DECODE_OP = _lib.torch_ops().moe_decode.default
    return _DECODE_OP


class TauSparseMoE(nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int, num_experts: int, group_size: int,
                 tau: float, router_bias: Optional[torch.Tensor] = None):
        super().__init__()
        if num_experts * group_size != intermediate_size:
            raise ValueError(f"num_experts*group_size ({num_experts}*{group_size}) != intermediate_size "
                             f"({intermediate_size})")
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.num_experts = num_experts
        self.group_size = group_size
        self.tau = tau
        self.EXPERTS_POWER2 = 1 << max(0, (num_experts - 1).bit_length())

        self.register_buffer("W_gate", torch.empty(hidden_size, intermediate_size, dtype=torch.bfloat16))
        self.register_buffer("W_up", torch.empty(hidden_size, intermediate_size, dtype=torch.bfloat16))
        self.register_buffer("W_down", torch.empty(intermediate_size, hidden_size, dtype=torch.bfloat16))
        self.register_buffer("router", torch.empty(hidden_size, num_experts, dtype=torch.float32))
        # optional router bias (not in the reference; used to skew expert load in benchmarks)
        self.register_buffer("router_bias", None if router_bias is None else router_bias.float().clone(),
                             persistent=False)
        # kernel-side copies
        self.register_buffer("packed_experts", None, persistent=False)
        self.register_buffer("router_packed", None, persistent=False)
        self.register_buffer("decode_workspace", None, persistent=False)
        self.register_buffer("batch_workspace", None, persistent=False)
        self._packed_key = None
        # expert buffers rebuilt from the packed records since the last packing:
        # name -> (data_ptr, version) when rebuilt (unchanged since means nothing to repack)
        self._rebuilt = {}
        self.checked = False
        # token counts up to which forward() takes the one-launch batch kernel
        self.batch_max = 64

    # ------------------------------------------------------------------ packing
    def _weights_key(self):
        # read from _buffers directly (nn.Module.__getattr__ costs ~1 us per lookup) and
        # with get_device() (an int, where .device builds an object): this runs per call
        b = self._buffers
        return tuple((t.data_ptr(), t._version, t.get_device(), t.dtype) for t in
                     (b["W_gate"], b["W_up"], b["W_down"], b["router"]))

    def mark_weights_changed(self) -> None:
        self._packed_key = None

    # ------------------------------------------------------------------ expert buffers
    def _ref_shape(self, name: str):
        H, I = self.hidden_size, self.intermediate_size
        return (I, H) if name == "W_down" else (H, I)

    def _released(self, name: str) -> bool:
        """The buffer has no storage: its values are those of the packed records."""
        return self._buffers[name].numel() == 0 and self._buffers.get("packed_experts") is not None

    def _from_records(self, name: str) -> torch.Tensor:
        """The reference-layout buffer rebuilt from the packed records (rows region
        [I][3][H]: gate row, up row, down column of each rearranged neuron; the same bf16
        values the buffer held): W_gate/W_up [H,I], W_down [I,H], new storage."""
        H, I = self.hidden_size, self.intermediate_size
        rec = self._buffers["packed_experts"][:3 * I * H].view(I, 3, H)
        if name == "W_down":
            return rec[:, 2, :].contiguous()
        return rec[:, 0 if name == "W_gate" else 1, :].t().contiguous()

    def _release(self) -> None:
        for name in _EXPERT_BUFFERS:
            t = self._buffers[name]
            t.data = torch.empty(0, dtype=torch.bfloat16, device=t.device)
        self._rebuilt.clear()

    def __getattr__(self, name: str):
        # buffers live in _buffers, so reads of them come here: a released expert buffer is
        # given storage again, rebuilt from the records, in the same tensor object
        if name in _EXPERT_BUFFERS:
            bufs = self.__dict__.get("_buffers")
            if bufs is not None and name in bufs and self._released(name):
                t = bufs[name]
                t.data = self._from_records(name)
                self._rebuilt[name] = (t.data_ptr(), t._version)
        return super().__getattr__(name)

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        for name in _EXPERT_BUFFERS:
            if self._released(name):
                destination[prefix + name] = self._from_records(name)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        for name in _EXPERT_BUFFERS:  # storage to copy into
            if prefix + name in state_dict and self._released(name):
                t = self._buffers[name]
                t.data = torch.empty(self._ref_shape(name), dtype=torch.bfloat16, device=t.device)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)

    def repack(self) -> None:
        """Build the kernel layouts from the reference-layout buffers, then drop the
        expert buffers' storage. A buffer without storage, or rebuilt from the records
        and not changed since, contributes the records' own values."""
        b = self._buffers
        dev = b["W_gate"].device
        if dev.type != "cuda":
            raise RuntimeError("TauSparseMoE: move the module to the GPU first; there is no CPU implementation")
        H, E, G = self.hidden_size, self.num_experts, self.group_size

        def changed(name):
            t = b[name]
            return not self._released(name) and self._rebuilt.get(name) != (t.data_ptr(), t._version)

        if b["packed_experts"] is None or b["packed_experts"].device != dev or \
                any(changed(n) for n in _EXPERT_BUFFERS):
            src = [b[n] if not self._released(n) else self._from_records(n) for n in _EXPERT_BUFFERS]
            self.packed_experts = ops.pack_experts(*(t.contiguous() for t in src), E, G, perm=None, layout="tau")
            del src
        self.router_packed = ops.pack_router(b["router"].contiguous(), layout="tau")
        if self.decode_workspace is None or self.decode_workspace.device != dev:
            self.decode_workspace = ops.decode_workspace(H, E, dev)
        self._release()
        self._packed_key = self._weights_key()

    def _ensure_packed(self) -> None:
        if self._packed_key is None or self._packed_key != self._weights_key():
            self.repack()

    @torch.no_grad()
    def load_from_masked(self, gate_weight: torch.Tensor, up_weight: torch.Tensor, down_weight: torch.Tensor,
                         router_weight: torch.Tensor, experts_masks_or_ids: torch.Tensor,
                         tau: Optional[float] = None) -> "TauSparseMoE":
        """One-time rearrangement from the masked model's weights
        (physical_reorder_for_inference, src/openpangu_moe.py:212-256).

        gate_weight/up_weight [I,H], down_weight [H,I] (nn.Linear), router_weight [E,H],
        experts_masks_or_ids: ``experts_masks`` [E,I] one-hot or neuron->expert ids [I].
        Neurons are grouped by expert with a stable order inside each expert.
        """
        dev = self._buffers["W_gate"].device
        ids = experts_masks_or_ids
        if ids.dim() == 2:
            ids = torch.argmax(ids.to(torch.int32), dim=0)
        ids = ids.to(device=dev, dtype=torch.int64)
        counts = torch.bincount(ids, minlength=self.num_experts)
        if counts.numel() != self.num_experts or bool((counts != self.group_size).any()):
            raise ValueError("load_from_masked: every expert must own exactly group_size neurons")
        perm = torch.argsort(ids, stable=True)
        gw = gate_weight.to(dev)
        uw = up_weight.to(dev)
        dw = down_weight.to(dev)
        # W_gate/W_up/W_down (gw[perm].T, uw[perm].T, dw[:, perm].T in bf16) are not formed:
        # the packed records below hold exactly those values (rebuilt from them on demand)
        self.router = router_weight.to(device=dev, dtype=torch.float32).t().contiguous()
        if tau is not None:
            self.tau = tau
        # pack straight from the fp32 masked weights (one bf16 rounding, as above)
        H, E, G = self.hidden_size, self.num_experts, self.group_size
        self.packed_experts = ops.pack_experts(gw.contiguous(), uw.contiguous(), dw.contiguous(), E, G,
                                               perm=perm.to(torch.int32), layout="linear")
        self.router_packed = ops.pack_router(router_weight.to(device=dev).contiguous(), layout="linear")
        if self.decode_workspace is None or self.decode_workspace.device != dev:
            self.decode_workspace = ops.decode_workspace(H, E, dev)
        self._release()
        self._packed_key = self._weights_key()
        return self

    # ------------------------------------------------------------------ decode errors
    def decode_error(self) -> int:
        """Sticky error bits of the decode workspace (0 = none; 1 = a logit wait timed
        out, 2 = inconsistent selection, 4 = reduction out of range). Synchronises."""
        if self.decode_workspace is None:
            return 0
        return ops.decode_state(self.decode_workspace, self.num_experts)["error"]

    def check_decode(self) -> None:
        """Raise RuntimeError if a decode call of this module failed (its outputs are NaN)."""
        err = self.decode_error()
        if err:
            raise RuntimeError(f"TauSparseMoE: decode failed (error bits {err:#x}); outputs since the failure "
                               "are NaN -- reset_decode_error() clears the flag")

    def reset_decode_error(self) -> None:
        """Re-initialise the decode workspace (clears the error flag)."""
        if self.decode_workspace is not None:
            ops.decode_workspace_init(self.decode_workspace, self.hidden_size, self.num_experts)

    # ------------------------------------------------------------------ forward
    def forward_decode(self, x_flat: torch.Tensor, B: int, L: int, H: int) -> torch.Tensor:
        # the op overload called directly with the buffers from _buffers: the eager host
        # cost of a decode call is what bounds an eager caller (the kernel takes ~11 us)
        b = self._buffers
        out = _decode_op()(x_flat, b["router_packed"], b["router_bias"], self.num_experts, self.group_size,
                           float(self.tau), b["packed_experts"], b["decode_workspace"], 0)
        if self.checked:
            self.check_decode()
        return out.view(B, L, H)

    def forward_decode_batch(self, x_flat: torch.Tensor, B: int, L: int, H: int) -> torch.Tensor:
        E, G = self.num_experts, self.group_size
        nb = ops.decode_batch_workspace_bytes(H, E, G)
        if self.batch_workspace is None or self.batch_workspace.device != x_flat.device or \
                self.batch_workspace.numel() < nb:
            self.batch_workspace = torch.empty(nb, dtype=torch.uint8, device=x_flat.device)
        out = ops.moe_decode_batch(x_flat, self.router_packed, self.router_bias, E, G, self.tau,
                                   self.packed_experts, self.decode_workspace, self.batch_workspace)
        if self.checked:
            self.check_decode()
        return out.view(B, L, H)

    def forward_prefill(self, N: int, x_flat: torch.Tensor, B: int, L: int, H: int) -> torch.Tensor:
        out = ops.moe_prefill(x_flat, self.router_packed, self.router_bias, self.num_experts, self.group_size,
                              self.tau, self.packed_experts)
        return out.view(B, L, H)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, L, H = x.shape
        if H != self.hidden_size:
            raise ValueError(f"TauSparseMoE: hidden size {H} != {self.hidden_size}")
        N = B * L
        self._ensure_packed()
        x_flat = x.reshape(N, H)
        if x_flat.dtype not in (torch.float32, torch.bfloat16):
            x_flat = x_flat.float()
        x_flat = x_flat.contiguous()
        if N == 0:
            return torch.empty(B, L, H, dtype=torch.bfloat16, device=x.device)
        if N == 1:
            return self.forward_decode(x_flat, B, L, H)
        if N <= self.batch_max and ops.decode_batch_supported(N, H, self.num_experts, self.group_size):
            return self.forward_decode_batch(x_flat, B, L, H)
        return self.forward_prefill(N, x_flat, B, L, H)
