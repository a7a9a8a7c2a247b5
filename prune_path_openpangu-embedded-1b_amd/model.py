"""Model-side drop-in for the openPangu MoE MLP: the eval path on the sparse kernels and
the masked training path.

Mirrors the module tree the reference builds around its kernels, so reference
checkpoints and model code line up key for key:

* ``IntegratedOpenPanguMoEMLP`` (src/openpangu_moe.py:43-130): ``gate_proj``,
  ``up_proj``, ``down_proj`` (nn.Linear, taken from the original MLP), ``moelayer``
  (``MoELayer``: ``mlp_router.0.weight``, ``experts_masks`` and the telemetry
  buffers), ``tau_moe`` (``TauSparseMoE``: ``W_gate``, ``W_up``, ``W_down``, ``router``).
  In eval mode ``forward`` runs the MI355X kernels through ``tau_moe``.
* ``physical_reorder_for_inference`` (src/openpangu_moe.py:212-256): neuron -> expert
  ids from ``experts_masks``, permuted weights into ``tau_moe`` (one packing pass),
  then the training-time projections and the masked layer are dropped.
* ``load_cluster_ids`` reads the reference's partition files
  (``Pangu_Clusters/layer_{i}_k{G}.txt``, written by ``np.savetxt`` as floats,
  src/openpangu_moe.py:188-209).
* Training (``IntegratedOpenPanguMoEMLP.train()``, src/openpangu_moe_origin.py:83-120):
  dense gate/up projections, ``MoELayer.forward`` (src/MoEBlock_origin.py:174-214) with
  the tau selection of the routing kernel on the fp32 router scores and the expert
  gating ``intermediate * (experts_prob @ experts_masks)`` as the masked-gate HIP
  kernels (forward and backward), then the down projection; the softmax probabilities
  go to ``penalize_logits_list`` for ``penalty_losses`` (entropy and load balance,
  src/openpangu_moe_origin.py:236-261).
"""
from __future__ import annotations

from typing import Any, Iterable, List, Optional

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .tau_sparse_moe import TauSparseMoE


def load_cluster_ids(path: str) -> np.ndarray:
    """Neuron -> expert ids from a reference partition file (one id per line, float
    formatted by np.savetxt). Raises if an entry is not an integer."""
    v = np.loadtxt(path, dtype=np.float64, ndmin=1)
    ids = np.rint(v)
    if not np.array_equal(ids, v):
        raise ValueError(f"{path}: non-integer expert id")
    return ids.astype(np.int32)


def experts_masks_from_ids(ids, num_experts: int, dtype=torch.float32) -> torch.Tensor:
    """[E, I] one-hot expert masks (MoELayer.experts_masks layout, src/MoEBlock.py:133-143)."""
    t = torch.as_tensor(np.asarray(ids), dtype=torch.long)
    return F.one_hot(t, num_classes=num_experts).t().to(dtype)


class MoELayer(nn.Module):
    """The reference's masked routing layer (src/MoEBlock.py:106-200, with the origin
    twin src/MoEBlock_origin.py:108-214): the router projection and the expert partition
    under the reference's names, and its forward
    ``(hidden_states, intermediate) -> (intermediate * mask, probs | None)``.

    Constructor as in the reference, ``MoELayer(config, train_args, experts,
    experts_id=None)``: the width is ``config.intermediate_size`` (the reference uses
    ``config.hidden_size * 4``, the same number for openPangu-Embedded-1B, and
    ``hidden_size * 4`` here too when the config has no ``intermediate_size``); the
    router ``Linear(hidden_size, experts, bias=False)`` starts at zero
    (``router_weights_init``, src/MoEBlock.py:98-103); ``tau`` comes from
    ``train_args.tau`` (default 0.95); ``experts_id`` (neuron -> expert, default
    contiguous blocks) builds the one-hot ``experts_masks`` [E, I].

    Telemetry (src/MoEBlock.py:145-162, 187-196): eval forwards add the per-expert
    activation counts to ``activated_statistics``; after
    ``reset_moe_sparsity_statistics()`` they also add the number of dropped (token,
    expert) gates to ``sparsity_accumulator`` and the number of gates to
    ``element_counter``, all on the device (no host sync); ``get_sparsity_statistics()``
    returns ``(element_counter, sparsity_accumulator)`` as Python numbers."""

    def __init__(self, config: Any, train_args: Any, experts: int, experts_id=None):
        super().__init__()
        self.config = config
        self.train_args = train_args
        self.experts = experts
        hidden = config.hidden_size
        self.dimension = getattr(config, "intermediate_size", None) or hidden * 4
        self.mlp_router = nn.Sequential(nn.Linear(hidden, experts, bias=False))
        nn.init.zeros_(self.mlp_router[0].weight)
        if self.dimension % experts:
            raise ValueError(f"MoELayer: dimension {self.dimension} is not divisible by {experts} experts")
        self.dimension_per_expert = self.dimension // experts
        if experts_id is None:
            experts_id = np.repeat(np.arange(experts), self.dimension_per_expert)
        self.register_buffer("experts_masks", experts_masks_from_ids(experts_id, experts,
                                                                      self.mlp_router[0].weight.dtype))
        self.register_buffer("activated_statistics", torch.zeros(experts, dtype=torch.long))
        self.register_buffer("sparsity_accumulator", torch.zeros(1, dtype=torch.double))
        self.register_buffer("element_counter", torch.zeros(1, dtype=torch.long))
        self.sparsity_tracking_enabled = False
        self.tau = getattr(train_args, "tau", 0.95)

    def reset_moe_sparsity_statistics(self) -> None:
        """Zero the sparsity counters and start tracking (src/MoEBlock.py:154-158)."""
        self.sparsity_tracking_enabled = True
        self.sparsity_accumulator.zero_()
        self.element_counter.zero_()

    def get_sparsity_statistics(self):
        """(gates seen, gates dropped) since the last reset (src/MoEBlock.py:160-162)."""
        return self.element_counter.item(), self.sparsity_accumulator.item()

    def expert_ids(self) -> torch.Tensor:
        """Neuron -> expert id [I] (argmax over the one-hot masks, src/openpangu_moe.py:229-230)."""
        return torch.argmax(self.experts_masks.to(torch.int32), dim=0)

    def _layout(self):
        """Expert ids / expert-sorted order for the masked-gate kernels, rebuilt when
        ``experts_masks`` changes (storage or in-place update)."""
        key = (self.experts_masks.data_ptr(), self.experts_masks._version, self.experts_masks.device)
        if getattr(self, "_layout_key", None) != key:
            self._layout_cache = ops.masked_gate_layout(self.expert_ids(), self.experts)
            self._layout_key = key
        return self._layout_cache

    def forward(self, hidden_states: torch.Tensor, intermediate: torch.Tensor):
        """src/MoEBlock_origin.py:174-214. score = router(hidden_states); the tau
        selection (softmax, descending sort, fp64-accumulated cumsum < tau, rank 0 always;
        src/MoEBlock_origin.py:50-97) comes from the routing kernel on the fp32 scores --
        bit-exact with the reference's torch ops given the same fp32 scores -- and
        experts_prob = sigmoid(score) on the selected experts, 0 elsewhere (the gradient of
        sigmoid(where(select, score, finfo.min))); the gating is the masked-gate kernel.
        Training returns the softmax probabilities for the penalties, eval updates
        ``activated_statistics``."""
        score = self.mlp_router(hidden_states)
        E = self.experts
        flat = score.detach().reshape(-1, E).float().contiguous()
        _, _, sel, _ = ops.route_logits(flat, float(self.tau))
        select = sel.view(score.shape).bool()
        experts_prob = torch.where(select, torch.sigmoid(score), torch.zeros((), dtype=score.dtype,
                                                                              device=score.device))
        probs = torch.softmax(score, dim=-1) if self.training else None
        if not self.training:
            flat = sel.reshape(-1, E)
            self.activated_statistics.add_(flat.sum(dim=0))
            if self.sparsity_tracking_enabled:
                # dropped gates: experts_prob <= 0 (src/MoEBlock.py:193-196); a selected
                # expert's gate is sigmoid(score) > 0 unless the score is -inf or NaN
                self.sparsity_accumulator.add_((experts_prob <= 0.0).sum())
                self.element_counter.add_(experts_prob.numel())
        out = ops.masked_gate(intermediate, experts_prob, self._layout())
        return out, probs


class IntegratedOpenPanguMoEMLP(nn.Module):
    """MoE MLP with the reference's module tree (src/openpangu_moe.py:43-130): eval runs
    the sparse kernels, training the masked path (src/openpangu_moe_origin.py:83-120).

    ``config`` needs ``hidden_size`` (and optionally ``intermediate_size``, default
    4 * hidden_size); ``train_args`` needs ``group_size`` (and optionally ``tau``).
    ``original_mlp`` supplies ``gate_proj``/``up_proj``/``down_proj`` (nn.Linear); new
    ones are created when it is None (for loading a checkpoint)."""

    def __init__(self, config: Any, train_args: Any, original_mlp: Optional[nn.Module] = None,
                 penalize_logits_list: Optional[List[torch.Tensor]] = None):
        super().__init__()
        self.config = config
        self.train_args = train_args
        H = getattr(config, "hidden_size", 1536)
        I = getattr(config, "intermediate_size", H * 4)
        G = train_args.group_size
        tau = getattr(train_args, "tau", 0.5)
        E = I // G
        if original_mlp is not None:
            self.gate_proj = getattr(original_mlp, "gate_proj", None)
            self.up_proj = getattr(original_mlp, "up_proj", None)
            self.down_proj = getattr(original_mlp, "down_proj", None)
            self.act_fn = getattr(original_mlp, "act_fn", None) or nn.SiLU()
        else:
            self.gate_proj = nn.Linear(H, I, bias=False)
            self.up_proj = nn.Linear(H, I, bias=False)
            self.down_proj = nn.Linear(I, H, bias=False)
            self.act_fn = nn.SiLU()
        self.penalize_logits_list = penalize_logits_list
        self.moelayer = MoELayer(config, train_args, E)
        self.tau_moe = TauSparseMoE(H, I, E, G, tau)

    def forward(self, hidden_states: torch.Tensor, *args, **kwargs) -> torch.Tensor:
        """Eval: the sparse kernels through ``tau_moe`` (src/openpangu_moe.py:123-127).
        Training: the masked path of src/openpangu_moe_origin.py:83-120 (dense gate/up,
        ``moelayer``, dense down); the probabilities go to ``penalize_logits_list``."""
        if not self.training:
            return self.tau_moe(hidden_states)
        if self.moelayer is None:
            raise RuntimeError("IntegratedOpenPanguMoEMLP: reordered for inference (projections dropped); "
                               "the masked training path needs them")
        intermediate = self.act_fn(self.gate_proj(hidden_states)) * self.up_proj(hidden_states)
        moe_intermediate, probs = self.moelayer(hidden_states, intermediate)
        if probs is not None and self.penalize_logits_list is not None:
            self.penalize_logits_list.append(probs)
        return self.down_proj(moe_intermediate)

    @torch.no_grad()
    def physical_reorder_for_inference(self, tau: float) -> None:
        """One layer of src/openpangu_moe.py:222-250: permuted weights into ``tau_moe``
        (fp32 router), then the projections and the masked layer are dropped."""
        if self.moelayer is None:
            raise RuntimeError("physical_reorder_for_inference: already reordered")
        self.tau_moe.load_from_masked(self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight,
                                      self.moelayer.mlp_router[0].weight, self.moelayer.experts_masks, tau)
        self.gate_proj = None
        self.up_proj = None
        self.down_proj = None
        self.moelayer = None


def physical_reorder_for_inference(layers: Iterable[nn.Module], tau: float) -> None:
    """Model-level reorder (src/openpangu_moe.py:212-256): every ``layer.mlp`` that is an
    ``IntegratedOpenPanguMoEMLP`` is reordered in place; the caching allocator is
    flushed at the end, as the reference does."""
    for layer in layers:
        mlp = getattr(layer, "mlp", layer)
        if isinstance(mlp, IntegratedOpenPanguMoEMLP):
            mlp.physical_reorder_for_inference(tau)
    if torch.cuda.is_available():
        torch.cuda.empty_cache()


def penalty_losses(penalize_logits_list: List[torch.Tensor], attention_mask: Optional[torch.Tensor],
                   experts: int, gamma: float, lb_gamma: Optional[float] = None):
    """Entropy and load-balance regularizers of the masked training step
    (src/openpangu_moe_origin.py:236-261), averaged over the recorded layers:
    entropy = mean over valid tokens of sum_e entr(p) (times gamma); load balance =
    experts * sum_e (mean over valid tokens of p_e)^2 (times lb_gamma, default gamma).
    Returns (entropy_loss, load_balance_loss); zeros when nothing was recorded."""
    if not penalize_logits_list:
        z = torch.zeros(())
        return z, z.clone()
    p0 = penalize_logits_list[0]
    dev = p0.device
    if attention_mask is None:
        mask_float = torch.ones(p0.shape[:-1], dtype=torch.float, device=dev)
    else:
        mask_float = attention_mask.float().to(dev)
    valid = mask_float.sum()
    eps = 1e-6
    lbg = gamma if lb_gamma is None else lb_gamma
    ent = torch.zeros((), device=dev)
    lb = torch.zeros((), device=dev)
    for probs in penalize_logits_list:
        entropy = torch.special.entr(probs).sum(dim=-1)
        ent = ent + (entropy * mask_float).sum() / (valid + eps) * gamma
        avg = (probs * mask_float.unsqueeze(-1)).reshape(-1, experts).sum(dim=0) / (valid + eps)
        lb = lb + (avg ** 2).sum() * experts * lbg
    n = len(penalize_logits_list)
    return ent / n, lb / n
