"""torch-CPU fp32 restatement of the reference's dense masked MoE-MLP layer -- TEST
INFRASTRUCTURE / CPU BASELINE ONLY.

Only ``tests/`` and ``bench.py``'s ``cpu_baseline`` leg use this module: it is the
reference's own CPU path, timed as the baseline the GPU numbers are reported beside, and
a second restatement the tests hold against the golden fixtures. The product package
never imports it.

Op for op, in the reference's order (paths relative to the reference repository root):
* ``IntegratedOpenPanguMoEMLP.forward`` (src/openpangu_moe_origin.py:96-118): dense
  ``act_fn(gate_proj(x)) * up_proj(x)`` over all I neurons, the masked layer, then
  ``down_proj``;
* ``MoELayer.forward`` (src/MoEBlock_origin.py:188-212): ``score = mlp_router(x)``,
  ``softmax_thresholding``, ``experts_prob @ experts_masks``, ``intermediate * mask``;
* ``softmax_thresholding`` (src/MoEBlock_origin.py:70-93): softmax, descending sort,
  cumsum, ``cum < tau``, scatter back, top-1 fallback, sigmoid of the kept logits
  (``finfo.min`` elsewhere).
The optional router bias (not in the reference) is the Zipf skew of the small-batch
benchmark configuration, added to the scores.

Pinned in tests/test_oracle.py against the config-1 fixture (torch fp32, the layer's
output) and against ``oracle.select`` (the selection, bit for bit).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def softmax_thresholding(logits: torch.Tensor, tau: float):
    """(gates, select_mask) of src/MoEBlock_origin.py:70-93 on logits [..., E] (eval mode)."""
    y_soft = torch.softmax(logits, dim=-1)
    sorted_prob, sorted_idx = torch.sort(y_soft, dim=-1, descending=True)
    cum_prob = torch.cumsum(sorted_prob, dim=-1)
    mask = cum_prob < tau
    select_mask = torch.zeros_like(mask, dtype=torch.bool)
    select_mask.scatter_(dim=-1, index=sorted_idx, src=mask)
    none = select_mask.sum(dim=-1) == 0
    if none.any():
        rows = torch.nonzero(none, as_tuple=True)
        select_mask[rows + (sorted_idx[..., 0][rows],)] = True
    safe = torch.full_like(logits, torch.finfo(logits.dtype).min)
    return torch.sigmoid(torch.where(select_mask, logits, safe)), select_mask


class MaskedLayer:
    """One dense masked MoE-MLP layer in torch fp32 on the CPU.

    w_gate / w_up [I, H], w_down [H, I], w_router [E, H] (nn.Linear layouts) and the
    neuron -> expert ids [I] (numpy or torch)."""

    def __init__(self, w_gate, w_up, w_down, w_router, expert_ids, bias=None):
        t = lambda a: torch.as_tensor(a, dtype=torch.float32).contiguous()  # noqa: E731
        self.w_gate, self.w_up, self.w_down, self.w_router = t(w_gate), t(w_up), t(w_down), t(w_router)
        E = self.w_router.shape[0]
        ids = torch.as_tensor(expert_ids, dtype=torch.long)
        self.experts_masks = F.one_hot(ids, num_classes=E).t().to(torch.float32).contiguous()  # [E, I]
        self.bias = None if bias is None else t(bias)

    @torch.no_grad()
    def __call__(self, x: torch.Tensor, tau: float) -> torch.Tensor:
        x = torch.as_tensor(x, dtype=torch.float32)
        intermediate = F.silu(F.linear(x, self.w_gate)) * F.linear(x, self.w_up)
        score = F.linear(x, self.w_router)
        if self.bias is not None:
            score = score + self.bias
        experts_prob, _ = softmax_thresholding(score, tau)
        mask = experts_prob @ self.experts_masks
        return F.linear(intermediate * mask, self.w_down)

    @torch.no_grad()
    def route(self, x: torch.Tensor, tau: float):
        """(score, (gates, select_mask)) of the layer's router on x."""
        score = F.linear(torch.as_tensor(x, dtype=torch.float32), self.w_router)
        if self.bias is not None:
            score = score + self.bias
        return score, softmax_thresholding(score, tau)
