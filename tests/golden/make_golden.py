"""Writes the committed golden fixtures under tests/golden/.

Run in the build container (torch 2.10 CPU, AVX512 -- the torch version the
reference pins in requirements.txt:3):  python tests/golden/make_golden.py

The expected values come from torch CPU ops applied in the order the reference
applies them (src/MoEBlock_origin.py:50-97 for routing; src/openpangu_moe_origin.py:96-118
with src/MoEBlock_origin.py:188-212 for the layer). Nothing from the reference
repository is imported; the cluster-map fixture is data read from its text files
(src/Pangu_Clusters/layer_*_k32.txt) when that directory is present.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import inputs as gi  # noqa: E402

torch.set_num_threads(1)


def torch_route(logits: torch.Tensor, tau: float):
    """torch ops of softmax_thresholding (src/MoEBlock_origin.py:70-93), any leading dims."""
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
    gates = torch.sigmoid(torch.where(select_mask, logits, safe))
    return gates, y_soft, select_mask


TAUS = (0.0, 0.5, 0.7, 0.95, 1.05)


def make_routing(E: int, n: int, seed: int):
    fam = gi.routing_logits(seed, n, E)
    out = {"E": np.int32(E), "taus": np.array(TAUS, np.float32)}
    for name, lg in fam.items():
        t = torch.from_numpy(lg)
        out[f"{name}/logits"] = lg
        for ti, tau in enumerate(TAUS):
            gates, probs, sel = torch_route(t, tau)
            out[f"{name}/tau{ti}/gates"] = gates.numpy()
            out[f"{name}/tau{ti}/mask"] = np.packbits(sel.numpy().astype(np.uint8), axis=-1)
            if ti == 0:
                out[f"{name}/probs"] = probs.numpy()
    path = os.path.join(HERE, f"routing_E{E}.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


def make_layer(name: str, seed_w: int, seed_x: int, n: int, taus, balanced_random=True):
    w = gi.layer_weights(seed_w, balanced_random=balanced_random)
    x = gi.tokens(seed_x, n)
    xt = torch.from_numpy(x)[None]  # [1, n, H] like the reference's [B, L, H]
    Wg, Wu, Wd, Wr = (torch.from_numpy(w[k]) for k in ("w_gate", "w_up", "w_down", "w_router"))
    inter = F.silu(F.linear(xt, Wg)) * F.linear(xt, Wu)
    score = F.linear(xt, Wr)
    onehot = F.one_hot(torch.from_numpy(w["expert_ids"]).long(), gi.E).t().float()
    res = {"seed_w": np.int32(seed_w), "seed_x": np.int32(seed_x), "n": np.int32(n),
           "balanced_random": np.int32(balanced_random),
           "input_sha256": np.array(gi.sha256(x, w["w_gate"], w["w_up"], w["w_down"],
                                              w["w_router"], w["expert_ids"])),
           "taus": np.array(taus, np.float32), "logits": score[0].numpy()}
    for ti, tau in enumerate(taus):
        gates, probs, sel = torch_route(score, tau)
        out = F.linear(inter * (gates @ onehot), Wd)
        res[f"tau{ti}/gates"] = gates[0].numpy()
        res[f"tau{ti}/out"] = out[0].numpy()
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **res)
    print("wrote", path)


def make_clusters():
    src = "/root/reference/src/Pangu_Clusters"
    if not os.path.isdir(src):
        print("cluster maps not present; keeping the committed fixture")
        return
    layers = []
    for i in range(26):
        ids = np.loadtxt(os.path.join(src, f"layer_{i}_k32.txt"), dtype=np.float64)
        layers.append(ids.astype(np.uint8))
    arr = np.stack(layers)
    path = os.path.join(HERE, "pangu_clusters_k32.npz")
    np.savez_compressed(path, expert_ids=arr)
    print("wrote", path, arr.shape)


if __name__ == "__main__":
    make_routing(16, 512, 101)
    make_routing(24, 256, 102)
    make_routing(32, 256, 103)
    make_routing(192, 64, 104)
    # 8 tokens, seed 0, tau 0.95 (plus tau 0.70 on the same layer)
    make_layer("c1_layer", seed_w=0, seed_x=1, n=8, taus=(0.95, 0.70))
    make_layer("c1_layer_contig", seed_w=2, seed_x=3, n=8, taus=(0.95,), balanced_random=False)
    make_clusters()
