"""Model-side drop-in, host logic (no GPU): reference state_dict keys, cluster files."""
import os
import types

import numpy as np
import pytest
import torch

from helpers import GOLDEN

# state_dict keys of the reference's IntegratedOpenPanguMoEMLP after model surgery
# (src/openpangu_moe.py:59-92; MoELayer src/MoEBlock.py:125-148; TauSparseMoE
# src/tl_kernel_optimized_Ultimate_PanGU.py:483-486; decode scratch is non-persistent)
REFERENCE_KEYS = {
    "gate_proj.weight", "up_proj.weight", "down_proj.weight",
    "moelayer.mlp_router.0.weight", "moelayer.experts_masks", "moelayer.activated_statistics",
    "moelayer.sparsity_accumulator", "moelayer.element_counter",
    "tau_moe.W_gate", "tau_moe.W_up", "tau_moe.W_down", "tau_moe.router",
}


def _cfg(H=256, I=1024, G=64, tau=0.7):
    return types.SimpleNamespace(hidden_size=H, intermediate_size=I), types.SimpleNamespace(group_size=G, tau=tau)


def test_state_dict_keys_match_reference(pkg):
    cfg, ta = _cfg()
    m = pkg.IntegratedOpenPanguMoEMLP(cfg, ta)
    sd = m.state_dict()
    assert set(sd) == REFERENCE_KEYS
    assert sd["moelayer.experts_masks"].shape == (16, 1024)
    assert sd["tau_moe.W_gate"].shape == (256, 1024) and sd["tau_moe.W_gate"].dtype == torch.bfloat16
    assert sd["moelayer.mlp_router.0.weight"].shape == (16, 256)


def test_original_mlp_projections_are_taken_over(pkg):
    cfg, ta = _cfg()
    orig = torch.nn.Module()
    orig.gate_proj = torch.nn.Linear(256, 1024, bias=False)
    orig.up_proj = torch.nn.Linear(256, 1024, bias=False)
    orig.down_proj = torch.nn.Linear(1024, 256, bias=False)
    m = pkg.IntegratedOpenPanguMoEMLP(cfg, ta, orig, [])
    assert m.gate_proj is orig.gate_proj and m.down_proj is orig.down_proj


def test_training_forward_is_not_built(pkg):
    cfg, ta = _cfg()
    m = pkg.IntegratedOpenPanguMoEMLP(cfg, ta)
    m.train()
    with pytest.raises(NotImplementedError):
        m(torch.zeros(1, 1, 256))


def test_load_cluster_ids_reference_format(pkg, tmp_path):
    """np.savetxt float format, as the reference writes its partition files
    (src/openpangu_moe.py:201-203); round trip through experts_masks."""
    ids = np.load(os.path.join(GOLDEN, "pangu_clusters_k32.npz"))["expert_ids"][5]
    f = tmp_path / "layer_5_k32.txt"
    np.savetxt(f, ids.astype(np.float64))
    got = pkg.load_cluster_ids(str(f))
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, ids)
    masks = pkg.experts_masks_from_ids(got, 192)
    assert masks.shape == (192, 6144)
    np.testing.assert_array_equal(torch.argmax(masks.to(torch.int32), 0).numpy(), ids)
    bad = tmp_path / "bad.txt"
    np.savetxt(bad, np.array([0.0, 1.5]))
    with pytest.raises(ValueError):
        pkg.load_cluster_ids(str(bad))
