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


def test_training_forward_has_no_cpu_fallback(pkg):
    """The masked training path runs the routing and gating kernels: CPU tensors are
    refused, not computed on the host."""
    cfg, ta = _cfg()
    m = pkg.IntegratedOpenPanguMoEMLP(cfg, ta)
    m.train()
    with pytest.raises(RuntimeError, match="GPU"):
        m(torch.zeros(1, 1, 256))


def test_penalty_losses_closed_forms(pkg):
    """src/openpangu_moe_origin.py:236-261 on inputs whose values are fixed by the
    definitions: uniform probabilities give entropy ln E and load balance 1; one-hot
    probabilities give entropy 0 and load balance E * sum_e f_e^2 (f_e = share of the
    valid tokens routed to e); masked-out tokens do not count; two layers average."""
    E, gamma, lbg = 16, 0.3, 0.7
    B, Lq = 2, 5
    uni = torch.full((B, Lq, E), 1.0 / E)
    ent, lb = pkg.penalty_losses([uni], None, E, gamma, lbg)
    assert abs(float(ent) - gamma * np.log(E)) < 1e-5
    assert abs(float(lb) - lbg * 1.0) < 1e-4
    ids = torch.tensor([[0, 0, 3, 5, 5], [5, 1, 0, 9, 9]])
    onehot = torch.nn.functional.one_hot(ids, E).float()
    am = torch.tensor([[1, 1, 1, 1, 0], [1, 1, 1, 0, 0]])  # 7 valid tokens: experts 0,0,3,5,5,1,0
    ent, lb = pkg.penalty_losses([onehot], am, E, gamma, lbg)
    assert float(ent) == 0.0
    f = np.bincount([0, 0, 3, 5, 5, 1, 0], minlength=E) / 7.0
    assert abs(float(lb) - lbg * E * float((f ** 2).sum())) < 1e-4
    # default lb_gamma = gamma; the two-layer average of the uniform and one-hot cases
    ent2, lb2 = pkg.penalty_losses([uni, onehot], am, E, gamma)
    assert abs(float(ent2) - gamma * np.log(E) / 2) < 1e-5
    assert abs(float(lb2) - gamma * (1.0 + E * float((f ** 2).sum())) / 2) < 1e-4
    z = pkg.penalty_losses([], None, E, gamma)
    assert float(z[0]) == 0.0 and float(z[1]) == 0.0


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


def test_moelayer_reference_constructor_and_statistics(pkg):
    """MoELayer(config, train_args, experts, experts_id=None) as in src/MoEBlock.py:106-162:
    width from the config (hidden_size * 4 when it has no intermediate_size), zero router,
    tau from train_args (0.95 default), contiguous default partition, counters that reset
    and report (element_counter, sparsity_accumulator)."""
    cfg = types.SimpleNamespace(hidden_size=64)
    m = pkg.MoELayer(cfg, types.SimpleNamespace(), 8)
    assert m.dimension == 256 and m.dimension_per_expert == 32 and m.tau == 0.95
    assert m.mlp_router[0].weight.shape == (8, 64) and float(m.mlp_router[0].weight.abs().sum()) == 0.0
    np.testing.assert_array_equal(m.expert_ids().numpy(), np.repeat(np.arange(8), 32))
    ids = np.random.default_rng(0).permutation(np.repeat(np.arange(8), 32))
    m2 = pkg.MoELayer(types.SimpleNamespace(hidden_size=64, intermediate_size=256),
                      types.SimpleNamespace(tau=0.7), 8, experts_id=ids)
    assert m2.tau == 0.7
    np.testing.assert_array_equal(m2.expert_ids().numpy(), ids)
    assert m2.get_sparsity_statistics() == (0, 0.0) and not m2.sparsity_tracking_enabled
    m2.element_counter.fill_(5)
    m2.reset_moe_sparsity_statistics()
    assert m2.sparsity_tracking_enabled and m2.get_sparsity_statistics() == (0, 0.0)
    with pytest.raises(ValueError):
        pkg.MoELayer(types.SimpleNamespace(hidden_size=64, intermediate_size=250), types.SimpleNamespace(), 8)


def test_expert_buffers_rebuilt_from_the_records(pkg):
    """Once packed, W_gate/W_up/W_down keep no storage: reading one, or state_dict(),
    rebuilds it from the packed records' rows region [I][3][H] (gate row, up row, down
    column of each rearranged neuron), and load_state_dict gives them storage again.
    Host logic only: the records are a synthetic buffer of random bf16 values, so a
    transposed or shifted index shows."""
    H, I, E, G = 128, 256, 4, 64
    m = pkg.TauSparseMoE(H, I, E, G, 0.7)
    rec = torch.randn(3 * I * H, generator=torch.Generator().manual_seed(5))
    packed = torch.cat([rec, torch.zeros(I * H)]).to(torch.bfloat16)  # + the down_t region
    m._buffers["packed_experts"] = packed
    m._release()
    assert all(m._buffers[n].numel() == 0 for n in ("W_gate", "W_up", "W_down"))
    r3 = packed[:3 * I * H].view(I, 3, H)
    sd = m.state_dict()
    assert sorted(sd) == ["W_down", "W_gate", "W_up", "router"]
    for name, want in (("W_gate", r3[:, 0, :].t()), ("W_up", r3[:, 1, :].t()), ("W_down", r3[:, 2, :])):
        assert sd[name].shape == want.shape and torch.equal(sd[name], want), name
    assert m._buffers["W_up"].numel() == 0  # state_dict() does not keep what it rebuilt
    w = m.W_up  # a read gives the buffer its storage again, in the same object
    assert w is m._buffers["W_up"] and torch.equal(w, r3[:, 1, :].t())
    assert m._rebuilt["W_up"] == (w.data_ptr(), w._version)
    # a state_dict loads into released buffers
    m._release()
    sd2 = {k: v.clone() + (1 if k != "router" else 0) for k, v in sd.items()}
    m.load_state_dict(sd2)
    assert torch.equal(m._buffers["W_down"], sd2["W_down"]) and "W_down" not in m._rebuilt
