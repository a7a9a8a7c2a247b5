"""GPU parity of the masked training path (src/MoEBlock_origin.py:174-214,
src/openpangu_moe_origin.py:83-120 and :236-261).

* masked-gate kernels against the reference's torch ops on the CPU: the forward
  ``inter * (experts_prob @ experts_masks)`` bit for bit (fp32; bf16 as the all-bf16
  reference rounds it), the backward's d_inter bit for bit and d_gates against the
  float64 autograd of the same ops, repeat calls bitwise identical;
* a whole training step of ``IntegratedOpenPanguMoEMLP`` (forward, penalties,
  backward) against a float32 torch-CPU run of the reference's op sequence with the
  selection of the oracle on the same scores, which also pins the routing kernel's
  selection bit for bit.
"""
import types

import numpy as np
import pytest
import torch

from helpers import dev, oracle

pytestmark = pytest.mark.gpu


def _partition(I, E, seed):
    rng = np.random.default_rng(seed)
    return rng.permutation(np.repeat(np.arange(E, dtype=np.int32), I // E)).astype(np.int32)


def _gates(N, E, seed):
    g = torch.Generator().manual_seed(seed)
    v = torch.sigmoid(torch.randn(N, E, generator=g) * 2)
    v[torch.rand(N, E, generator=g) < 0.5] = 0.0  # unselected experts
    return v


@pytest.mark.parametrize("N,I,E", [(1, 1024, 16), (37, 6144, 16), (9, 6144, 192), (5, 16384, 256), (3, 512, 1)])
def test_masked_gate_fwd_bwd_vs_reference_ops(pkg, N, I, E):
    ops = pkg.ops
    ids = _partition(I, E, N + I + E)
    masks = torch.nn.functional.one_hot(torch.from_numpy(ids).long(), E).t().float()  # [E, I]
    g = torch.Generator().manual_seed(7)
    inter = torch.randn(N, I, generator=g)
    gates = _gates(N, E, 11)
    d_out = torch.randn(N, I, generator=g)
    layout = ops.masked_gate_layout(torch.from_numpy(ids).to(dev()), E)

    # fp32: the reference's two ops (one-hot matmul, multiply), bit for bit
    ref = inter * (gates @ masks)
    out = ops.masked_gate_fwd(inter.to(dev()), gates.to(dev()), layout[0]).cpu()
    np.testing.assert_array_equal(out.numpy(), ref.numpy())
    # backward vs autograd of the same ops in float64
    i64, g64 = inter.double().requires_grad_(), gates.double().requires_grad_()
    (i64 * (g64 @ masks.double())).backward(d_out.double())
    d_inter, d_gates = ops.masked_gate_bwd(d_out.to(dev()), inter.to(dev()), gates.to(dev()), *layout)
    np.testing.assert_array_equal(d_inter.cpu().numpy(), (d_out * (gates @ masks)).numpy())
    np.testing.assert_allclose(d_gates.cpu().numpy(), g64.grad.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(d_inter.cpu().double().numpy(), i64.grad.numpy(), rtol=1e-6, atol=0)
    d_inter2, d_gates2 = ops.masked_gate_bwd(d_out.to(dev()), inter.to(dev()), gates.to(dev()), *layout)
    np.testing.assert_array_equal(d_gates2.cpu().numpy(), d_gates.cpu().numpy())
    np.testing.assert_array_equal(d_inter2.cpu().numpy(), d_inter.cpu().numpy())

    # bf16: the all-bf16 reference (bf16 gates, bf16 product)
    ib = inter.bfloat16()
    refb = (ib.float() * (gates.bfloat16().float() @ masks)).bfloat16()
    outb = ops.masked_gate_fwd(ib.to(dev()), gates.to(dev()), layout[0]).cpu()
    np.testing.assert_array_equal(outb.view(torch.int16).numpy(), refb.view(torch.int16).numpy())
    db_inter, db_gates = ops.masked_gate_bwd(d_out.bfloat16().to(dev()), ib.to(dev()), gates.to(dev()), *layout)
    gb = gates.bfloat16().float()
    np.testing.assert_array_equal(db_inter.cpu().view(torch.int16).numpy(),
                                  (d_out.bfloat16().float() * (gb @ masks)).bfloat16().view(torch.int16).numpy())
    ref_dg = (d_out.bfloat16().double() * ib.double()) @ masks.double().t()
    np.testing.assert_allclose(db_gates.cpu().numpy(), ref_dg.numpy(), rtol=1e-5, atol=1e-5)


def test_masked_gate_rejects_bad_shapes(pkg):
    ops = pkg.ops
    with pytest.raises(RuntimeError):
        ops.masked_gate_fwd(torch.zeros(2, 12, device=dev()), torch.zeros(2, 4, device=dev()),
                            torch.zeros(12, dtype=torch.int32, device=dev()))  # I % 8 != 0
    with pytest.raises(RuntimeError):
        ops.masked_gate_layout(torch.tensor([0, 1, 4], dtype=torch.int32, device=dev()), 4)  # id outside [0, E)


def _ref_step(w, x, ids, tau, sel_mask, am, gamma, lbg, w_out, pkg):
    """float32 torch-CPU restatement of the reference's training step: dense SwiGLU
    (src/openpangu_moe_origin.py:96-99), MoELayer (src/MoEBlock_origin.py:188-212 with
    the selection given), down projection, penalties (:236-261)."""
    Wg, Wu, Wd, Wr = (torch.from_numpy(w[k]).clone().requires_grad_() for k in ("wg", "wu", "wd", "wr"))
    xx = torch.from_numpy(x).clone().requires_grad_()
    E = Wr.shape[0]
    masks = torch.nn.functional.one_hot(torch.from_numpy(ids).long(), E).t().float()
    inter = torch.nn.functional.silu(xx @ Wg.t()) * (xx @ Wu.t())
    score = xx @ Wr.t()
    experts_prob = torch.sigmoid(torch.where(torch.from_numpy(sel_mask), score,
                                             torch.full_like(score, torch.finfo(torch.float32).min)))
    out = (inter * (experts_prob @ masks)) @ Wd.t()
    probs = torch.softmax(score, dim=-1)
    ent, lb = pkg.penalty_losses([probs], am, E, gamma, lbg)
    loss = (out * w_out).sum() + ent + lb
    loss.backward()
    return out.detach(), score.detach(), {"wg": Wg.grad, "wu": Wu.grad, "wd": Wd.grad, "wr": Wr.grad, "x": xx.grad}


@pytest.mark.parametrize("H,I,G,tau", [(256, 1024, 64, 0.7), (256, 6144, 32, 0.7), (512, 2048, 128, 0.95)])
def test_masked_mlp_training_step_vs_reference(pkg, H, I, G, tau):
    E = I // G
    rng = np.random.default_rng(H + I + G)
    w = {"wg": rng.normal(0, 0.02, (I, H)).astype(np.float32), "wu": rng.normal(0, 0.02, (I, H)).astype(np.float32),
         "wd": rng.normal(0, 0.02, (H, I)).astype(np.float32), "wr": rng.normal(0, 0.1, (E, H)).astype(np.float32)}
    ids = _partition(I, E, H + G)
    B, Lq = 2, 8
    x = rng.standard_normal((B, Lq, H)).astype(np.float32)
    am = torch.ones(B, Lq, dtype=torch.long)
    am[1, 5:] = 0
    gamma, lbg = 0.05, 0.02
    w_out = torch.from_numpy(rng.standard_normal((B, Lq, H)).astype(np.float32))

    cfg = types.SimpleNamespace(hidden_size=H, intermediate_size=I)
    ta = types.SimpleNamespace(group_size=G, tau=tau)
    plist = []
    m = pkg.IntegratedOpenPanguMoEMLP(cfg, ta, penalize_logits_list=plist).to(dev())
    with torch.no_grad():
        m.gate_proj.weight.copy_(torch.from_numpy(w["wg"]))
        m.up_proj.weight.copy_(torch.from_numpy(w["wu"]))
        m.down_proj.weight.copy_(torch.from_numpy(w["wd"]))
        m.moelayer.mlp_router[0].weight.copy_(torch.from_numpy(w["wr"]))
        m.moelayer.experts_masks.copy_(pkg.experts_masks_from_ids(ids, E))
    m.train()
    xg = torch.from_numpy(x).to(dev()).requires_grad_()
    out = m(xg)
    assert len(plist) == 1
    ent, lb = pkg.penalty_losses(plist, am.to(dev()), E, gamma, lbg)
    ((out * w_out.to(dev())).sum() + ent + lb).backward()

    # the selection the kernels used, pinned against the oracle on the GPU's own scores
    with torch.no_grad():
        score_gpu = m.moelayer.mlp_router(xg).cpu().numpy()  # the same router call as the forward
    sel = oracle.select(score_gpu.reshape(-1, E), tau).mask.reshape(B, Lq, E).astype(bool)
    _, _, mask_k, _ = pkg.ops.route_logits(torch.from_numpy(score_gpu.reshape(-1, E)).to(dev()), tau)
    np.testing.assert_array_equal(mask_k.cpu().numpy().reshape(B, Lq, E).astype(bool), sel)

    ref_out, _, ref_grads = _ref_step(w, x, ids, tau, sel, am, gamma, lbg, w_out, pkg)

    def rel(a, b):
        a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
        return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)

    assert rel(out.detach().cpu().numpy(), ref_out.numpy()) < 1e-5
    got = {"wg": m.gate_proj.weight.grad, "wu": m.up_proj.weight.grad, "wd": m.down_proj.weight.grad,
           "wr": m.moelayer.mlp_router[0].weight.grad, "x": xg.grad}
    for k, v in got.items():
        assert rel(v.cpu().numpy(), ref_grads[k].numpy()) < 1e-4, k


def test_masked_layer_eval_statistics(pkg):
    """Eval-mode MoELayer.forward (the reference's origin path) counts the selections per
    expert in activated_statistics and returns no probabilities; after
    reset_moe_sparsity_statistics the dropped / total gate counts accumulate on the device
    (src/MoEBlock.py:154-162, 187-196)."""
    import types
    H, I, E = 256, 1024, 16
    cfg = types.SimpleNamespace(hidden_size=H, intermediate_size=I)
    layer = pkg.MoELayer(cfg, types.SimpleNamespace(tau=0.7), E).to(dev())
    assert float(layer.mlp_router[0].weight.detach().abs().sum()) == 0.0  # router_weights_init: zeros
    with torch.no_grad():
        layer.mlp_router[0].weight.normal_(0, 0.1)
    layer.eval()
    x = torch.randn(3, 5, H, device=dev())
    inter = torch.randn(3, 5, I, device=dev())
    assert layer.get_sparsity_statistics() == (0, 0.0)
    layer.reset_moe_sparsity_statistics()
    with torch.no_grad():
        out, probs = layer(x, inter)
        layer(x[:1], inter[:1])
    assert probs is None
    with torch.no_grad():
        score = layer.mlp_router(x).reshape(-1, E).cpu().numpy()
    sel = oracle.select(score, 0.7)
    sel1 = oracle.select(score.reshape(3, 5, E)[:1].reshape(-1, E), 0.7)
    np.testing.assert_array_equal(layer.activated_statistics.cpu().numpy(), sel.mask.sum(0) + sel1.mask.sum(0))
    n, dropped = layer.get_sparsity_statistics()
    assert n == 20 * E and dropped == float(20 * E - sel.mask.sum() - sel1.mask.sum())
    ids = layer.expert_ids().cpu().numpy()
    ref = inter.cpu().numpy().reshape(-1, I) * sel.gates[:, ids]
    np.testing.assert_allclose(out.cpu().numpy().reshape(-1, I), ref, rtol=1e-6, atol=1e-7)
