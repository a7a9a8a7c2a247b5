"""GPU parity of the full MoE-MLP layer: fused decode and grouped-GEMM prefill.

Bars:
* selection bit-exact against the oracle applied to the kernel's own fp32 logits;
* bf16 outputs within rtol 2e-2 / atol 2e-3, elementwise, of the float64 sparse
  restatement on the same bf16 operands (the kernels' own arithmetic error);
* against the fp32 masked reference (torch CPU fixture of
  src/openpangu_moe_origin.py:96-118): rtol 2e-2 / atol 2e-3 plus the per-element
  bf16 quantization term of the operands, and normwise relative error < 1e-2
  (helpers.assert_close_fp32 explains why the bare tolerance is unreachable for
  any bf16-weight implementation).
"""
import os

import numpy as np
import pytest
import torch

from helpers import (GOLDEN, abi_prefill as _abi_prefill, assert_close, assert_close_fp32, bits, gi, make_module,
                     oracle, sparse_expected, sparse_expected_gpu, to_gpu)

pytestmark = pytest.mark.gpu


def _c1(name="c1_layer"):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    w = gi.layer_weights(int(z["seed_w"]), balanced_random=bool(z["balanced_random"]))
    x = gi.tokens(int(z["seed_x"]), int(z["n"]))
    return z, w, x


@pytest.fixture(scope="module")
def c1(pkg):
    z, w, x = _c1()
    return z, w, x, make_module(pkg, w, float(z["taus"][0]))


def _decode_one(pkg, m, xrow):
    out = m(to_gpu(xrow[None, None, :]))
    st = pkg.ops.decode_state(m.decode_workspace, m.num_experts)
    return out.float().cpu().numpy()[0, 0], st


@pytest.mark.parametrize("ti", [0, 1])
def test_decode_c1_vs_fixture(pkg, c1, ti):
    z, w, x, m = c1
    tau = float(z["taus"][ti])
    m.tau = tau
    epoch = None
    for t in range(x.shape[0]):
        out, st = _decode_one(pkg, m, x[t])
        assert st["error"] == 0
        # the E = 16 kernel's call epoch (act bank parity) advances by one per call; the
        # general kernel's epoch is left alone
        if epoch is not None:
            assert st["epoch16"] == epoch[0] + 1 and st["router_ticket"] == epoch[1]
        epoch = (st["epoch16"], st["router_ticket"])
        lg = st["logits"].numpy()
        np.testing.assert_allclose(lg, z["logits"][t], rtol=1e-5, atol=1e-5)
        sel = oracle.select(lg[None], tau)
        # selection: descending-probability order, gates bit-exact
        np.testing.assert_array_equal(st["sel_ids"].numpy(), sel.ranked[0, :sel.count[0]])
        np.testing.assert_array_equal(bits(st["sel_gates"].numpy()),
                                      bits(sel.gates[0, sel.ranked[0, :sel.count[0]]]))
        ref_sel = oracle.select(z["logits"][t:t + 1], tau)
        sp = sparse_expected(x[t:t + 1], w, sel.gates)[0]
        if np.array_equal(ref_sel.mask, sel.mask):
            assert_close_fp32(out, z[f"tau{ti}/out"][t], sp, what=f"decode token {t} vs fp32 fixture")
        assert_close(out, sp, what=f"decode token {t} vs fp64 sparse")


def test_decode_repeated_calls_and_bf16_input(pkg, c1):
    z, w, x, m = c1
    m.tau = 0.7
    outs = []
    for rep in range(3):
        for t in (0, 5, 2):
            o, st = _decode_one(pkg, m, x[t])
            assert st["error"] == 0
            outs.append((t, o))
    for t, o in outs:  # bitwise: the fixed-point reduction's sum does not depend on atomic order
        ref = [oo for tt, oo in outs if tt == t][0]
        np.testing.assert_array_equal(o, ref)
    xb = torch.from_numpy(x[3]).to(torch.bfloat16)
    o = m(xb.view(1, 1, -1).to("cuda:0")).float().cpu().numpy()[0, 0]
    st = pkg.ops.decode_state(m.decode_workspace, m.num_experts)
    sel = oracle.select(st["logits"].numpy()[None], 0.7)
    xr = xb.float().numpy()
    assert_close(o, sparse_expected(xr[None], w, sel.gates)[0], what="bf16 input decode")


@pytest.mark.parametrize("tau", [0.0, 0.3, 1.05])
def test_decode_tau_extremes(pkg, c1, tau):
    z, w, x, m = c1
    m.tau = tau
    out, st = _decode_one(pkg, m, x[1])
    sel = oracle.select(st["logits"].numpy()[None], tau)
    assert st["k"] == sel.count[0]
    if tau == 0.0:
        assert st["k"] == 1
    if tau > 1:
        assert st["k"] == 16
    assert_close(out, sparse_expected(x[1:2], w, sel.gates)[0], what=f"tau={tau}")


@pytest.mark.parametrize("grid", [16, 64, 1000])
def test_decode_grid_sizes(pkg, c1, grid):
    z, w, x, m = c1
    out = pkg.ops.moe_decode(to_gpu(x[4]), m.router_packed, None, 16, 384, 0.95, m.packed_experts,
                             m.decode_workspace, grid=grid).float().cpu().numpy()[0]
    st = pkg.ops.decode_state(m.decode_workspace, 16)
    assert st["error"] == 0
    sel = oracle.select(st["logits"].numpy()[None], 0.95)
    assert_close(out, sparse_expected(x[4:5], w, sel.gates)[0], what=f"grid={grid}")


def test_prefill_c1_vs_fixture(pkg, c1):
    z, w, x, m = c1
    for ti, tau in enumerate(z["taus"]):
        m.tau = float(tau)
        res = pkg.ops.route(to_gpu(x), m.router_packed, 16, float(tau))
        lg = res["logits"].cpu().numpy()
        sel = oracle.select(lg, float(tau))
        np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
        ref_sel = oracle.select(z["logits"], float(tau))
        same = np.all(ref_sel.mask == sel.mask, axis=1)
        assert same.sum() >= 7
        sp = sparse_expected(x, w, sel.gates)
        # the module (8 tokens: the one-launch batch kernel) and the prefill pipeline
        outs = {"module": m(to_gpu(x[None])).float().cpu().numpy()[0],
                "prefill": pkg.ops.moe_prefill(to_gpu(x), m.router_packed, None, 16, 384, float(tau),
                                               m.packed_experts).float().cpu().numpy()}
        for name, out in outs.items():
            assert_close_fp32(out[same], z[f"tau{ti}/out"][same], sp[same], what=f"{name} vs fp32 fixture")
            assert_close(out, sp, what=f"{name} vs fp64 sparse")


def _layer(seed, H=1536, E=16, G=384):
    w = gi.layer_weights(seed, H=H, I=E * G, E=E)
    return w


@pytest.mark.parametrize("N,tau,zipf", [(2, 0.7, False), (37, 0.7, False), (16, 0.95, True),
                                        (64, 0.95, True), (300, 0.7, False), (2048, 0.7, False),
                                        (8200, 0.7, False)])
def test_prefill_shapes_vs_oracle(pkg, N, tau, zipf):
    w = _layer(100 + N)
    bias = gi.zipf_bias(16) if zipf else None
    m = make_module(pkg, w, tau, bias=bias)
    x = gi.tokens(200 + N, N)
    prefill = lambda: pkg.ops.moe_prefill(to_gpu(x), m.router_packed, m.router_bias, 16, 384, tau,
                                          m.packed_experts).float().cpu().numpy()
    out = prefill()
    res = pkg.ops.route(to_gpu(x), m.router_packed, 16, tau, bias=m.router_bias)
    sel = oracle.select(res["logits"].cpu().numpy(), tau)
    np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
    # every row: float64 reference on the GPU (the numpy restatement pins it on a slice)
    exp = sparse_expected_gpu(x, w, sel.gates)
    sl = slice(0, min(N, 24))
    np.testing.assert_allclose(exp[sl], sparse_expected(x[sl], w, sel.gates[sl]), rtol=1e-9, atol=1e-12)
    assert_close(out, exp, what=f"prefill N={N}")
    # deterministic: bitwise identical on a second call
    np.testing.assert_array_equal(prefill(), out)
    # the module: the batch kernel for N <= 64, the prefill pipeline beyond
    om = m(to_gpu(x[None])).float().cpu().numpy()[0]
    assert_close(om, exp, what=f"module N={N}")
    np.testing.assert_array_equal(m(to_gpu(x[None])).float().cpu().numpy()[0], om)


def test_prefill_stages_vs_oracle(pkg):
    """gate/up+SwiGLU act and down y per pair, checked separately."""
    N, tau = 512, 0.7
    w = _layer(7)
    m = make_module(pkg, w, tau)
    x = gi.tokens(8, N)
    xb = to_gpu(x, torch.bfloat16)
    res = pkg.ops.route(xb, m.router_packed, 16, tau)
    bk = pkg.ops.bucket(res["mask"], res["gates"])
    act = pkg.ops.expert_gateup(xb, m.packed_experts, 16, 384, bk)
    y = pkg.ops.expert_down(act, m.packed_experts, 1536, 16, 384, bk)
    out = pkg.ops.combine(y, bk["token_pairs"], res["count"], 1536, 16)
    torch.cuda.synchronize()
    off = bk["offsets"].cpu().numpy()
    tok = bk["token_ids"].cpu().numpy()
    pg = bk["pair_gates"].cpu().numpy()
    perm = oracle.pack_permutation(w["expert_ids"])
    from helpers import bf16_round
    Wg = bf16_round(w["w_gate"])[perm].astype(np.float64)
    Wu = bf16_round(w["w_up"])[perm].astype(np.float64)
    Wd = bf16_round(w["w_down"])[:, perm].T.astype(np.float64)
    xr = xb.float().cpu().numpy().astype(np.float64)
    act_np = act.float().cpu().numpy()
    y_np = y.float().cpu().numpy()
    rng = np.random.default_rng(0)
    for p in rng.choice(off[-1], 64, replace=False):
        e = int(np.searchsorted(off, p, side="right") - 1)
        sl = slice(e * 384, (e + 1) * 384)
        g = xr[tok[p]] @ Wg[sl].T
        u = xr[tok[p]] @ Wu[sl].T
        a = g / (1 + np.exp(-g)) * u * pg[p]
        assert_close(act_np[p], a, what=f"act pair {p}")
        assert_close(y_np[p], act_np[p].astype(np.float64) @ Wd[sl], what=f"y pair {p}")
    full = m(xb[None]).float().cpu().numpy()[0]
    np.testing.assert_array_equal(out.float().cpu().numpy(), full)


def test_prefill_dense_form_e192(pkg):
    """E = 192, G = 32 (the checkpoint's shape: the dense form of csrc/dense.hip), 1000 tokens:
    * the routing the call used (its own logits, read back): the selection bit-exact against
      the oracle on those logits, and every row against the float64 restatement with that
      selection, acts rounded to bf16 (the reference's rounding point);
    * the C ABI and the torch op (module) give the same bits, and repeated calls too;
    * the logits of a token do not depend on the batch: rows 500..599 routed alone equal
      the same rows of the 1000-token call, and pp_route gives the same logits;
    * no global torch state reaches the routing (TF32 allowed or not: the same logits)."""
    E, G, N, H = 192, 32, 1000, 1536
    w = gi.layer_weights(41, E=E)
    m = make_module(pkg, w, 0.7)
    x = gi.tokens(42, N)
    xg = to_gpu(x)
    y, lg, mk = _abi_prefill(pkg, m, xg, E, G)
    sel = oracle.select(lg.cpu().numpy(), 0.7)
    np.testing.assert_array_equal(mk.cpu().numpy(), sel.mask)
    out = y.float().cpu().numpy()
    assert_close(out, sparse_expected_gpu(x, w, sel.gates, act_bf16=True), what="E=192 dense prefill (C ABI)")
    outm = m(xg[None]).float().cpu()
    assert torch.equal(outm[0], y.float().cpu()), "module (torch op) and C ABI differ"
    assert torch.equal(m(xg[None]).float().cpu(), outm), "repeated call differs"
    _, lg2, mk2 = _abi_prefill(pkg, m, xg[500:600].contiguous(), E, G)
    assert torch.equal(lg2, lg[500:600]) and torch.equal(mk2, mk[500:600])
    res = pkg.ops.route(xg, m.router_packed, E, 0.7)
    assert torch.equal(res["logits"], lg) and torch.equal(res["mask"], mk)
    old = torch.backends.cuda.matmul.allow_tf32
    try:
        torch.backends.cuda.matmul.allow_tf32 = True
        torch.set_float32_matmul_precision("high")
        _, lg3, _ = _abi_prefill(pkg, m, xg, E, G)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old
        torch.set_float32_matmul_precision("highest")
    assert torch.equal(lg3, lg)


@pytest.mark.parametrize("H,E,G,N,xdt", [
    (384, 1, 32, 1, torch.float32),      # the smallest call: one token, one 32-neuron expert
    (128, 3, 32, 5, torch.bfloat16),     # I = 96: the down GEMM's K padded to 128 with zero acts
    (4096, 192, 32, 300, torch.float32), # H = 4096, two row tiles (the second ragged)
    (640, 5, 160, 70, torch.float32),    # G = 160: experts straddle K blocks; a short last hidden tile
    (1536, 24, 32, 257, torch.bfloat16), # E = 24 (two 16-expert logit tiles), bf16 x, ragged N
    (1536, 16, 96, 40, torch.float32),   # E = 16 with G % 64 != 0: the E = 16 router feeds the dense form
    (1536, 192, 32, 1800, torch.float32),  # whole rounds of 256-row gate/up tiles, then 128-row tiles; ragged N
])
def test_prefill_dense_form_shapes(pkg, H, E, G, N, xdt):
    """The dense form across shapes: selection bit-exact on the call's own logits, every row
    against the float64 restatement (acts rounded to bf16), a router bias on E > 1."""
    seed = H + E * 5 + G + N
    w = gi.layer_weights(seed, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.7, bias=gi.zipf_bias(E) if E > 1 else None)
    x = gi.tokens(seed + 1, N, H=H)
    xg = to_gpu(x, xdt)
    y, lg, mk = _abi_prefill(pkg, m, xg, E, G)
    sel = oracle.select(lg.cpu().numpy(), 0.7)
    np.testing.assert_array_equal(mk.cpu().numpy(), sel.mask)
    xr = xg.float().cpu().numpy()
    assert_close(y.float().cpu().numpy(), sparse_expected(xr, w, sel.gates, act_bf16=True),
                 what=f"dense form H={H} E={E} G={G} N={N}")
    y2, _, _ = _abi_prefill(pkg, m, xg, E, G, routed=False)
    assert torch.equal(y, y2)


def test_prefill_dense_form_unselected_expert_not_evaluated(pkg):
    """An expert no token selects may hold huge weights: its gate/up products overflow to
    inf, and inf * 0 would make NaN. The dense form never evaluates an unselected expert's
    act (gate 0 -> act exactly 0), so the outputs stay finite and equal the restatement."""
    E, G, N, H = 8, 32, 64, 256
    w = gi.layer_weights(77, H=H, I=E * G, E=E)
    w["w_router"][5] = -1.0 * np.abs(w["w_router"][5]).sum() - 50.0  # expert 5: never selected
    x = np.abs(gi.tokens(78, N, H=H)).astype(np.float32)
    perm = oracle.pack_permutation(w["expert_ids"])
    hot = perm[5 * G:6 * G]  # source neurons of rearranged expert 5
    w2 = {k: v.copy() for k, v in w.items()}
    w2["w_gate"][hot] = 3e38
    w2["w_up"][hot] = 3e38
    m2 = make_module(pkg, w2, 0.7)
    xg = to_gpu(x)
    y, lg, mk = _abi_prefill(pkg, m2, xg, E, G)
    assert not mk.cpu().numpy()[:, 5].any()
    out = y.float().cpu().numpy()
    assert np.isfinite(out).all()
    sel = oracle.select(lg.cpu().numpy(), 0.7)
    assert_close(out, sparse_expected(x, w, sel.gates, act_bf16=True), what="huge unselected expert")


def test_real_checkpoint_shape_e192_g32(pkg):
    """E=192 experts of G=32 neurons with a reference cluster map (layer 3)."""
    ids = np.load(os.path.join(GOLDEN, "pangu_clusters_k32.npz"))["expert_ids"][3].astype(np.int32)
    w = gi.layer_weights(31, E=192)
    w["expert_ids"] = ids
    m = make_module(pkg, w, 0.7)
    x = gi.tokens(32, 96)
    out = m(to_gpu(x[None])).float().cpu().numpy()[0]
    y, lg, mk = _abi_prefill(pkg, m, to_gpu(x), 192, 32)
    sel = oracle.select(lg.cpu().numpy(), 0.7)
    np.testing.assert_array_equal(mk.cpu().numpy(), sel.mask)  # the path's own routing
    np.testing.assert_array_equal(y.float().cpu().numpy(), out)
    assert_close(out, sparse_expected_gpu(x, w, sel.gates, act_bf16=True), what="E=192 prefill, every row")
    rows = np.arange(0, 96, 6)
    assert_close(out[rows], sparse_expected(x[rows], w, sel.gates[rows], act_bf16=True),
                 what="E=192 prefill (numpy fp64 rows)")
    od = m(to_gpu(x[None, :1])).float().cpu().numpy()[0, 0]
    st = pkg.ops.decode_state(m.decode_workspace, 192)
    assert st["error"] == 0
    sel1 = oracle.select(st["logits"].numpy()[None], 0.7)
    np.testing.assert_array_equal(np.sort(st["sel_ids"].numpy()), np.nonzero(sel1.mask[0])[0])
    assert_close(od, sparse_expected(x[:1], w, sel1.gates)[0], what="E=192 decode")


def test_module_state_dict_roundtrip(pkg, c1):
    z, w, x, m = c1
    m.tau = 0.7
    ref = m(to_gpu(x[None])).float().cpu()
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    m2 = pkg.TauSparseMoE(1536, 6144, 16, 384, 0.7).to("cuda:0")
    # a reference-format state_dict stores the router in bf16; it loads by conversion
    m2.load_state_dict(sd)
    out2 = m2(to_gpu(x[None])).float().cpu()
    assert torch.equal(out2, ref)
    sd_bf = dict(sd)
    sd_bf["router"] = sd["router"].to(torch.bfloat16)
    m2.load_state_dict(sd_bf)
    out3 = m2(to_gpu(x[None])).float().cpu()
    assert out3.shape == ref.shape  # repacked from the converted router


def test_reference_reorder_data_assignment(pkg):
    """Drop-in as the reference mounts weights: physical_reorder_for_inference
    (src/openpangu_moe.py:226-244) argsorts the neuron->expert ids, assigns .data of
    W_gate/W_up [H,I], W_down [I,H] in bf16 and router [H,E] in bf16. The module
    repacks on the next forward (prefill and decode) and routes from the bf16 router."""
    H, I, E, G = 1536, 6144, 16, 384
    w = _layer(55)
    m = pkg.TauSparseMoE(H, I, E, G, 0.7).to("cuda:0")
    sort_idx = torch.argsort(torch.from_numpy(w["expert_ids"]).long(), stable=True)
    dev = torch.device("cuda:0")
    m.W_gate.data = torch.from_numpy(w["w_gate"])[sort_idx, :].t().contiguous().to(dev, torch.bfloat16)
    m.W_up.data = torch.from_numpy(w["w_up"])[sort_idx, :].t().contiguous().to(dev, torch.bfloat16)
    m.W_down.data = torch.from_numpy(w["w_down"])[:, sort_idx].t().contiguous().to(dev, torch.bfloat16)
    m.router.data = torch.from_numpy(w["w_router"]).T.contiguous().to(dev, torch.bfloat16)
    x = gi.tokens(56, 40)
    out = m(to_gpu(x[None])).float().cpu().numpy()[0]
    res = pkg.ops.route(to_gpu(x), m.router_packed, E, 0.7)
    lg = res["logits"].cpu().numpy()
    wr_bf = torch.from_numpy(w["w_router"]).to(torch.bfloat16).double().numpy()
    np.testing.assert_allclose(lg, x.astype(np.float64) @ wr_bf.T, rtol=1e-5, atol=1e-5)
    sel = oracle.select(lg, 0.7)
    np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
    assert_close(out, sparse_expected(x, w, sel.gates), what="prefill after .data mount")
    od = m(to_gpu(x[None, :1])).float().cpu().numpy()[0, 0]
    st = pkg.ops.decode_state(m.decode_workspace, E)
    sel1 = oracle.select(st["logits"].numpy()[None], 0.7)
    assert_close(od, sparse_expected(x[:1], w, sel1.gates)[0], what="decode after .data mount")


def test_module_footprint_and_partial_mount(pkg):
    """Once packed, a layer keeps the packed records + down_t (75.5 MB at H=1536, I=6144)
    and the fp32 router, not the reference-layout W_gate/W_up/W_down (56.6 MB more).
    Mounting only W_up by .data (here another layer's) repacks with W_gate and W_down
    taken from the records: the same bits as a module with all three mounted."""
    H, I, E, G = 1536, 6144, 16, 384
    dev = torch.device("cuda:0")
    w, w2 = _layer(57), _layer(59)
    m = make_module(pkg, w, 0.7)
    x = to_gpu(gi.tokens(58, 40)[None])
    ref = m(x)
    work = {"decode_workspace", "batch_workspace"}
    weights = sum(t.numel() * t.element_size() for n, t in m.named_buffers() if n not in work)
    assert weights <= 76e6, weights
    assert all(getattr(m, "_buffers")[n].numel() == 0 for n in ("W_gate", "W_up", "W_down"))
    perm = torch.argsort(torch.from_numpy(w["expert_ids"]).long(), stable=True)
    tau_gu = lambda a: torch.from_numpy(a)[perm, :].t().contiguous().to(dev, torch.bfloat16)  # noqa: E731
    up2 = tau_gu(w2["w_up"])
    m.W_up.data = up2.clone()
    out1 = m(x)
    assert all(m._buffers[n].numel() == 0 for n in ("W_gate", "W_up", "W_down"))
    full = pkg.TauSparseMoE(H, I, E, G, 0.7).to(dev)
    full.W_gate.data = tau_gu(w["w_gate"])
    full.W_up.data = up2
    full.W_down.data = torch.from_numpy(w["w_down"])[:, perm].t().contiguous().to(dev, torch.bfloat16)
    full.router.data = torch.from_numpy(w["w_router"]).t().contiguous().to(dev)
    out2 = full(x)
    assert torch.equal(out1, out2) and not torch.equal(out1, ref)
    # reading a buffer rebuilds it from the records; the next call packs nothing and drops it
    pe = m._buffers["packed_experts"]
    assert torch.equal(m.W_up, up2)
    assert torch.equal(m(x), out1)
    assert m._buffers["packed_experts"] is pe and m._buffers["W_up"].numel() == 0


def _wrapper(pkg, w, tau, G=384):
    import types
    I, H = w["w_gate"].shape
    cfg = types.SimpleNamespace(hidden_size=H, intermediate_size=I)
    ta = types.SimpleNamespace(group_size=G, tau=tau)
    m = pkg.IntegratedOpenPanguMoEMLP(cfg, ta)
    with torch.no_grad():
        m.gate_proj.weight.copy_(torch.from_numpy(w["w_gate"]))
        m.up_proj.weight.copy_(torch.from_numpy(w["w_up"]))
        m.down_proj.weight.copy_(torch.from_numpy(w["w_down"]))
        m.moelayer.mlp_router[0].weight.copy_(torch.from_numpy(w["w_router"]))
        m.moelayer.experts_masks.copy_(pkg.experts_masks_from_ids(w["expert_ids"], w["w_router"].shape[0]))
    return m.to("cuda:0").eval()


@pytest.mark.parametrize("E,G", [(16, 384), (192, 32)])
def test_model_wrapper_reorder_and_forward(pkg, E, G):
    """Model-side drop-in: reference module tree -> physical_reorder_for_inference ->
    eval forward through the kernels (E=192/G=32 with a reference cluster map)."""
    w = gi.layer_weights(70 + E, E=E)
    if E == 192:
        w["expert_ids"] = np.load(os.path.join(GOLDEN, "pangu_clusters_k32.npz"))["expert_ids"][7].astype(np.int32)
    m = _wrapper(pkg, w, 0.7, G)
    layer = torch.nn.Module()
    layer.mlp = m
    pkg.physical_reorder_for_inference([layer], 0.7)
    assert m.gate_proj is None and m.moelayer is None
    x = gi.tokens(71, 24)
    out = m(to_gpu(x[None])).float().cpu().numpy()[0]
    res = pkg.ops.route(to_gpu(x), m.tau_moe.router_packed, E, 0.7)
    sel = oracle.select(res["logits"].cpu().numpy(), 0.7)
    assert_close(out, sparse_expected(x, w, sel.gates), what=f"wrapper prefill E={E}")
    od = m(to_gpu(x[None, :1])).float().cpu().numpy()[0, 0]
    st = pkg.ops.decode_state(m.tau_moe.decode_workspace, E)
    sel1 = oracle.select(st["logits"].numpy()[None], 0.7)
    assert_close(od, sparse_expected(x[:1], w, sel1.gates)[0], what=f"wrapper decode E={E}")


def test_model_wrapper_reference_checkpoint_roundtrip(pkg):
    """A checkpoint with the reference's keys (before reorder) loads into a fresh
    wrapper and gives the same outputs after the reorder."""
    import types
    w = gi.layer_weights(73)
    m = _wrapper(pkg, w, 0.7)
    sd = {k: v.detach().cpu().clone() for k, v in m.state_dict().items()}
    cfg = types.SimpleNamespace(hidden_size=1536, intermediate_size=6144)
    m2 = pkg.IntegratedOpenPanguMoEMLP(cfg, types.SimpleNamespace(group_size=384, tau=0.7))
    m2.load_state_dict(sd)
    m2 = m2.to("cuda:0").eval()
    m.physical_reorder_for_inference(0.7)
    m2.physical_reorder_for_inference(0.7)
    x = gi.tokens(74, 16)
    a = m(to_gpu(x[None])).float().cpu()
    b = m2(to_gpu(x[None])).float().cpu()
    assert torch.equal(a, b)


def test_decoder_stack_config5_full_size(pkg):
    """BASELINE config 5 at its stated size (src/evaluation_triton.py:403-460): 26 layers
    of RMSNorm + causal attention (12 x 128) + MoE-MLP (E=16 x 384, tau 0.70), vocabulary
    153,376, a 1024-token prompt, then 128 greedy steps. Every one of the 128 graph-replayed
    steps gives the eager step's token, every eager step's logits are finite, and every
    layer's MoE-MLP call of the first two decode steps is checked against the oracle: the
    selection bit-exact on the kernel's own logits (the logits within 1e-5 of float64 on the
    layer's fp32 router), the output against the float64 sparse restatement."""
    cache = {}
    checked = []

    def hook(li, mlp, h, out):
        tm = mlp.tau_moe
        E, G, H = tm.num_experts, tm.group_size, tm.hidden_size
        if li not in cache:
            cache[li] = {"w_gate": tm.W_gate.float().t().cpu().numpy(), "w_up": tm.W_up.float().t().cpu().numpy(),
                         "w_down": tm.W_down.float().t().cpu().numpy(), "w_router": tm.router.t().cpu().numpy(),
                         "expert_ids": np.repeat(np.arange(E, dtype=np.int32), G)}
        w = cache[li]
        st = pkg.ops.decode_state(tm.decode_workspace, E)
        assert st["error"] == 0, f"layer {li}: decode error {st['error']}"
        x = h.float().reshape(1, H).cpu().numpy()
        lg = st["logits"].numpy()
        np.testing.assert_allclose(lg, (x.astype(np.float64) @ w["w_router"].T.astype(np.float64))[0],
                                   rtol=1e-5, atol=1e-5)
        sel = oracle.select(lg[None], tm.tau)
        np.testing.assert_array_equal(st["sel_ids"].numpy(), sel.ranked[0, :sel.count[0]])
        assert_close(out.float().reshape(-1).cpu().numpy(), sparse_expected(x, w, sel.gates)[0],
                     what=f"config 5 layer {li} decode MoE-MLP")
        checked.append(li)

    r = pkg.decoder_stack.run(prompt_len=1024, steps=128, layers=26, tau=0.7, verify_steps=128, moe_hook=hook,
                              moe_hook_steps=2)
    print({k: r[k] for k in ("prefill_ms", "decode_ms_per_step", "decode_moe_us_per_layer")}, flush=True)
    assert sorted(checked) == sorted(list(range(26)) * 2)
    assert r["verified_steps"] == 128 and r["graph_replays_match_eager"] and r["logits_finite"]
    assert 0.0 <= r["decode_moe_share"] < 1.0 and 0.0 < r["prefill_moe_share"] < 1.0


def test_prefill_expert_with_129_pairs(pkg):
    """Tile edges of the grouped GEMMs: an identity router (logits = x[:, :16]) routes
    each token to one chosen expert (tau 0.7, one dominant logit), expert 3 gets 129
    tokens (a full 128-row tile plus a one-row tile), the others between 1 and ~40; every
    output row against the float64 sparse restatement."""
    E, H, G, N = 16, 1536, 384, 600
    w = _layer(129)
    wr = np.zeros((E, H), np.float32)
    wr[np.arange(E), np.arange(E)] = 1.0
    w["w_router"] = wr
    m = make_module(pkg, w, 0.7)
    x = gi.tokens(130, N)
    owner = np.empty(N, np.int64)
    owner[:129] = 3
    others = [e for e in range(E) if e != 3]
    owner[129:] = np.array(others)[np.random.default_rng(5).integers(0, E - 1, N - 129)]
    x[:, :E] = -4.0
    x[np.arange(N), owner] = 4.0
    out = m(to_gpu(x[None])).float().cpu().numpy()[0]
    res = pkg.ops.route(to_gpu(x), m.router_packed, E, 0.7)
    sel = oracle.select(res["logits"].cpu().numpy(), 0.7)
    np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
    assert sel.mask[:, 3].sum() == 129 and (sel.mask.sum(1) == 1).all()
    assert_close(out, sparse_expected(x, w, sel.gates), what="129-pair expert")


@pytest.mark.parametrize("tau,want", [(0.2, [1]), (0.7, [1, 3, 0, 2, 4, 5, 6])])
def test_decode_top_expert_speculation(pkg, tau, want):
    """E = 16 decode requests the records and down rows of the largest-logit expert (as
    rank 0) before the selection is known. With an identity router the logits are
    x[:16]: experts 1 and 3 get logits one ulp apart at 1e-4 (the other 14 at -2), so
    exp(x - max) is exactly 1 for both, their probabilities tie and rank 0 is expert 1
    (lower index) although expert 3 has the larger logit: the speculative loads (expert
    3) must be replaced by expert 1's. tau=0.2 selects only expert 1; tau=0.7 selects
    expert 3 at rank 1 and five more. Twice in a row (both act banks). Output vs the fp64
    sparse reference on the oracle's selection."""
    E, H, G = 16, 1536, 384
    w = np.zeros((E, H), np.float32)
    w[np.arange(E), np.arange(E)] = 1.0
    rp = pkg.ops.pack_router(to_gpu(w), layout="linear")
    rng = np.random.default_rng(7)
    I = E * G
    wts = {"w_gate": rng.normal(0, 0.02, (I, H)).astype(np.float32),
           "w_up": rng.normal(0, 0.02, (I, H)).astype(np.float32),
           "w_down": rng.normal(0, 0.02, (H, I)).astype(np.float32),
           "w_router": w, "expert_ids": np.repeat(np.arange(E), G).astype(np.int32)}
    packed = pkg.ops.pack_experts(to_gpu(wts["w_gate"]), to_gpu(wts["w_up"]), to_gpu(wts["w_down"]), E, G,
                                  layout="linear")
    ws = pkg.ops.decode_workspace(H, E, torch.device("cuda:0"))
    x = rng.normal(0, 1, H).astype(np.float32)
    x[:E] = -2.0
    x[3] = np.float32(1e-4)
    x[1] = np.nextafter(x[3], np.float32(-np.inf))
    for _ in range(2):  # both act banks
        out = pkg.ops.moe_decode(to_gpu(x), rp, None, E, G, tau, packed, ws)
        st = pkg.ops.decode_state(ws, E)
        assert st["error"] == 0
        k = int(st["k"])
        assert st["sel_ids"].numpy()[:k].tolist() == want
        sel = oracle.select(st["logits"].numpy()[None], tau)
        assert sel.ranked[0, :sel.count[0]].tolist() == want
        sp = sparse_expected(x[None], wts, sel.gates)[0]
        assert_close(out.float().cpu().numpy().reshape(-1), sp, what=f"speculation tau={tau}")


@pytest.mark.gpu
def test_prefill_dense_form_two_passes(pkg):
    """The dense form over more tokens than one pass holds: E = 64 experts of G = 800
    neurons at H = 128 (about 100 KB of per-token buffers: 2613 tokens a pass), 2700 tokens
    in two passes on one workspace; the down GEMM's K of 51200 is split over many parts per
    tile. Selection bit-exact on the call's own logits, every row against the float64
    restatement (acts rounded to bf16), repeated calls bit-identical."""
    E, G, N, H = 64, 800, 2700, 128
    w = gi.layer_weights(43, H=H, I=E * G, E=E)
    m = make_module(pkg, w, 0.7)
    x = gi.tokens(44, N, H=H)
    xg = to_gpu(x)
    assert pkg.ops.prefill_workspace_bytes(N, H, E, G) == pkg.ops.prefill_workspace_bytes(2 * N, H, E, G)
    y, lg, mk = _abi_prefill(pkg, m, xg, E, G)
    sel = oracle.select(lg.cpu().numpy(), 0.7)
    np.testing.assert_array_equal(mk.cpu().numpy(), sel.mask)
    assert_close(y.float().cpu().numpy(), sparse_expected_gpu(x, w, sel.gates, act_bf16=True),
                 what="dense form, two passes")
    y2, _, _ = _abi_prefill(pkg, m, xg, E, G, routed=False)
    assert torch.equal(y, y2)
