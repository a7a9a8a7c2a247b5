"""CPU checks that pin the oracle (oracle/) before anything is compared against it.

* softmax / select bits against torch CPU ops (the library the reference calls,
  same torch 2.10 as requirements.txt:3) and against the committed fixtures;
* planted mistakes (fp32 cumsum, <= instead of <, wrong tie order) must be caught;
* bucket layout against a brute-force construction;
* the masked layer against torch fp32 fixtures and against its sparse form;
* the rearrangement permutation against the reference-held cluster maps.
"""
import math
import os

import numpy as np
import pytest
import torch

import inputs as gi
from make_golden import TAUS, torch_route

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
AVX512 = torch.backends.cpu.get_cpu_capability() == "AVX512"


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_expf_special_values(oracle):
    e = oracle.expf_u10(np.array([0.0, -0.0, -104.5, -200.0, -np.inf, 1.0, -1.0, 10.0], np.float32))
    assert e[0] == 1.0 and e[1] == 1.0
    assert e[2] == 0.0 and e[3] == 0.0 and e[4] == 0.0
    for v, got in zip([1.0, -1.0, 10.0], e[5:]):
        ref = np.float32(math.exp(v))
        assert abs(int(_bits(np.float32(got))[()]) - int(_bits(ref)[()])) <= 1  # u10: within 1 ulp of the true value


def test_expf_accuracy_and_monotone(oracle):
    x = np.linspace(-87.0, 0.0, 4001, dtype=np.float32)
    e = oracle.expf_u10(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    ulps = np.abs(_bits(e).astype(np.int64) - _bits(ref).astype(np.int64))
    assert ulps.max() <= 1
    assert np.all(np.diff(e.astype(np.float64)) >= 0)


@pytest.mark.skipif(not AVX512, reason="torch CPU softmax lane order is for AVX512 hosts")
@pytest.mark.parametrize("E", [1, 3, 15, 16, 17, 24, 32, 48, 100, 192, 256])
def test_softmax_bits_vs_torch(oracle, E):
    rng = np.random.default_rng(E)
    x = (rng.standard_normal((3000, E)) * rng.choice([0.1, 0.78, 3.0, 20.0], (3000, 1))).astype(np.float32)
    ref = torch.softmax(torch.from_numpy(x), -1).numpy()
    np.testing.assert_array_equal(_bits(oracle.softmax(x)), _bits(ref))


@pytest.mark.skipif(not AVX512, reason="torch CPU sigmoid/exp lane order is for AVX512 hosts")
def test_sigmoid_bits_vs_torch(oracle):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(4096) * 8).astype(np.float32)
    ref = torch.sigmoid(torch.from_numpy(x)).numpy()
    lib = oracle._load()
    got = np.array([lib.oracle_sigmoid(float(v)) for v in x], np.float32)
    np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("E", [2, 15, 16, 17, 24, 33, 64, 100, 129, 192, 256])
def test_sort_tie_order_vs_torch(oracle, E):
    """Equal probabilities: torch CPU sort order (introsort above 16) must be reproduced."""
    rng = np.random.default_rng(E + 5)
    rows = [np.zeros(E, np.float32), np.full(E, 0.25, np.float32)]
    for k in (2, 3, max(2, E // 4), max(2, E // 2)):
        for _ in range(6):
            rows.append(rng.integers(0, k, E).astype(np.float32))
    rows.append(rng.standard_normal(E).astype(np.float32))
    x = np.stack(rows)
    ref = torch.sort(torch.from_numpy(x), -1, descending=True)[1].numpy()
    np.testing.assert_array_equal(oracle.sort_desc(x), ref)


def _load_routing(E):
    return np.load(os.path.join(GOLDEN, f"routing_E{E}.npz"))


@pytest.mark.parametrize("E", [16, 24, 32, 192])
def test_select_vs_golden(oracle, E):
    z = _load_routing(E)
    fams = sorted({k.split("/")[0] for k in z.files if "/" in k})
    assert len(fams) >= 9
    for fam in fams:
        lg = z[f"{fam}/logits"]
        np.testing.assert_array_equal(_bits(oracle.softmax(lg)), _bits(z[f"{fam}/probs"]))
        for ti, tau in enumerate(TAUS):
            sel = oracle.select(lg, tau)
            mask = np.unpackbits(z[f"{fam}/tau{ti}/mask"], axis=-1, count=E)
            np.testing.assert_array_equal(sel.mask, mask, err_msg=f"{fam} tau={tau}")
            np.testing.assert_array_equal(_bits(sel.gates), _bits(z[f"{fam}/tau{ti}/gates"]),
                                          err_msg=f"{fam} tau={tau}")
            assert np.all(sel.count == mask.sum(-1))


@pytest.mark.skipif(not AVX512, reason="bitwise torch comparison needs an AVX512 host")
@pytest.mark.parametrize("tau", [0.3, 0.7, 0.95])
def test_select_vs_torch_fresh(oracle, tau):
    rng = np.random.default_rng(int(tau * 100))
    lg = (rng.standard_normal((20000, 16)) * 0.78).astype(np.float32)
    gates, probs, sel = torch_route(torch.from_numpy(lg), tau)
    got = oracle.select(lg, tau)
    np.testing.assert_array_equal(got.mask, sel.numpy().astype(np.uint8))
    np.testing.assert_array_equal(_bits(got.gates), _bits(gates.numpy()))


def _variant_select(probs, tau, cum_fp32=False, le=False, ties_high_first=False):
    """Planted-mistake variants of the selection rule (numpy, CPU only)."""
    n, E = probs.shape
    mask = np.zeros((n, E), np.uint8)
    for t in range(n):
        p = probs[t]
        idx = np.arange(E)
        order = sorted(idx, key=lambda j: (-p[j], -j if ties_high_first else j))
        acc64, acc32 = 0.0, np.float32(0)
        kept = 0
        for r, j in enumerate(order):
            if cum_fp32:
                acc32 = np.float32(acc32 + p[j])
                cum = acc32
            else:
                acc64 += float(p[j])
                cum = np.float32(acc64)
            ok = cum <= np.float32(tau) if le else cum < np.float32(tau)
            if ok:
                kept = r + 1
            else:
                break
        for j in order[:max(kept, 1)]:
            mask[t, j] = 1
    return mask


def test_planted_mistakes_are_caught(oracle):
    # ties: the "higher index first" mistake must change some selections
    z = _load_routing(16)
    probs = z["ties/probs"]
    ref_mask = np.unpackbits(z["ties/tau2/mask"], axis=-1, count=16)
    assert np.array_equal(_variant_select(probs, TAUS[2]), ref_mask)
    assert not np.array_equal(_variant_select(probs, TAUS[2], ties_high_first=True), ref_mask)
    # strict '<': rows whose cumulative sum hits tau exactly (uniform probs 1/4 -> 0.5)
    lg = np.zeros((4, 4), np.float32)
    sel = oracle.select(lg, 0.5)
    assert sel.count.tolist() == [1, 1, 1, 1]
    assert _variant_select(oracle.softmax(lg), 0.5, le=True).sum(-1).tolist() == [2, 2, 2, 2]
    # fp64-accumulated cumsum: find a row whose fp32 running sum differs from the fp64 one at
    # some rank k and put tau exactly between the two values; only the fp64 rule matches torch.
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal((2000, 16)) * 0.78).astype(np.float32)
    p = oracle.softmax(lg)
    srt = -np.sort(-p, axis=1)
    c64 = np.cumsum(srt.astype(np.float64), axis=1).astype(np.float32)
    c32 = np.cumsum(srt, axis=1, dtype=np.float32)
    rows, ks = np.nonzero(c64 != c32)
    assert rows.size > 0
    checked = 0
    for r, k in zip(rows[:50], ks[:50]):
        tau = float(max(c64[r, k], c32[r, k]))
        if k > 0 and min(c64[r, k - 1], c32[r, k - 1]) >= tau:
            continue
        row = lg[r:r + 1]
        ref = torch_route(torch.from_numpy(row), tau)[2].numpy().astype(np.uint8)
        assert np.array_equal(oracle.select(row, tau).mask, ref)
        assert not np.array_equal(_variant_select(p[r:r + 1], tau, cum_fp32=True), ref)
        checked += 1
    assert checked > 0


def _bucket_brute(mask, gates):
    n, E = mask.shape
    offs = [0]
    toks, pg = [], []
    for e in range(E):
        for t in range(n):
            if mask[t, e]:
                toks.append(t)
                pg.append(gates[t, e])
        offs.append(len(toks))
    pos = {}
    k = 0
    for e in range(E):
        for t in range(n):
            if mask[t, e]:
                pos[(t, e)] = k
                k += 1
    tp = -np.ones((n, E), np.int32)
    for t in range(n):
        s = 0
        for e in range(E):
            if mask[t, e]:
                tp[t, s] = pos[(t, e)]
                s += 1
    return np.array(offs, np.int32), np.array(toks, np.int32), np.array(pg, np.float32), tp


@pytest.mark.parametrize("n,E,p", [(1, 16, 0.4), (37, 16, 0.4), (64, 24, 0.1), (50, 192, 0.05),
                                   (20, 16, 0.0), (20, 16, 1.0)])
def test_bucket_vs_brute_force(oracle, n, E, p):
    rng = np.random.default_rng(n * 1000 + E)
    mask = (rng.random((n, E)) < p).astype(np.uint8)
    gates = rng.random((n, E)).astype(np.float32) * mask
    b = oracle.bucket(mask, gates)
    offs, toks, pg, tp = _bucket_brute(mask, gates)
    np.testing.assert_array_equal(b.offsets, offs)
    np.testing.assert_array_equal(b.token_ids, toks)
    np.testing.assert_array_equal(b.pair_gates, pg)
    np.testing.assert_array_equal(b.token_pairs, tp)


def _c1(name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    w = gi.layer_weights(int(z["seed_w"]), balanced_random=bool(z["balanced_random"]))
    x = gi.tokens(int(z["seed_x"]), int(z["n"]))
    assert gi.sha256(x, w["w_gate"], w["w_up"], w["w_down"], w["w_router"], w["expert_ids"]) == str(z["input_sha256"])
    return z, w, x


@pytest.mark.parametrize("name", ["c1_layer", "c1_layer_contig"])
def test_masked_layer_vs_torch_fixture(oracle, name):
    z, w, x = _c1(name)
    for ti, tau in enumerate(z["taus"]):
        out, sel = oracle.masked_moe_mlp(x, w["w_gate"], w["w_up"], w["w_down"], w["w_router"],
                                         w["expert_ids"], float(tau), logits=z["logits"])
        np.testing.assert_array_equal(_bits(sel.gates), _bits(z[f"tau{ti}/gates"]))
        ref = z[f"tau{ti}/out"].astype(np.float64)
        np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("name", ["c1_layer", "c1_layer_contig"])
def test_torch_masked_layer_vs_fixture(oracle, name):
    """oracle/torch_masked.py (the torch-fp32 CPU baseline) reproduces the config-1
    fixture's logits, gates (bit for bit) and outputs, and its selection equals
    oracle.select's on the same logits; with the Zipf bias its selection is
    oracle.select of (logits + bias)."""
    import torch
    from oracle.torch_masked import MaskedLayer
    z, w, x = _c1(name)
    layer = MaskedLayer(w["w_gate"], w["w_up"], w["w_down"], w["w_router"], w["expert_ids"])
    torch.set_num_threads(1)
    for ti, tau in enumerate(z["taus"]):
        score, (gates, sel) = layer.route(torch.from_numpy(x), float(tau))
        np.testing.assert_allclose(score.numpy(), z["logits"], rtol=1e-6, atol=1e-6)
        ref = oracle.select(score.numpy(), float(tau))
        np.testing.assert_array_equal(sel.numpy(), ref.mask.astype(bool))
        np.testing.assert_array_equal(_bits(gates.numpy()), _bits(ref.gates))
        if np.array_equal(score.numpy(), z["logits"]):
            np.testing.assert_array_equal(_bits(gates.numpy()), _bits(z[f"tau{ti}/gates"]))
        out = layer(torch.from_numpy(x), float(tau)).numpy()
        np.testing.assert_allclose(out, z[f"tau{ti}/out"], rtol=1e-4, atol=1e-5)
    bias = gi.zipf_bias(16)
    lb = MaskedLayer(w["w_gate"], w["w_up"], w["w_down"], w["w_router"], w["expert_ids"], bias=bias)
    score, (gates, sel) = lb.route(torch.from_numpy(x), 0.95)
    ref = oracle.select(score.numpy(), 0.95)
    np.testing.assert_array_equal(sel.numpy(), ref.mask.astype(bool))
    np.testing.assert_allclose(score.numpy(), z["logits"] + bias, rtol=1e-6, atol=1e-6)


def test_masked_equals_sparse_form(oracle):
    z, w, x = _c1("c1_layer")
    perm = oracle.pack_permutation(w["expert_ids"])
    out, sel = oracle.masked_moe_mlp(x, w["w_gate"], w["w_up"], w["w_down"], w["w_router"],
                                     w["expert_ids"], 0.7, logits=z["logits"])
    sp = oracle.sparse_moe_from_selection(x, w["w_gate"][perm], w["w_up"][perm],
                                          w["w_down"][:, perm].T, sel.gates, gi.G)
    np.testing.assert_allclose(sp, out, rtol=1e-9, atol=1e-12)
    # unselected experts truly contribute nothing: zeroing their weights changes nothing
    dead = np.nonzero(sel.mask.sum(0) == 0)[0]
    if dead.size:
        wg = w["w_gate"].copy()
        for e in dead:
            wg[w["expert_ids"] == e] = 0
        out2, _ = oracle.masked_moe_mlp(x, wg, w["w_up"], w["w_down"], w["w_router"],
                                        w["expert_ids"], 0.7, logits=z["logits"])
        np.testing.assert_allclose(out2, out, rtol=0, atol=0)


def test_bf16_rne_matches_torch(oracle):
    rng = np.random.default_rng(5)
    a = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-40, 39, 20000),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-45, 1.0 + 2.0 ** -8,
                                  1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20], np.float32)])
    # exact ties: mantissas ending in 0x8000 with an even and an odd kept bit
    ties = (np.arange(1, 2001, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    a = np.concatenate([a.astype(np.float32), ties, -ties])
    got = oracle.bf16_rne(a)
    ref = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_sparse_bf16_act_within_half_ulp(oracle):
    """The bf16-act form differs from the exact one by at most the acts' half-ulp
    rounding carried through the down projection, and does differ (the rounding is
    applied)."""
    z, w, x = _c1("c1_layer")
    perm = oracle.pack_permutation(w["expert_ids"])
    sel = oracle.select(z["logits"], 0.7)
    args = (x, w["w_gate"][perm], w["w_up"][perm], w["w_down"][:, perm].T, sel.gates, gi.G)
    ex = oracle.sparse_moe_from_selection(*args)
    rb = oracle.sparse_moe_from_selection(*args, act_bf16=True)
    # bound: sum over neurons of |act| 2^-8 |down|, per (token, column)
    Wg, Wu, Wd = (np.asarray(a, np.float64) for a in args[1:4])
    bound = np.zeros_like(ex)
    for e in range(sel.gates.shape[1]):
        t = np.nonzero(sel.gates[:, e] != 0)[0]
        if t.size == 0:
            continue
        sl = slice(e * gi.G, (e + 1) * gi.G)
        g = x[t].astype(np.float64) @ Wg[sl].T
        act = g / (1 + np.exp(-g)) * (x[t].astype(np.float64) @ Wu[sl].T) * sel.gates[t, e][:, None]
        bound[t] += np.abs(act) * 2.0 ** -8 @ np.abs(Wd[sl])
    assert np.all(np.abs(rb - ex) <= bound * (1 + 1e-9) + 1e-12)
    assert np.abs(rb - ex).max() > 0


def test_pack_permutation_vs_cluster_maps(oracle):
    ids = np.load(os.path.join(GOLDEN, "pangu_clusters_k32.npz"))["expert_ids"]
    assert ids.shape == (26, 6144)
    for layer in range(26):
        e = ids[layer].astype(np.int64)
        assert np.array_equal(np.bincount(e, minlength=192), np.full(192, 32))
        perm = oracle.pack_permutation(e)
        assert np.array_equal(np.sort(perm), np.arange(6144))
        grouped = e[perm]
        assert np.array_equal(grouped, np.repeat(np.arange(192), 32))
        # stable: original order kept inside each expert
        for g in range(0, 6144, 32):
            assert np.all(np.diff(perm[g:g + 32]) > 0)
