"""GPU routing parity: pp_route_logits / pp_route vs the pinned oracle and fixtures.

Bit-exact bar: given identical fp32 logits, probabilities, selection mask and
gates must equal torch CPU softmax_thresholding (src/MoEBlock_origin.py:50-97)
bit for bit. Logits computed on the GPU from x are fp32 with a different
summation order than CPU sgemm, so they are compared with a tolerance and the
selection is checked bit-exactly against the oracle applied to the GPU's own logits.
"""
import os

import numpy as np
import pytest
import torch

from helpers import GOLDEN, bits, gi, oracle, to_gpu
from make_golden import TAUS

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E", [16, 24, 32, 192])
def test_route_logits_vs_golden(pkg, E):
    z = np.load(os.path.join(GOLDEN, f"routing_E{E}.npz"))
    fams = sorted({k.split("/")[0] for k in z.files if "/" in k})
    for fam in fams:
        lg = z[f"{fam}/logits"]
        for ti, tau in enumerate(TAUS):
            probs, gates, mask, count = pkg.ops.route_logits(to_gpu(lg), tau)
            torch.cuda.synchronize()
            ref_mask = np.unpackbits(z[f"{fam}/tau{ti}/mask"], axis=-1, count=E)
            np.testing.assert_array_equal(mask.cpu().numpy(), ref_mask, err_msg=f"E={E} {fam} tau={tau}")
            np.testing.assert_array_equal(bits(gates.cpu().numpy()), bits(z[f"{fam}/tau{ti}/gates"]),
                                          err_msg=f"E={E} {fam} tau={tau}")
            np.testing.assert_array_equal(count.cpu().numpy(), ref_mask.sum(-1))
            if ti == 0:
                np.testing.assert_array_equal(bits(probs.cpu().numpy()), bits(z[f"{fam}/probs"]))


@pytest.mark.parametrize("E,n", [(16, 4096), (48, 1000), (192, 500)])
def test_route_logits_random_vs_oracle(pkg, E, n):
    rng = np.random.default_rng(E * 7 + n)
    lg = (rng.standard_normal((n, E)) * rng.choice([0.3, 0.78, 2.0], (n, 1))).astype(np.float32)
    for tau in (0.5, 0.7, 0.95):
        probs, gates, mask, count = pkg.ops.route_logits(to_gpu(lg), tau)
        sel = oracle.select(lg, tau)
        np.testing.assert_array_equal(mask.cpu().numpy(), sel.mask)
        np.testing.assert_array_equal(bits(gates.cpu().numpy()), bits(sel.gates))
        np.testing.assert_array_equal(bits(probs.cpu().numpy()), bits(sel.probs))
        np.testing.assert_array_equal(count.cpu().numpy(), sel.count)


@pytest.mark.parametrize("E,xdtype", [(16, torch.float32), (16, torch.bfloat16), (192, torch.float32)])
def test_route_from_x(pkg, E, xdtype):
    H, n = 1536, 300
    rng = np.random.default_rng(E)
    x = rng.standard_normal((n, H)).astype(np.float32)
    wr = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    bias = gi.zipf_bias(E) if E == 16 else None
    xt = to_gpu(x, xdtype)
    rp = pkg.ops.pack_router(to_gpu(wr), layout="linear")
    bt = None if bias is None else to_gpu(bias)
    res = pkg.ops.route(xt, rp, E, 0.7, bias=bt, want_logits=True, want_probs=True)
    lg = res["logits"].cpu().numpy()
    xin = xt.float().cpu().numpy().astype(np.float64)
    ref = xin @ wr.astype(np.float64).T
    if bias is not None:
        ref = ref + bias
    np.testing.assert_allclose(lg, ref, rtol=1e-5, atol=1e-5)
    sel = oracle.select(lg, 0.7)
    np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
    np.testing.assert_array_equal(bits(res["gates"].cpu().numpy()), bits(sel.gates))
    np.testing.assert_array_equal(bits(res["probs"].cpu().numpy()), bits(sel.probs))
    # deterministic: a second call gives the same bits
    res2 = pkg.ops.route(xt, rp, E, 0.7, bias=bt)
    np.testing.assert_array_equal(bits(res2["logits"].cpu().numpy()), bits(lg))


def test_route_router_layouts_agree(pkg):
    H, E = 1536, 16
    rng = np.random.default_rng(3)
    wr = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    a = pkg.ops.pack_router(to_gpu(wr), layout="linear")
    b = pkg.ops.pack_router(to_gpu(np.ascontiguousarray(wr.T)), layout="tau")
    assert torch.equal(a, b)
    assert a.shape == (16, H)
    c = pkg.ops.pack_router(to_gpu(wr[:10]), layout="linear")
    assert c.shape == (16, H) and torch.all(c[10:] == 0) and torch.equal(c[:10], a[:10])


def _identity_router(pkg, E, H):
    w = np.zeros((E, H), np.float32)
    w[np.arange(E), np.arange(E)] = 1.0
    return pkg.ops.pack_router(to_gpu(w), layout="linear")


def test_route16_selection_vs_golden(pkg):
    """E = 16 path computing logits from x: with an identity router the GPU logits are
    x itself (exact: one non-zero product per sum), so the torch-CPU golden families
    pin the fused selection bit for bit (rows with non-finite logits excluded: inf * 0
    would turn them into NaN)."""
    E, H = 16, 128
    z = np.load(os.path.join(GOLDEN, "routing_E16.npz"))
    rp = _identity_router(pkg, E, H)
    fams = sorted({k.split("/")[0] for k in z.files if "/" in k})
    for fam in fams:
        lg = z[f"{fam}/logits"]
        keep = np.all(np.isfinite(lg), axis=1)
        x = np.zeros((int(keep.sum()), H), np.float32)
        x[:, :E] = lg[keep]
        for ti, tau in enumerate(TAUS):
            res = pkg.ops.route(to_gpu(x), rp, E, tau, want_logits=True, want_probs=True)
            np.testing.assert_array_equal(bits(res["logits"].cpu().numpy()), bits(lg[keep]))
            ref_mask = np.unpackbits(z[f"{fam}/tau{ti}/mask"], axis=-1, count=E)[keep]
            np.testing.assert_array_equal(res["mask"].cpu().numpy(), ref_mask, err_msg=f"{fam} tau={tau}")
            np.testing.assert_array_equal(bits(res["gates"].cpu().numpy()), bits(z[f"{fam}/tau{ti}/gates"][keep]),
                                          err_msg=f"{fam} tau={tau}")
            np.testing.assert_array_equal(res["count"].cpu().numpy(), ref_mask.sum(-1))
            if ti == 0:
                np.testing.assert_array_equal(bits(res["probs"].cpu().numpy()), bits(z[f"{fam}/probs"][keep]))


@pytest.mark.parametrize("H", [128, 640, 4096])
def test_route16_hidden_sizes(pkg, H):
    """K split over eight waves with partial chunks (H/128 = 1, 5, 32 blocks per wave)."""
    E, n = 16, 40
    rng = np.random.default_rng(H)
    x = rng.standard_normal((n, H)).astype(np.float32)
    wr = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    rp = pkg.ops.pack_router(to_gpu(wr), layout="linear")
    res = pkg.ops.route(to_gpu(x), rp, E, 0.7, want_logits=True, want_probs=True)
    lg = res["logits"].cpu().numpy()
    np.testing.assert_allclose(lg, x.astype(np.float64) @ wr.astype(np.float64).T, rtol=1e-5, atol=1e-5)
    sel = oracle.select(lg, 0.7)
    np.testing.assert_array_equal(res["mask"].cpu().numpy(), sel.mask)
    np.testing.assert_array_equal(bits(res["gates"].cpu().numpy()), bits(sel.gates))
    np.testing.assert_array_equal(bits(res["probs"].cpu().numpy()), bits(sel.probs))


@pytest.mark.parametrize("E", [16, 24, 32, 192])
def test_decode_selection_vs_golden(pkg, E):
    """The fused decode kernels' in-kernel selection, pinned the same way: identity
    router, x = golden logits, one token per call (E = 16: decode16_kernel; otherwise
    the gathered-logits path of decode_kernel with the workgroup selection)."""
    H, G = 512, 32
    z = np.load(os.path.join(GOLDEN, f"routing_E{E}.npz"))
    rp = _identity_router(pkg, E, H)
    rng = np.random.default_rng(1)
    I = E * G
    wg, wu = (rng.normal(0, 0.02, (I, H)).astype(np.float32) for _ in range(2))
    wd = rng.normal(0, 0.02, (H, I)).astype(np.float32)
    packed = pkg.ops.pack_experts(to_gpu(wg), to_gpu(wu), to_gpu(wd), E, G, layout="linear")
    ws = pkg.ops.decode_workspace(H, E, torch.device("cuda:0"))
    fams = sorted({k.split("/")[0] for k in z.files if "/" in k})
    for fam in fams:
        lg = z[f"{fam}/logits"]
        rows = [i for i in range(0, lg.shape[0], 23) if np.all(np.isfinite(lg[i]))][:20]
        for ti, tau in enumerate(TAUS):
            ref_mask = np.unpackbits(z[f"{fam}/tau{ti}/mask"], axis=-1, count=E)
            for i in rows:
                x = np.zeros(H, np.float32)
                x[:E] = lg[i]
                pkg.ops.moe_decode(to_gpu(x), rp, None, E, G, tau, packed, ws)
                st = pkg.ops.decode_state(ws, E)
                assert st["error"] == 0
                np.testing.assert_array_equal(bits(st["logits"].numpy()), bits(lg[i]))
                k = int(st["k"])
                ids = st["sel_ids"].numpy()[:k]
                np.testing.assert_array_equal(np.sort(ids), np.nonzero(ref_mask[i])[0], err_msg=f"{fam} row {i} tau={tau}")
                np.testing.assert_array_equal(bits(st["sel_gates"].numpy()[:k]), bits(z[f"{fam}/tau{ti}/gates"][i][ids]))
