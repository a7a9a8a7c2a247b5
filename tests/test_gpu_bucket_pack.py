"""GPU parity of bucketing (bit-exact CSR layout and tile map) and of the one-time
expert rearrangement (bit-exact bf16 layout)."""
import os

import numpy as np
import pytest
import torch

from helpers import GOLDEN, bf16_round, gi, oracle, to_gpu

pytestmark = pytest.mark.gpu


def _check_bucket(pkg, mask, gates):
    N, E = mask.shape
    bk = pkg.ops.bucket(to_gpu(mask), to_gpu(gates))
    ref = oracle.bucket(mask, gates)
    P = int(mask.astype(np.int64).sum())
    off = bk["offsets"].cpu().numpy()
    np.testing.assert_array_equal(off, ref.offsets)
    np.testing.assert_array_equal(bk["token_ids"].cpu().numpy()[:P], ref.token_ids)
    np.testing.assert_array_equal(bk["pair_gates"].cpu().numpy()[:P].view(np.uint32), ref.pair_gates.view(np.uint32))
    np.testing.assert_array_equal(bk["token_pairs"].cpu().numpy(), ref.token_pairs)
    # tile map: closed form, tile_m = 128
    tm = pkg.ops.gemm_tile_m()
    meta = bk["meta"].cpu().numpy()
    exp = []
    for e in range(E):
        c = ref.offsets[e + 1] - ref.offsets[e]
        for i in range((c + tm - 1) // tm):
            exp.append((e, ref.offsets[e] + i * tm, min(tm, c - i * tm), 0))
    assert meta[0] == len(exp) and meta[1] == P
    assert len(exp) <= bk["max_tiles"]
    if exp:
        np.testing.assert_array_equal(bk["tiles"].cpu().numpy()[:len(exp)], np.array(exp, np.int32))


@pytest.mark.parametrize("N,E,p", [(1, 16, 0.4), (37, 16, 0.4), (256, 16, 0.38), (300, 16, 0.9),
                                   (2048, 16, 0.38), (513, 192, 0.05), (64, 24, 0.0), (64, 16, 1.0),
                                   (100, 40, 0.3), (4096, 64, 0.1), (4097, 16, 0.3), (5000, 16, 0.4),
                                   (0, 16, 0.5), (3000, 192, 0.02)])
def test_bucket_random_vs_oracle(pkg, N, E, p):
    rng = np.random.default_rng(N * 31 + E)
    mask = (rng.random((N, E)) < p).astype(np.uint8)
    gates = (rng.random((N, E)).astype(np.float32) * mask).astype(np.float32)
    _check_bucket(pkg, mask, gates)


def test_bucket_from_routing(pkg):
    rng = np.random.default_rng(11)
    lg = ((rng.standard_normal((2048, 16)) * 0.78) + gi.zipf_bias(16)[None]).astype(np.float32)
    probs, gates, mask, count = pkg.ops.route_logits(to_gpu(lg), 0.95)
    _check_bucket(pkg, mask.cpu().numpy(), gates.cpu().numpy())


def _expected_packed(wg, wu, wd, perm, E, G):
    """Packed layout restated in numpy: rows [I][3][H] then down_t [E][H][G]."""
    g = bf16_round(wg)[perm]
    u = bf16_round(wu)[perm]
    d = bf16_round(wd)[:, perm].T  # [I, H]
    I, H = g.shape
    rows = np.stack([g, u, d], axis=1).reshape(-1)
    down_t = d.reshape(E, G, H).transpose(0, 2, 1).reshape(-1)
    return np.concatenate([rows, down_t])


@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_pack_linear_layout(pkg, src):
    H, E, G = 256, 16, 64
    I = E * G
    rng = np.random.default_rng(5)
    wg, wu = (rng.normal(0, 0.02, (I, H)).astype(np.float32) for _ in range(2))
    wd = rng.normal(0, 0.02, (H, I)).astype(np.float32)
    ids = rng.permutation(np.repeat(np.arange(E), G))
    perm = oracle.pack_permutation(ids)
    dt = torch.float32 if src == "f32" else torch.bfloat16
    out = pkg.ops.pack_experts(to_gpu(wg, dt), to_gpu(wu, dt), to_gpu(wd, dt), E, G,
                               perm=to_gpu(perm.astype(np.int32)), layout="linear")
    got = out.float().cpu().numpy()
    np.testing.assert_array_equal(got, _expected_packed(wg, wu, wd, perm, E, G))


def test_pack_tau_layout_equals_linear(pkg):
    H, E, G = 128, 8, 32
    I = E * G
    rng = np.random.default_rng(9)
    wg, wu = (rng.normal(0, 0.02, (I, H)).astype(np.float32) for _ in range(2))
    wd = rng.normal(0, 0.02, (H, I)).astype(np.float32)
    a = pkg.ops.pack_experts(to_gpu(wg), to_gpu(wu), to_gpu(wd), E, G, layout="linear")
    b = pkg.ops.pack_experts(to_gpu(np.ascontiguousarray(wg.T), torch.bfloat16),
                             to_gpu(np.ascontiguousarray(wu.T), torch.bfloat16),
                             to_gpu(np.ascontiguousarray(wd.T), torch.bfloat16), E, G, layout="tau")
    assert torch.equal(a, b)


def test_pack_with_reference_cluster_maps(pkg):
    """E=192, G=32 partition from the reference's own cluster files (layer 0), H=128."""
    ids = np.load(os.path.join(GOLDEN, "pangu_clusters_k32.npz"))["expert_ids"][0].astype(np.int64)
    E, G, H = 192, 32, 128
    I = E * G
    rng = np.random.default_rng(1)
    wg, wu = (rng.normal(0, 0.02, (I, H)).astype(np.float32) for _ in range(2))
    wd = rng.normal(0, 0.02, (H, I)).astype(np.float32)
    perm = oracle.pack_permutation(ids)
    m = None
    out = pkg.ops.pack_experts(to_gpu(wg), to_gpu(wu), to_gpu(wd), E, G, perm=to_gpu(perm.astype(np.int32)),
                               layout="linear")
    np.testing.assert_array_equal(out.float().cpu().numpy(), _expected_packed(wg, wu, wd, perm, E, G))
    # every expert's 32 records come from neurons the cluster map assigns to it
    rows = out.float().cpu().numpy()[:I * 3 * H].reshape(I, 3, H)
    src = bf16_round(wg)
    for e in (0, 57, 191):
        owned = np.nonzero(ids == e)[0]
        np.testing.assert_array_equal(rows[e * G:(e + 1) * G, 0], src[owned])
    del m


def test_pack_bf16_rounding_bits(pkg):
    """fp32 -> bf16 conversion of the packer, bit for bit against torch's CPU
    .to(bfloat16) (round to nearest even): halfway ties both ways, denormals, the
    overflow boundary, infinities, random bit patterns; NaN stays NaN."""
    H, E, G = 128, 2, 32
    I = E * G
    rng = np.random.default_rng(11)
    bits_u = rng.integers(0, 2**32, size=(I, H), dtype=np.uint64).astype(np.uint32)
    special = np.array([0x00000000, 0x80000000, 0x3f800000, 0xbf800000, 0x00000001, 0x80000001, 0x007fffff,
                        0x00800000, 0x00008000, 0x00018000, 0x00017fff, 0x00018001, 0x3f808000, 0x3f818000,
                        0x3f807fff, 0x3f818001, 0x7f7fffff, 0xff7fffff, 0x7f7f8000, 0x7f7f7fff, 0x7f800000,
                        0xff800000, 0x7fc00000, 0x7f800001, 0xffffffff, 0x4b3fffff], dtype=np.uint32)
    bits_u[0, :special.size] = special
    wg = bits_u.view(np.float32)
    wu = np.zeros((I, H), np.float32)
    wd = np.zeros((H, I), np.float32)
    out = pkg.ops.pack_experts(to_gpu(wg), to_gpu(wu), to_gpu(wd), E, G, layout="linear")
    got = out[: I * 3 * H].view(I, 3, H)[:, 0, :].cpu().view(torch.int16).numpy().view(np.uint16)
    want = torch.from_numpy(wg).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan_in = np.isnan(wg)
    np.testing.assert_array_equal(got[~nan_in], want[~nan_in])
    g_exp = (got[nan_in] >> 7) & 0xFF
    g_man = got[nan_in] & 0x7F
    assert np.all(g_exp == 0xFF) and np.all(g_man != 0), "NaN input must stay NaN"
