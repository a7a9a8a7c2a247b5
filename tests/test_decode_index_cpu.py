"""CPU restatement of decode2p_kernel's down-row DMA addressing (csrc/decode.hip, dma_rows).

The kernel DMAs the rows [r0, r1) of down_t for the k selected experts into LDS as one flat
list of 16-byte chunks: rank s's chunk c (row c // cpr, 8 neurons 8 * (c % cpr)) at LDS chunk
s * pp + c with pp = per + 1 (per = rows * cpr; the chunk after each rank is padding). Lane
`lane` of DMA instruction (round c0, slot j) writes LDS chunk c0 + 64 j + lane and derives
its rank with a multiply-high by a magic number instead of a division. Checked here:
* the LDS image the DMAs build, read back where the row sums read (rank s, row wr, chunk cc
  at LDS chunk s * pp + wr * cpr + cc), holds down_t[e_s][r0 + wr][8 cc .. 8 cc + 8];
* every source chunk lies inside down_t and every written LDS chunk inside the dynamic LDS
  the host launches with;
* the multiply-high division equals floor division over every (c, pp) the kernel can form;
* a planted mistake (the magic number without its + 1) fails the image check.
The batch kernel's down-row DMAs (decodeb_kernel, dma_rows: rows of one slice of union
neurons, spread over the eight waves) are checked the same way.
"""
import numpy as np
import pytest

DEC2_DOWN_LDS = 96 * 1024


def host_rp(E, G, H, W):
    """Rows per pass and dynamic LDS bytes, as the host computes them for decode2p."""
    nh = (H + W - 1) // W
    rp = min(8, nh)
    while rp > 1 and ((E * (rp * (G // 8) + 1) + 63) // 64 * 64) * 16 > DEC2_DOWN_LDS:
        rp -= 1
    smem = ((E * (rp * (G // 8) + 1) + 63) // 64 * 64) * 16
    return rp, smem


def magic_of(pp, plus_one=True):
    return ((0xFFFFFFFF // pp) + (1 if plus_one else 0)) & 0xFFFFFFFF


def dma_image(k, L, r0, r1, H, G, plus_one=True):
    """LDS chunk -> source element index in down_t ([E][H][G] bf16), restating dma_rows."""
    cpr = G >> 3
    per = (r1 - r0) * cpr
    pp = per + 1
    nq = k * pp
    magic = magic_of(pp, plus_one)
    img = {}
    for c0 in range(0, nq, 256):
        for j in range(4):
            if c0 + 64 * j >= nq:
                continue
            for lane in range(64):
                c = min(c0 + 64 * j + lane, nq - 1)
                s = (c * magic) >> 32
                rq = min(c - s * pp, per - 1)
                assert s < k, "rank beyond the selection (L_s read out of range)"
                e = L[s]
                src = (e * H + r0) * G + 8 * rq  # element index of the 16-byte chunk
                img[c0 + 64 * j + lane] = src
    return img


@pytest.mark.parametrize("E,G,H,W,k", [(192, 32, 1536, 256, 75), (192, 32, 1536, 256, 192), (96, 64, 1024, 256, 40),
                                       (24, 96, 512, 24, 7), (32, 256, 2048, 64, 32), (16, 512, 4096, 200, 3)])
def test_dma_image_matches_row_reads(E, G, H, W, k):
    rng = np.random.default_rng(E * 7 + G + k)
    L = list(rng.permutation(E)[:k])
    rp, smem = host_rp(E, G, H, W)
    cpr = G >> 3
    for b in (0, 1, W // 2, W - 1):
        q, rem = divmod(H, W)  # pp_split
        h0 = b * q + min(b, rem)
        h1 = h0 + q + (1 if b < rem else 0)
        for r0 in range(h0, h1, rp):
            r1 = min(h1, r0 + rp)
            img = dma_image(k, L, r0, r1, H, G)
            per = (r1 - r0) * cpr
            assert max(img) * 16 + 16 <= smem, "DMA writes beyond the dynamic LDS"
            assert all(0 <= v and v + 8 <= E * H * G for v in img.values()), "DMA source outside down_t"
            for s in range(k):
                for wr in range(r1 - r0):
                    for cc in range(cpr):
                        got = img[s * (per + 1) + wr * cpr + cc]
                        assert got == (L[s] * H + r0 + wr) * G + 8 * cc, (s, wr, cc)


def test_planted_magic_without_plus_one_fails():
    E, G, H, W, k = 192, 32, 1536, 256, 75
    L = list(range(0, 2 * k, 2))
    r0, r1 = 0, 6
    cpr, per = G >> 3, 6 * (G >> 3)
    img = dma_image(k, L, r0, r1, H, G, plus_one=False)
    bad = sum(img[s * (per + 1) + wr * cpr + cc] != (L[s] * H + r0 + wr) * G + 8 * cc
              for s in range(k) for wr in range(r1 - r0) for cc in range(cpr))
    assert bad > 0


def test_multiply_high_division_exact_over_kernel_range():
    # c < 6144 + 64 (the LDS chunks of one pass plus one instruction), 5 <= pp <= 8 * 64 + 1
    c = np.arange(0, 6144 + 64, dtype=np.uint64)
    for pp in range(5, 8 * 64 + 2):
        m = np.uint64(magic_of(pp))
        assert np.array_equal((c * m) >> np.uint64(32), c // np.uint64(pp)), pp


def batch_dma_image(nr, cpr, a0, G, H, p0, ul, part, nparts):
    """decodeb_kernel's dma_rows (csrc/decode.hip): LDS chunk -> source element of down_t, one
    wave's share (instructions part, part + nparts, ...), four instructions per round."""
    mag_c = magic_of(cpr + 1)
    mag_g = magic_of(G)
    total, step = nr * (cpr + 1), 64 * nparts
    img = {}
    for i00 in range(64 * part, total, 4 * step):
        for j in range(4):
            if i00 + j * step >= total:
                continue
            for lane in range(64):
                f = min(i00 + j * step + lane, total - 1)
                rho = (f * mag_c) >> 32
                c = min(f - rho * (cpr + 1), cpr - 1)
                q = a0 + 8 * c
                ue = (q * mag_g) >> 32
                assert ue < len(ul), "union expert index out of range"
                img[i00 + j * step + lane] = ul[ue] * H * G + (p0 + rho) * G + q - ue * G
    return img


@pytest.mark.parametrize("G,nu,slice_", [(384, 16, 0), (384, 16, 15), (384, 11, 7), (256, 16, 3), (512, 5, 2), (96, 9, 4)])
def test_batch_dma_image(G, nu, slice_):
    """Every wave's share together covers each staged row chunk with down_t[e][p0 + rho] at the
    slice's union neurons; sources inside down_t; writes inside the kernel's LDS."""
    H, E, NW, DECB_SMEM = 1536, 16, 8, 8 * 3 * 2 * 24 * 128
    T = nu * G
    ul = list(np.random.default_rng(G + nu).permutation(E)[:nu])
    nblk = T // 16
    q, rem = divmod(nblk, 16)  # pp_split over the 16 slices
    sb0 = slice_ * q + min(slice_, rem)
    sb1 = sb0 + q + (1 if slice_ < rem else 0)
    a0, nk = 16 * sb0, 16 * (sb1 - sb0)
    cpr = nk // 8
    if cpr == 0:
        return
    rows = 96
    while rows > 1 and ((rows * (G // 8 + 1) + 63) // 64 * 64) * 16 > DECB_SMEM:
        rows -= 1
    p0 = 8 * 37
    img = {}
    for wv in range(NW):
        part = batch_dma_image(rows, cpr, a0, G, H, p0, ul, wv, NW)
        assert not set(part) & set(img), "two waves write one LDS chunk"
        img.update(part)
    assert max(img) * 16 + 16 <= DECB_SMEM
    assert all(0 <= v and v + 8 <= E * H * G for v in img.values())
    for rho in range(rows):
        for c in range(cpr):
            qn = a0 + 8 * c
            assert img[rho * (cpr + 1) + c] == ul[qn // G] * H * G + (p0 + rho) * G + qn % G, (rho, c)
