"""CPU restatement of the dense prefill kernels' address arithmetic (csrc/dense.hip).

For every workgroup item, K block, wave, lane and DMA instruction of dense_gemm_kernel
(both modes) and route_logits_kernel, the global element each lane's DMA reads is
computed the way the kernel computes it, and checked:
* in range of its buffer (no access outside x, act, the packed records, down_t, the router);
* at the position the fragment reads expect: the LDS image the DMAs build, read back at
  each MFMA fragment's LDS address, holds operand (row, k) of that fragment -- so a wrong
  swizzle, chunk or row mapping fails here, before any GPU run.
A planted mistake (the fragment chunk not swizzled) must fail the same check.
"""
import numpy as np
import pytest


def swz(r, BK):
    return (r >> 1) & 7 if BK == 64 else (r >> 2) & 3


def mfma32_row(q, lane):
    return (q >> 2) * 8 + (lane >> 5) * 4 + (q & 3)


def dense_gemm_dma(mode, N, H, E, G, BM=256, BK=64, NW=8, BN=256, WR=2):
    """Per (item ct/rt, kb): dict LDS byte -> (operand, global element index) of the
    8-element chunk a lane's DMA writes there, restating setup_item / issue."""
    I = E * G
    Ipad = (I + 63) // 64 * 64
    ROWB, CH = BK * 2, BK // 8
    RPI = 1024 // ROWB
    NIA, NIB = BM // (NW * RPI), BN // (NW * RPI)
    assert NIA * NW * RPI == BM and NIB * NW * RPI == BN
    WC = BN // (NW // WR)
    NJ = WC // 32
    NB2 = BN // 2
    TA = BM * ROWB
    arow = H if mode == 0 else Ipad
    n_rt = (N + BM - 1) // BM
    n_ct = (Ipad + NB2 - 1) // NB2 if mode == 0 else (H + BN - 1) // BN
    nkb = (H if mode == 0 else Ipad) // BK
    lanes = np.arange(64)
    for ct in range(n_ct):
        for rt in range(n_rt):
            t0 = rt * BM
            for kb in range(nkb):
                lds = {}
                for w in range(NW):
                    gc8 = ((lanes % CH) ^ swz(w * RPI + lanes // CH, BK)) * 8
                    for i in range(NIA):
                        r = (NW * i + w) * RPI + lanes // CH
                        tr = np.minimum(t0 + r, N - 1) - t0
                        elem = t0 * arow + kb * BK + tr * arow + gc8
                        for ln in range(64):
                            lds[(NW * i + w) * 1024 + ln * 16] = ("A", int(elem[ln]))
                    for i in range(NIB):
                        r = (NW * i + w) * RPI + lanes // CH
                        if mode == 0:
                            jb = (r % WC) >> 5
                            nl = np.minimum(ct * NB2 + (r // WC) * (WC // 2) + (jb % (NJ // 2)) * 32 + (r & 31),
                                            I - 1) - ct * NB2
                            elem = ct * NB2 * 3 * H + kb * BK + (nl * 3 + jb // (NJ // 2)) * H + gc8
                        else:
                            hl = np.minimum(ct * BN + r, H - 1) - ct * BN
                            bk_whole = BK % G == 0
                            # lane_k_all: a lane's expert / offset inside a block of whole experts
                            lane_k = (gc8 // G) * H * G + gc8 % G if bk_whole else 0
                            boff = hl * G + lane_k
                            if bk_whole and (kb + 1) * BK <= I:
                                elem = ct * BN * G + kb * (BK // G) * H * G + boff
                            else:
                                e0 = (kb * BK) // G
                                g = (kb * BK - e0 * G) + gc8
                                de = np.zeros(64, dtype=np.int64)
                                for _ in range(2):
                                    wrap = g >= G
                                    g = np.where(wrap, g - G, g)
                                    de = de + wrap
                                pad = kb * BK + gc8 >= I
                                de = np.where(pad, E - 1 - e0, de)
                                g = np.where(pad, G - 8, g)
                                elem = ct * BN * G + e0 * H * G + boff + (de * H * G + g - lane_k)
                        for ln in range(64):
                            lds[TA + (NW * i + w) * 1024 + ln * 16] = ("B", int(elem[ln]))
                yield ct, rt, kb, lds


def expected_elem(mode, operand, row, k, ct, rt, N, H, E, G, BM=256, NW=8, BN=256, WR=2):
    """Global element index of operand row `row` (tile row), K index k (first of 8): for
    the gate/up B tile, wave column wn = row // WC holds the gate rows of its WC/2 neurons
    ct * BN/2 + wn * WC/2 + ..., then their up rows."""
    I = E * G
    Ipad = (I + 63) // 64 * 64
    if operand == "A":
        t = min(rt * BM + row, N - 1)
        return t * (H if mode == 0 else Ipad) + k
    if mode == 0:
        WC = BN // (NW // WR)
        wn, within = divmod(row, WC)
        part, nb = divmod(within, WC // 2)
        n = min(ct * (BN // 2) + wn * (WC // 2) + nb, I - 1)
        return (n * 3 + part) * H + k
    h = min(ct * BN + row, H - 1)
    if k >= I:
        return None  # the pad: act is zero there, any in-range weight
    e, g = divmod(k, G)
    return (e * H + h) * G + g


def check_dense(mode, N, H, E, G, BM=256, BK=64, NW=8, BN=256, WR=2, plant=False):
    I = E * G
    Ipad = (I + 63) // 64 * 64
    ROWB, CH = BK * 2, BK // 8
    TA = BM * ROWB
    WN = NW // WR
    WM, WC = BM // WR, BN // WN
    a_size = N * (H if mode == 0 else Ipad)
    b_size = I * 3 * H if mode == 0 else E * H * G
    for ct, rt, kb, lds in dense_gemm_dma(mode, N, H, E, G, BM, BK, NW, BN, WR):
        for byte, (op, el) in lds.items():
            assert 0 <= el and el + 8 <= (a_size if op == "A" else b_size), (mode, op, ct, rt, kb, byte, el)
        for wm in range(WR):
            for wn in range(WN):
                for ks in range(BK // 16):
                    for lane in range(64):
                        r, c = lane & 31, ks * 2 + (lane >> 5)
                        pos = c if plant else c ^ swz(r, BK)
                        o = (r * CH + pos) * 16
                        k = kb * BK + ks * 16 + 8 * (lane >> 5)
                        for i in range(WM // 32):
                            row = wm * WM + 32 * i + r
                            op, el = lds[wm * WM * ROWB + o + i * 32 * ROWB]
                            assert op == "A" and el == expected_elem(mode, "A", row, k, ct, rt, N, H, E, G, BM, NW, BN, WR), \
                                (mode, "A", ct, rt, kb, wm, ks, lane, i)
                        for j in range(WC // 32):
                            row = wn * WC + 32 * j + r
                            op, el = lds[TA + wn * WC * ROWB + o + j * 32 * ROWB]
                            exp = expected_elem(mode, "B", row, k, ct, rt, N, H, E, G, BM, NW, BN, WR)
                            assert op == "B" and (exp is None or el == exp), (mode, "B", ct, rt, kb, wn, ks, lane, j)


SHAPES = [
    (300, 256, 8, 32),   # ragged N (two row tiles, the second short), I = 256
    (5, 128, 3, 32),     # I = 96: Ipad = 128 (a zero pad block in the down K), one 128-neuron tile
    (1, 384, 1, 32),     # E = 1, N = 1 (the smallest call)
    (40, 128, 2, 96),    # G = 96: expert boundaries inside K blocks
    (17, 640, 5, 160),   # H = 640 (a short last hidden tile), G = 160, I = 800 (pad 32)
]


@pytest.mark.parametrize("N,H,E,G", SHAPES)
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("BM,BK,NW,BN,WR", [(256, 64, 8, 256, 2), (256, 32, 8, 256, 2), (256, 64, 4, 256, 2),
                                          (128, 64, 8, 256, 2), (256, 32, 8, 384, 4), (128, 64, 8, 128, 4),
                                          (256, 64, 8, 192, 4), (256, 32, 4, 128, 2), (128, 32, 4, 128, 2)])
def test_dense_gemm_addresses(mode, N, H, E, G, BM, BK, NW, BN, WR):
    if mode == 0 and (BN // (NW // WR)) // 32 % 2:
        pytest.skip("gate/up needs an even number of 32-column blocks per wave")
    check_dense(mode, N, H, E, G, BM, BK, NW, BN, WR)


def test_dense_gemm_planted_swizzle_fails():
    with pytest.raises(AssertionError):
        check_dense(0, 64, 128, 4, 32, plant=True)


@pytest.mark.parametrize("BM,BN,BK,NW,WR,ST", [(256, 256, 64, 8, 2, 2), (256, 256, 32, 8, 2, 4),
                                                (256, 384, 32, 8, 4, 3), (128, 256, 64, 8, 2, 3),
                                                (256, 192, 64, 8, 4, 2), (128, 128, 64, 8, 4, 4),
                                                (256, 128, 32, 4, 2, 3), (128, 128, 32, 4, 2, 3)])
def test_dense_gemm_epilogue_bounds(BM, BN, BK, NW, WR, ST):
    """The epilogue through LDS: passes of RP rows x GB 32-column blocks; every accumulator
    lands once in the wave's share of the free stage (in range of it), the 16-byte row
    chunks read back cover what was written, global stores stay inside [N, Ipad] / [N, H]
    and the gate reads inside the staged [BM][GX] gates (GX 8 for 128-neuron column tiles, 4
    for 64-neuron ones)."""
    ROWB = BK * 2
    STAGE = BM * ROWB + BN * ROWB
    EPW = STAGE // NW
    WN = NW // WR
    WM, WC = BM // WR, BN // WN
    MI, NJ = WM // 32, WC // 32
    NB2 = BN // 2
    GX = 8 if NB2 > 64 else 4
    for (N, H, E, G) in SHAPES:
        I = E * G
        Ipad = (I + 63) // 64 * 64
        for mode in (0, 1):
            if mode == 0 and NJ % 2:
                continue  # gate/up needs gate and up blocks in pairs
            NB = NJ // 2 if mode == 0 else NJ
            GB = min(EPW // (32 * 64), NB)
            RW = GB * 64
            RP0 = EPW // RW // 32 * 32
            RP = WM  # dg_pass_rows: the largest multiple of 32 dividing WM that is <= RP0
            while RP > 32 and (RP > RP0 or WM % RP):
                RP -= 32
            assert GB >= 1 and RP >= 32 and WM % RP == 0 and RP * RW <= EPW
            cpr = RW // 16
            assert (RP * cpr) % 64 == 0
            n_rt = (N + BM - 1) // BM
            n_ct = (Ipad + NB2 - 1) // NB2 if mode == 0 else (H + BN - 1) // BN
            ncol = Ipad if mode == 0 else H
            for ct in range(n_ct):
                e_lo = ct * NB2 // G
                ne = min(E, (ct * NB2 + NB2 - 1) // G + 1) - e_lo
                assert ne <= GX
                for rt in range(n_rt):
                    for wm in range(WR):
                        for wn in range(WN):
                            t0 = rt * BM + wm * WM
                            rows_in = min(WM, max(0, N - t0))
                            c0 = ct * NB2 + wn * (WC // 2) if mode == 0 else ct * BN + wn * WC
                            cols_in = min(NB * 32, ncol - c0)
                            assert cols_in <= 0 or cols_in % 8 == 0
                            stored = set()
                            for hf in range(WM // RP):
                                for jg in range(0, NB, GB):
                                    written = set()
                                    jjs = range(jg, min(jg + GB, NB))
                                    for lane in range(64):
                                        for jj in jjs:
                                            nl = jj * 32 + (lane & 31)
                                            if mode == 0 and c0 + nl < I:
                                                assert 0 <= (c0 + nl) // G - e_lo < ne
                                            for i in range(hf * (RP // 32), (hf + 1) * (RP // 32)):
                                                for q in range(16):
                                                    rl = i * 32 + mfma32_row(q, lane)
                                                    byte = (rl - hf * RP) * RW + (nl - jg * 32) * 2
                                                    assert 0 <= byte < RP * RW and byte not in written
                                                    written.add(byte)
                                    assert len(written) == RP * 32 * len(jjs)
                                    for k in range(RP * cpr // 64):
                                        for lane in range(64):
                                            idx = lane + 64 * k
                                            rl, c = divmod(idx, cpr)
                                            rg, cg = hf * RP + rl, jg * 32 + c * 8
                                            if rg < rows_in and cg < cols_in and cg < (jg + GB) * 32:
                                                # the chunk was written in this pass, stored once, in range
                                                assert all((rl * RW + c * 16 + 2 * e) in written for e in range(8))
                                                assert (rg, cg) not in stored
                                                stored.add((rg, cg))
                                                assert t0 + rg < N and c0 + cg + 8 <= ncol
                            # every in-range output chunk of the wave tile is stored
                            assert len(stored) == rows_in * max(0, cols_in) // 8


@pytest.mark.parametrize("xs", [4, 2])
@pytest.mark.parametrize("N,H,E,TE", [(33, 384, 192, 3), (1, 128, 24, 2), (70, 1536, 40, 3), (33, 384, 192, 4),
                                      (40, 256, 200, 4)])
def test_route_logits_addresses(xs, N, H, E, TE):
    """route_logits_kernel: DMA sources in range; the LDS rows read back as the fragment
    operands x[t][k + 8g + j] and W[e][k + 8g + j]."""
    KC, TT = 128, 2
    Epad = (E + 15) // 16 * 16
    XROW, WROW = KC * xs, KC * 4
    XB = 16 * TT * XROW
    NWV = 8
    lanes = np.arange(64)
    for bx in range((N + 31) // 32):
        for by in range((E + 16 * TE - 1) // (16 * TE)):
            tok0, e0 = bx * 32, by * 16 * TE
            for c in range(H // KC):
                k0 = c * KC
                lds = {}
                for w in range(NWV):
                    for i in range(XB // (1024 * NWV)):
                        rpi = 1024 // XROW
                        cpr = XROW // 16
                        row = (NWV * i + w) * rpi + lanes // cpr
                        gc = (lanes % cpr) ^ (row & 15)
                        tok = np.minimum(tok0 + row, N - 1)
                        el = tok * H + k0 + gc * (16 // xs)
                        assert el.min() >= 0 and (el + 16 // xs).max() <= N * H
                        for ln in range(64):
                            lds[(NWV * i + w) * 1024 + ln * 16] = ("x", int(tok[ln]), int(k0 + gc[ln] * (16 // xs)))
                    for i in range(16 * TE * WROW // (1024 * NWV)):
                        row = (NWV * i + w) * 2 + lanes // 32
                        gc = (lanes % 32) ^ (row & 15)
                        er = np.minimum(e0 + row, Epad - 1)
                        el = er * H + k0 + gc * 4
                        assert el.min() >= 0 and (el + 4).max() <= Epad * H
                        for ln in range(64):
                            lds[XB + (NWV * i + w) * 1024 + ln * 16] = ("w", int(er[ln]), int(k0 + gc[ln] * 4))
                assert len(lds) == (XB + 16 * TE * WROW) // 16  # every 16-byte slot written once
                for w in range(NWV):
                    kq, ta = w & 3, w >> 2
                    for lane in range(64):
                        t_l, g = lane & 15, lane >> 4
                        r = 16 * ta + t_l
                        if xs == 4:
                            c0 = 8 * kq + 2 * g
                            for h, cc in enumerate((c0, c0 + 1)):
                                src = lds[r * XROW + ((cc ^ (r & 15)) << 4)]
                                assert src == ("x", min(tok0 + r, N - 1), k0 + 32 * kq + 8 * g + 4 * h)
                        else:
                            src = lds[r * XROW + (((4 * kq + g) ^ (r & 15)) << 4)]
                            assert src == ("x", min(tok0 + r, N - 1), k0 + 32 * kq + 8 * g)
                        for b in range(TE):
                            rb = 16 * b + t_l
                            c0 = 8 * kq + 2 * g
                            for h, cc in enumerate((c0, c0 + 1)):
                                src = lds[XB + rb * WROW + ((cc ^ (rb & 15)) << 4)]
                                assert src == ("w", min(e0 + rb, Epad - 1), k0 + 32 * kq + 8 * g + 4 * h)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("NW,BK,ST,BN,WR", [(8, 64, 2, 256, 2), (8, 32, 4, 256, 2), (4, 64, 2, 256, 2),
                                          (8, 32, 3, 384, 4), (8, 64, 2, 192, 4)])
def test_dense_split_join_lds_chunks(mode, NW, BK, ST, BN, WR):
    """The distributed join of a split tile: for every part count, the slabs partition the
    words each thread reduces; every chunk's DMA pieces stay inside the stages and inside
    the part slots (np parts of NF floats x threads); the word a thread reads back from LDS
    is its own word of part q -- the one the part's thread tid stored."""
    BM = 256
    NT = NW * 64
    WN = NW // WR
    NJ = (BN // WN) // 32
    if mode == 0 and NJ % 2:
        pytest.skip("gate/up needs gate and up blocks in pairs")
    MI = BM // WR // 32
    NF = MI * NJ * 16
    WS = NT * 8
    SLOT = NF * NT * 4
    STAGE = BM * BK * 2 + BN * BK * 2
    LDS = ST * STAGE
    NG = NF // 4 if mode == 0 else NF // 2
    HW = 2 if mode == 0 else 1
    for np_ in range(2, 9):
        upc = LDS // (np_ * HW * WS)
        assert upc >= 1
        covered = []
        for slab in range(np_):
            g_lo, g_hi = slab * NG // np_, (slab + 1) * NG // np_
            covered += list(range(g_lo, g_hi))
            for c0 in range(g_lo, g_hi, upc):
                cn = min(upc, g_hi - c0)
                total = np_ * cn * HW * (WS // 1024)
                piece = {}
                for m in range(total):
                    quarter, r1 = m % (WS // 1024), m // (WS // 1024)
                    hh, r2 = r1 % HW, r1 // HW
                    k, q = r2 % cn, r2 // cn
                    gw = c0 + k
                    b, c = gw // 8, gw % 8
                    wg = ((b // (NJ // 2)) * NJ + b % (NJ // 2) + hh * (NJ // 2)) * 8 + c if mode == 0 else gw
                    assert 0 <= wg < NF // 2 and q < np_
                    src = q * SLOT + wg * WS + quarter * 1024
                    assert src + 1024 <= np_ * SLOT
                    assert (m + 1) * 1024 <= LDS
                    piece[m] = (q, wg, quarter)
                for k in range(cn):
                    gw = c0 + k
                    b, c = gw // 8, gw % 8
                    for q in range(np_):
                        for hh in range(HW):
                            for tid in (0, 1, 63, 64, NT - 1):
                                off = ((q * cn + k) * HW + hh) * WS + tid * 8
                                m, within = divmod(off, 1024)
                                pq, pwg, quarter = piece[m]
                                # lane within // 16 of the piece loaded bytes [quarter*1024 + within ...)
                                assert pq == q and (quarter * 1024 + within) // 8 == tid
                                if mode == 0:
                                    # gate (hh = 0) / up (hh = 1) block of the same 32-row block and column block
                                    i, jj = b // (NJ // 2), b % (NJ // 2)
                                    assert pwg == (i * NJ + jj + hh * (NJ // 2)) * 8 + c
                                else:
                                    assert pwg == gw
        assert sorted(covered) == list(range(NG))
