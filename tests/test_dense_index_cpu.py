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


def dense_gemm_dma(mode, N, H, E, G, BM=256, BK=64, NW=8):
    """Per (item ct/rt, kb): dict LDS byte -> (operand, global element index) of the
    8-element chunk a lane's DMA writes there, restating setup_item / issue."""
    I = E * G
    Ipad = (I + 63) // 64 * 64
    ROWB, CH = BK * 2, BK // 8
    RPI = 1024 // ROWB
    NIA, NIB = BM // (NW * RPI), 256 // (NW * RPI)
    WC = 256 // (NW // 2)
    NJ = WC // 32
    TA = BM * ROWB
    arow = H if mode == 0 else Ipad
    n_rt = (N + BM - 1) // BM
    n_ct = (Ipad + 127) // 128 if mode == 0 else (H + 255) // 256
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
                            nl = np.minimum(ct * 128 + (r // WC) * (WC // 2) + (jb % (NJ // 2)) * 32 + (r & 31),
                                            I - 1) - ct * 128
                            elem = ct * 128 * 3 * H + kb * BK + (nl * 3 + jb // (NJ // 2)) * H + gc8
                        else:
                            hl = np.minimum(ct * 256 + r, H - 1) - ct * 256
                            bk_whole = BK % G == 0
                            # lane_k_all: a lane's expert / offset inside a block of whole experts
                            lane_k = (gc8 // G) * H * G + gc8 % G if bk_whole else 0
                            boff = hl * G + lane_k
                            if bk_whole and (kb + 1) * BK <= I:
                                elem = ct * 256 * G + kb * (BK // G) * H * G + boff
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
                                elem = ct * 256 * G + e0 * H * G + boff + (de * H * G + g - lane_k)
                        for ln in range(64):
                            lds[TA + (NW * i + w) * 1024 + ln * 16] = ("B", int(elem[ln]))
                yield ct, rt, kb, lds


def expected_elem(mode, operand, row, k, ct, rt, N, H, E, G, BM=256, NW=8):
    """Global element index of operand row `row` (tile row), K index k (first of 8): for
    the gate/up B tile, wave column wn = row // WC holds the gate rows of its WC/2 neurons
    ct * 128 + wn * WC/2 + ..., then their up rows."""
    I = E * G
    Ipad = (I + 63) // 64 * 64
    if operand == "A":
        t = min(rt * BM + row, N - 1)
        return t * (H if mode == 0 else Ipad) + k
    if mode == 0:
        WC = 256 // (NW // 2)
        wn, within = divmod(row, WC)
        part, nb = divmod(within, WC // 2)
        n = min(ct * 128 + wn * (WC // 2) + nb, I - 1)
        return (n * 3 + part) * H + k
    h = min(ct * 256 + row, H - 1)
    if k >= I:
        return None  # the pad: act is zero there, any in-range weight
    e, g = divmod(k, G)
    return (e * H + h) * G + g


def check_dense(mode, N, H, E, G, BM=256, BK=64, NW=8, plant=False):
    I = E * G
    Ipad = (I + 63) // 64 * 64
    ROWB, CH = BK * 2, BK // 8
    TA = BM * ROWB
    WN = NW // 2
    WC = 256 // WN
    a_size = N * (H if mode == 0 else Ipad)
    b_size = I * 3 * H if mode == 0 else E * H * G
    for ct, rt, kb, lds in dense_gemm_dma(mode, N, H, E, G, BM, BK, NW):
        for byte, (op, el) in lds.items():
            assert 0 <= el and el + 8 <= (a_size if op == "A" else b_size), (mode, op, ct, rt, kb, byte, el)
        for wm in range(2):
            for wn in range(WN):
                for ks in range(BK // 16):
                    for lane in range(64):
                        r, c = lane & 31, ks * 2 + (lane >> 5)
                        pos = c if plant else c ^ swz(r, BK)
                        o = (r * CH + pos) * 16
                        k = kb * BK + ks * 16 + 8 * (lane >> 5)
                        for i in range(BM // 64):
                            row = wm * (BM // 2) + 32 * i + r
                            op, el = lds[wm * (BM // 2) * ROWB + o + i * 32 * ROWB]
                            assert op == "A" and el == expected_elem(mode, "A", row, k, ct, rt, N, H, E, G, BM, NW), \
                                (mode, "A", ct, rt, kb, wm, ks, lane, i)
                        for j in range(WC // 32):
                            row = wn * WC + 32 * j + r
                            op, el = lds[TA + wn * WC * ROWB + o + j * 32 * ROWB]
                            exp = expected_elem(mode, "B", row, k, ct, rt, N, H, E, G, BM, NW)
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
@pytest.mark.parametrize("BM,BK,NW", [(256, 64, 8), (256, 32, 8), (256, 64, 4), (128, 64, 8)])
def test_dense_gemm_addresses(mode, N, H, E, G, BM, BK, NW):
    check_dense(mode, N, H, E, G, BM, BK, NW)


def test_dense_gemm_planted_swizzle_fails():
    with pytest.raises(AssertionError):
        check_dense(0, 64, 128, 4, 32, plant=True)


@pytest.mark.parametrize("BM,BK,NW,ST", [(256, 64, 8, 2), (256, 32, 8, 4)])
def test_dense_gemm_epilogue_bounds(BM, BK, NW, ST):
    """The epilogue through LDS: every accumulator lands once in the wave's share of the
    free stage (in range of it), the 16-byte row chunks read back cover exactly what was
    written, global stores stay inside [N, Ipad] / [N, H] and the gate reads inside the
    staged [BM][8] gates."""
    DG_GX = 8
    ROWB = BK * 2
    STAGE = BM * ROWB + 256 * ROWB
    EPW = STAGE // NW
    WN = NW // 2
    WC = 256 // WN
    MI, NJ = BM // 64, WC // 32
    for (N, H, E, G) in SHAPES:
        I = E * G
        Ipad = (I + 63) // 64 * 64
        for mode in (0, 1):
            RW = (WC // 2) * 2 if mode == 0 else WC * 2
            HR = min(EPW // RW, BM // 2)
            assert HR % 32 == 0 and (BM // 2) % HR == 0 and HR * RW <= EPW
            n_rt = (N + BM - 1) // BM
            n_ct = (Ipad + 127) // 128 if mode == 0 else (H + 255) // 256
            for ct in range(n_ct):
                e_lo = ct * 128 // G
                ne = min(E, (ct * 128 + 127) // G + 1) - e_lo
                assert ne <= DG_GX
                for rt in range(n_rt):
                    for wm in range(2):
                        for wn in range(WN):
                            t0 = rt * BM + wm * (BM // 2)
                            rows_in = min(BM // 2, max(0, N - t0))
                            if mode == 0:
                                n0 = ct * 128 + wn * (WC // 2)
                                cols_in = min(WC // 2, Ipad - n0)
                                ncols = WC // 2
                            else:
                                n0 = ct * 256 + wn * WC
                                cols_in = min(WC, H - n0)
                                ncols = WC
                            assert cols_in % 8 == 0
                            for hf in range((BM // 2) // HR):
                                written = set()
                                for lane in range(64):
                                    for i in range(hf * (HR // 32), (hf + 1) * (HR // 32)):
                                        for jb in range(NJ // 2 if mode == 0 else NJ):
                                            col = jb * 32 + (lane & 31)
                                            if mode == 0 and n0 + col < I:
                                                assert 0 <= (n0 + col) // G - e_lo < ne
                                            for q in range(16):
                                                rl = i * 32 + mfma32_row(q, lane)
                                                byte = (rl - hf * HR) * RW + col * 2
                                                assert 0 <= byte < HR * RW and byte not in written
                                                written.add(byte)
                                assert len(written) == HR * ncols
                                cpr = RW // 16
                                assert (HR * cpr) % 64 == 0
                                for k in range(HR * cpr // 64):
                                    for lane in range(64):
                                        idx = lane + 64 * k
                                        rl, c = divmod(idx, cpr)
                                        rg = hf * HR + rl
                                        if rg < rows_in and c * 8 < cols_in:
                                            assert t0 + rg < N
                                            assert n0 + c * 8 + 8 <= (Ipad if mode == 0 else H)


@pytest.mark.parametrize("xs", [4, 2])
@pytest.mark.parametrize("N,H,E", [(33, 384, 192), (1, 128, 24), (70, 1536, 40)])
def test_route_logits_addresses(xs, N, H, E):
    """route_logits_kernel: DMA sources in range; the LDS rows read back as the fragment
    operands x[t][k + 8g + j] and W[e][k + 8g + j]."""
    KC, TT = 128, 2
    TE = 1 if E <= 16 else 2 if E <= 32 else 3
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
@pytest.mark.parametrize("NW,BK,ST", [(8, 64, 2), (8, 32, 4), (4, 64, 2)])
def test_dense_split_join_lds_chunks(mode, NW, BK, ST):
    """The distributed join of a split tile: for every part count, the slabs partition the
    words each thread reduces; every chunk's DMA pieces stay inside the stages and inside
    the part slots (np parts of NF floats x threads); the word a thread reads back from LDS
    is its own word of part q -- the one the part's thread tid stored."""
    BM = 256
    NT = NW * 64
    WN = NW // 2
    NJ = (256 // WN) // 32
    MI = BM // 64
    NF = MI * NJ * 16
    WS = NT * 8
    SLOT = NF * NT * 4
    STAGE = BM * BK * 2 + 256 * BK * 2
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
