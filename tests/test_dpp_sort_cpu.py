"""CPU restatement of the workgroup rank computation of the E > 16 decode selection
(select_one_token_wg in csrc/pp_common.h; above E = 128): per 64-lane wave a bitonic sort of 64-bit
keys whose partner exchanges use DPP lane moves for xor 1, 2, 4 and 8 and permlane swaps
for 16 and 32, then each key's rank = its place in its run + the number of smaller keys in
every other run (binary search). No GPU.

The DPP lane maps are written from the ISA definitions of the two controls the kernel
uses (lane i of the result reads source lane src[i]):
* quad_perm [p0, p1, p2, p3]: src[i] = 4 * (i // 4) + p[i % 4];
* row_half_mirror: src[i] = 8 * (i // 8) + 7 - i % 8;
* row_ror:n: inside each 16-lane row, the row rotated by n lanes. The direction is the
  thing that once went wrong (a two-rotation xor 4 that assumed the opposite direction
  lost keys), so every check below runs under BOTH directions, and the kernel only uses
  row_ror:8, which is direction-free. xor 4 is now quad_perm [3,2,1,0] followed by
  row_half_mirror: two fixed involutions, no direction involved.

Checks: each DPP exchange the kernel uses is the permutation lane i <-> lane i ^ j
(an involution pairing i with i ^ j) under either rotation direction; row_ror:4 is not
i ^ 4 under either direction (why the kernel builds xor 4 from the two mirrors); the whole
rank computation equals a plain sort of the keys on random, tie-heavy, all-equal and NaN
rows for E = 17 .. 256 (a permutation of 0 .. E-1 with no lost or duplicated key).
"""
import numpy as np
import pytest

WAVE = 64


def quad_perm(p):
    return np.array([4 * (i // 4) + p[i % 4] for i in range(WAVE)])


def row_ror(n, direction):
    # direction +1: lane i reads lane i + n of its row; -1: lane i - n
    return np.array([16 * (i // 16) + (i % 16 + direction * n) % 16 for i in range(WAVE)])


XOR1 = [1, 0, 3, 2]  # PP_DPP_XOR1 = 0xB1: quad_perm fields 1,0,3,2 (2 bits each, lane 0 first)
XOR2 = [2, 3, 0, 1]  # PP_DPP_XOR2 = 0x4E
QREV = [3, 2, 1, 0]  # PP_DPP_QREV = 0x1B


def half_mirror():
    return np.array([8 * (i // 8) + 7 - i % 8 for i in range(WAVE)])


def then(first, second):
    """Source lanes of DPP move `second` applied to the result of `first`: lane i of
    the result reads lane second[i] of the intermediate, which holds lane first[second[i]]."""
    return first[second]


def _decode_quad_perm(ctrl):
    return [(ctrl >> (2 * k)) & 3 for k in range(4)]


def permlane_swap(rows):
    """v_permlane16_swap (rows = 16) / v_permlane32_swap (rows = 32) of a register with
    itself, as source lanes of the two results (ISA: the odd rows / the upper half of the
    first operand are swapped with the even rows / the lower half of the second): returns
    (src of result 0, src of result 1)."""
    lanes = np.arange(WAVE)
    blk = lanes // rows
    r0 = np.where(blk % 2 == 1, lanes - rows, lanes)  # odd blocks take the even block below
    r1 = np.where(blk % 2 == 0, lanes + rows, lanes)  # even blocks take the odd block above
    return r0, r1


def pl_xor(j):
    """pl_xor16 / pl_xor32 (csrc/pp_common.h): a lane takes result 0 in odd blocks of j
    lanes, result 1 in even ones."""
    r0, r1 = permlane_swap(j)
    lanes = np.arange(WAVE)
    return np.where((lanes // j) % 2 == 1, r0, r1)


def lane_maps(direction):
    """Source lane of every lane for the partner exchange of distance j, as the kernel
    does it (key_xor): DPP for j = 1, 2, 4, 8, permlane swaps for 16 and 32."""
    m = {1: quad_perm(XOR1), 2: quad_perm(XOR2), 4: then(quad_perm(QREV), half_mirror()),
         8: row_ror(8, direction)}
    for j in (16, 32):
        m[j] = pl_xor(j)
    return m


def test_permlane_selection_is_xor():
    """A planted mistake (the two results taken the other way round) must not pair i with
    i ^ j: the selection in pl_xor16 / pl_xor32 is what makes the swap an xor."""
    lanes = np.arange(WAVE)
    for j in (16, 32):
        r0, r1 = permlane_swap(j)
        wrong = np.where((lanes // j) % 2 == 1, r1, r0)
        assert not np.array_equal(wrong, lanes ^ j)
        np.testing.assert_array_equal(pl_xor(j), lanes ^ j)


def test_dpp_controls_encode_the_quad_perms():
    assert _decode_quad_perm(0xB1) == XOR1
    assert _decode_quad_perm(0x4E) == XOR2
    assert _decode_quad_perm(0x1B) == QREV


@pytest.mark.parametrize("direction", [+1, -1])
def test_dpp_exchanges_pair_lane_i_with_i_xor_j(direction):
    lanes = np.arange(WAVE)
    for j, src in lane_maps(direction).items():
        np.testing.assert_array_equal(src, lanes ^ j, err_msg=f"j={j}")
        np.testing.assert_array_equal(src[src], lanes)  # an involution: a pairing


@pytest.mark.parametrize("direction", [+1, -1])
def test_row_ror4_is_not_xor4(direction):
    assert not np.array_equal(row_ror(4, direction), np.arange(WAVE) ^ 4)


def sel_key(p, j):
    """The kernel's 64-bit rank key: ~bits(p) << 32 | j, NaN mapped to all ones first."""
    b = p.view(np.uint32).astype(np.uint64)
    b = np.where(np.isnan(p), np.uint64(0xFFFFFFFF), b)
    return ((~b & np.uint64(0xFFFFFFFF)) << np.uint64(32)) | j.astype(np.uint64)


def wg_ranks(keys, maps):
    """select_one_token_wg's rank step on E keys (E <= 256): per wave a bitonic sort with
    the given exchange maps, then ranks by binary search over the other waves' runs.
    Returns order[rank] = expert id (-1 where no key landed) and the collision flag."""
    E = keys.size
    nwk = (E + WAVE - 1) // WAVE
    allk = np.full(nwk * WAVE, np.uint64(0xFFFFFFFFFFFFFFFF))
    allk[:E] = keys
    runs = allk.reshape(nwk, WAVE).copy()
    lanes = np.arange(WAVE)
    for w in range(nwk):
        key = runs[w]
        k2 = 2
        while k2 <= WAVE:
            j = k2 >> 1
            while j > 0:
                o = key[maps[j]]
                keep_min = ((lanes & j) == 0) == ((lanes & k2) == 0)
                key = np.where(keep_min, np.minimum(o, key), np.maximum(o, key))
                j >>= 1
            k2 <<= 1
        runs[w] = key
    order = np.full(E, -1, np.int64)
    writes = np.zeros(E, np.int64)
    for w in range(nwk):
        for lane in range(WAVE):
            key = runs[w, lane]
            if key == np.uint64(0xFFFFFFFFFFFFFFFF):
                continue
            rank = lane
            for w2 in range(nwk):
                if w2 == w:
                    continue
                run = runs[w2]
                lo = 0
                step = 32
                while step >= 1:
                    lo += step if run[lo + step - 1] < key else 0
                    step >>= 1
                lo += 1 if (lo == 63 and run[63] < key) else 0
                rank += lo
            idx = int(key & np.uint64(0xFFFFFFFF))
            if rank < E and idx < E:
                order[rank] = idx
                writes[rank] += 1
    return order, bool((writes != 1).any())


def _rows(E, rng):
    yield rng.standard_normal(E).astype(np.float32)
    yield (rng.integers(-2, 3, E) * 0.25).astype(np.float32)          # many exact ties
    yield np.full(E, np.float32(1.0 / E))                              # all equal: index order
    p = rng.random(E).astype(np.float32)
    p[rng.choice(E, 3, replace=False)] = np.nan                        # NaN first
    yield p
    yield np.zeros(E, np.float32)


@pytest.mark.parametrize("direction", [+1, -1])
@pytest.mark.parametrize("E", [17, 24, 32, 63, 64, 65, 100, 127, 128, 129, 191, 192, 200, 255, 256])
def test_wg_ranks_equal_a_plain_sort(E, direction):
    rng = np.random.default_rng(E * 3 + (direction > 0))
    maps = lane_maps(direction)
    for p in _rows(E, rng):
        keys = sel_key(p, np.arange(E))
        order, collided = wg_ranks(keys, maps)
        assert not collided
        np.testing.assert_array_equal(order, np.argsort(keys, kind="stable"))
        # torch's descending order with NaN first and equal values by index
        assert sorted(order.tolist()) == list(range(E))


def w1_sort(keys, maps, NS):
    """select_one_token_w1's network (csrc/pp_common.h), E <= 64 * NS: key i in slot
    i // 64 of lane i % 64 (padding ~0), bitonic over positions n = 64 q + lane: partner
    n ^ j in another lane (the exchange maps) for j < 64, in the other slot of the same
    lane for j >= 64. Returns the keys in position order."""
    N = 64 * NS
    allk = np.full(N, np.uint64(0xFFFFFFFFFFFFFFFF))
    allk[:keys.size] = keys
    key = allk.reshape(NS, WAVE).copy()
    lanes = np.arange(WAVE)
    k2 = 2
    while k2 <= N:
        j = k2 >> 1
        while j > 0:
            if j >= 64:
                js = j >> 6
                for q in range(NS):
                    if q & js:
                        continue
                    q2 = q | js
                    up = ((64 * q + lanes) & k2) == 0
                    lo, hi = np.minimum(key[q], key[q2]), np.maximum(key[q], key[q2])
                    key[q], key[q2] = np.where(up, lo, hi), np.where(up, hi, lo)
            else:
                for q in range(NS):
                    n = 64 * q + lanes
                    o = key[q][maps[j]]
                    keep_min = ((n & j) == 0) == ((n & k2) == 0)
                    key[q] = np.where((o < key[q]) == keep_min, o, key[q])
            j >>= 1
        k2 <<= 1
    return key.reshape(-1)


@pytest.mark.parametrize("direction", [+1, -1])
@pytest.mark.parametrize("E", [17, 24, 32, 63, 64, 65, 96, 100, 127, 128])
def test_one_wave_sort_equals_a_plain_sort(E, direction):
    """The one-wave form (E <= 128): sorted positions are the ranks, the first E of them
    the real keys strictly increasing (the kernel's sortedness check), the same order as
    the multi-wave form and a plain sort."""
    rng = np.random.default_rng(E * 5 + (direction > 0))
    maps = lane_maps(direction)
    NS = 1 if E <= 64 else 2
    for p in _rows(E, rng):
        keys = sel_key(p, np.arange(E))
        srt = w1_sort(keys, maps, NS)
        order = (srt[:E] & np.uint64(0xFFFFFFFF)).astype(np.int64)
        assert (srt[1:E] > srt[:E - 1]).all()
        np.testing.assert_array_equal(order, np.argsort(keys, kind="stable"))
        np.testing.assert_array_equal(order, wg_ranks(keys, maps)[0])


def test_one_wave_sort_with_a_wrong_exchange_fails_the_sortedness_check():
    """xor 4 as a row rotation breaks the network: the first E positions are no longer
    strictly increasing, which the kernel reports through its bad flag."""
    E = 100
    maps = lane_maps(+1)
    maps[4] = row_ror(4, +1)
    keys = sel_key(np.random.default_rng(3).standard_normal(E).astype(np.float32), np.arange(E))
    srt = w1_sort(keys, maps, 2)
    assert not (srt[1:E] > srt[:E - 1]).all()


def test_a_wrong_exchange_is_caught_by_the_permutation_check():
    """The failure mode the kernel now reports instead of hiding: xor 4 done as one
    row rotation by 4 loses keys, two keys share a rank and the collision flag is set
    (the kernel raises its error flag and streams nothing)."""
    E = 192
    rng = np.random.default_rng(1)
    maps = lane_maps(+1)
    maps[4] = row_ror(4, +1)
    keys = sel_key(rng.standard_normal(E).astype(np.float32), np.arange(E))
    order, collided = wg_ranks(keys, maps)
    assert collided and (order == -1).any()


def _dpp_scan_step(v, ctrl, row_mask):
    """One `v += update_dpp(0, v, ctrl, row_mask, 0xf, false)` of wave_incl_scan_f64
    (csrc/pp_common.h): row_shr:n (0x110 + n) reads lane i - n of the row, row_bcast:15
    (0x142) lane 15 of the previous row, row_bcast:31 (0x143) lane 31; a lane with no
    source, or in a row the row mask leaves out, reads the identity 0."""
    out = np.zeros_like(v)
    for i in range(WAVE):
        row, r = divmod(i, 16)
        if not (row_mask >> row) & 1:
            continue
        if 0x111 <= ctrl <= 0x11F:
            n = ctrl - 0x110
            if r >= n:
                out[i] = v[i - n]
        elif ctrl == 0x142:
            if row > 0:
                out[i] = v[16 * row - 1]
        elif ctrl == 0x143:
            out[i] = v[31]
        else:
            raise AssertionError(hex(ctrl))
    return v + out


def test_dpp_wave_scan_is_an_inclusive_prefix_sum():
    """The six DPP steps of wave_incl_scan_f64 give every lane the sum of lanes 0..i (on
    integers, where the addition order cannot matter -- as for the exact fp64 partial
    sums the selection cut feeds it)."""
    rng = np.random.default_rng(7)
    for _ in range(20):
        v = rng.integers(0, 1 << 20, WAVE).astype(np.int64)
        s = v.copy()
        for ctrl, mask in ((0x111, 0xF), (0x112, 0xF), (0x114, 0xF), (0x118, 0xF), (0x142, 0xA), (0x143, 0xC)):
            s = _dpp_scan_step(s, ctrl, mask)
        np.testing.assert_array_equal(s, np.cumsum(v))
