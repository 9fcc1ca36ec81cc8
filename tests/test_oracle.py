"""The oracle (oracle/oracle.c) pinned without trusting its own formulas.

Each check is one the reference's arithmetic fixes independently of how the oracle is written:
  * closed forms: quantize_x's scalar steps (tests/int8-check.ts:248-257, and NumPy's packing.quantize at bias 0),
    int8_sums/six_sums = -64 * sum, interleave's byte map and sums (tests/ternary-check.ts:95-103), float16 widening
    against IEEE binary16 over all 65536 halves;
  * round trips: pack6 -> six unpack (tests/test_int6.py), hand-derived bytes of the int6 layout;
  * hand-derived float32 answers of order-revealing inputs: big/small products that tell the reference's lane
    chains, the order of the horizontal sum, the place of the tail groups and the separate (unfused) roundings apart
    from every plausible alternative (relaxed/int8.ts:26-47, kernel/matmul.ts:60-97, relaxed/signs.ts:28-55);
  * the lane membership of matmul_q8's integer partial sums, found position by position;
  * exact float64 sums of the same integers within a bound, and power-of-two scales where every order is exact;
  * the reference tests' own models (int8-check.ts:65-90, ternary-check.ts:129-139) on their LCG streams, bit for bit.
"""
import numpy as np
import pytest

import models
from models import F
from streams import LCG, pack6, pack_binary, pack_ternary, scale_rule, uninterleave_index


# ---- quantize_x ---------------------------------------------------------------------------------------------
def quantize_cases():
    rng = LCG(644)
    groups = 12
    x = np.zeros(groups * 32, F)
    for g in range(groups):
        size = [1, 3.0000002, 1e-30, 65504, 1.5e-5, 2 ** -140][g % 6]
        for j in range(32):
            x[g * 32 + j] = 0 if g == 4 else (-0.0 if g == 5 else F(((rng.next() % 2001) - 1000) * 1e-3 * size))
    x[6 * 32], x[6 * 32 + 31] = F(-3), F(3)
    for j in range(1, 31):
        x[7 * 32 + j] = F((j - 15) * 0.5)
    x[7 * 32], x[7 * 32 + 31] = F(63), F(-63)
    return x


@pytest.mark.parametrize("bias", [0, 64])
def test_quantize_x_scalar_steps(oracle, bias):
    """tests/int8-check.ts:232-265's cases: every scale size, zeros, -0, the ends, half steps, 1/scale overflow."""
    x = quantize_cases()
    xq, xs = oracle.quantize_x(x, bias)
    want_q, want_s = models.quantize_x_model(x, bias)
    assert np.array_equal(xs.view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(xq, want_q)


def test_quantize_x_matches_numpy_packing_at_bias0(oracle):
    """At bias 0 quantize_x is the converter's NumPy quantize() (src/python/engine/packing.py:40-45, quantize.ts:125-128),
    written here as that one expression: scales max|x|/127, values rint(x * (1/scale))."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(64 * 32) * rng.choice([1e-3, 1, 50], 64 * 32)).astype(F)
    xq, xs = oracle.quantize_x(x, 0)
    groups = x.reshape(-1, 32)
    scales = (np.abs(groups).max(axis=1) / 127.0).astype(F)
    inverse = np.divide(F(1.0), scales, out=np.zeros_like(scales), where=scales > 0)
    want = np.rint(groups * inverse[:, None]).astype(np.int8).reshape(-1)
    assert np.array_equal(xs, scales)
    assert np.array_equal(xq.view(np.int8), want)


def test_quantize_x_bounds(oracle):
    """bias 64 writes 1..127 and bias 0 -127..127 wherever 1/scale is finite (int8-check.ts:258-260); the value
    (q - bias) * scale is within half a step of x."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(4096).astype(F)
    for bias, lo, hi in [(64, 1, 127), (0, -127, 127)]:
        xq, xs = oracle.quantize_x(x, bias)
        q = xq.astype(np.int32) if bias else xq.view(np.int8).astype(np.int32)
        assert q.min() >= lo and q.max() <= hi
        back = (q - bias).reshape(-1, 32) * xs[:, None].astype(np.float64)
        assert np.all(np.abs(back - x.reshape(-1, 32)) <= xs[:, None] * 0.5 * (1 + 1e-6))


def test_quantize_x_nan_lane_rule(oracle):
    """quantize.ts:10-19: a NaN in lane 0 (values 4i) makes the scale NaN; a NaN elsewhere is passed over by the
    scalar comparisons of lanes 1..3 (the NaN lane's maximum is NaN, and NaN > amax is false)."""
    x = np.ones(64, F)
    x[0] = np.nan          # group 0: lane 0
    x[32 + 5] = np.nan     # group 1: lane 1
    x[32 + 1] = F(2.0)     # group 1's largest is in lane 1 too: lost with the NaN
    x[32 + 2] = F(1.5)     # lane 2
    xq, xs = oracle.quantize_x(x, 0)
    assert np.isnan(xs[0])
    assert xs[1] == F(F(1.5) / F(127.0))
    assert np.all(xq[:32] == 0)  # inv = 0 where the scale is NaN


# ---- corrections, int6 layout, interleave, halves ----------------------------------------------------------
def test_int8_sums_closed_form(oracle):
    rng = np.random.default_rng(3)
    w = rng.integers(-128, 128, 32 * 37).astype(np.int8)
    w[:32] = 127
    w[32:64] = -128
    want = -64 * w.astype(np.int64).reshape(-1, 32).sum(axis=1)
    assert np.array_equal(oracle.int8_sums(w), want.astype(np.int32))


def test_six_unpack_round_trip_and_bytes(oracle):
    rng = np.random.default_rng(4)
    v = (4 * rng.integers(-32, 32, 32 * 29)).astype(np.int8)
    assert np.array_equal(oracle.six_unpack(pack6(v)), v)
    # hand-derived bytes: -128 = six bits 100000 (low nibble 0, top 10): bytes 0..15 = 0x00, tops 0b10101010;
    # 124 = 011111 (low 1111, top 01): 0xff and 0b01010101
    assert np.array_equal(pack6(np.full(32, -128, np.int8)), [0] * 16 + [0xAA] * 8)
    assert np.array_equal(pack6(np.full(32, 124, np.int8)), [0xFF] * 16 + [0x55] * 8)
    assert np.array_equal(oracle.six_unpack(np.array([0] * 16 + [0xAA] * 8, np.uint8)), [-128] * 32)
    assert np.array_equal(oracle.six_unpack(np.array([0xFF] * 16 + [0x55] * 8, np.uint8)), [124] * 32)
    # one value at a time: value j alone nonzero lands at j
    for j in range(32):
        one = np.zeros(32, np.int8)
        one[j] = -4
        assert np.array_equal(oracle.six_unpack(pack6(one)), one)


def test_six_sums_closed_form(oracle):
    rng = np.random.default_rng(5)
    v = (4 * rng.integers(-32, 32, 32 * 19)).astype(np.int8)
    want = -64 * v.astype(np.int64).reshape(-1, 32).sum(axis=1)
    assert np.array_equal(oracle.six_sums(pack6(v)), want.astype(np.int32))


@pytest.mark.parametrize("n", [128, 256, 384, 640, 1152])
def test_interleave_byte_map(oracle, n):
    """tests/ternary-check.ts:84-106."""
    rng = LCG(231)
    a = np.array([(rng.next() & 255) - 128 for _ in range(n)], np.int8)
    a[:32], a[32:64] = 127, -128
    xs = (np.arange(n // 32) + 0.5).astype(F)
    got, area = oracle.interleave(a, xs)
    want_bytes, want_sums = models.interleave_model(a)
    assert np.array_equal(got, want_bytes)
    assert np.array_equal(area[: n // 32], xs)
    assert np.array_equal(area[n // 32:].view(np.int32), want_sums)


def test_half_all_65536(oracle):
    """kernels/kernel/halves.ts: exact IEEE binary16 -> binary32 for every finite half; an infinity reads as 65536."""
    import ctypes
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([L.o_half(ctypes.c_uint16(int(b))) for b in bits], F)
    halves = bits.astype(np.uint16).view(np.float16)
    finite = np.isfinite(halves)
    assert np.array_equal(got[finite].view(np.uint32), halves[finite].astype(F).view(np.uint32))
    assert got[0x7C00] == 65536.0 and got[0xFC00] == -65536.0


# ---- matmul_q8r: order-revealing inputs ----------------------------------------------------------------------
BIG = 24  # 2^24: adding 1 to it is lost (16777217 rounds to 16777216, ties to even)


def q8r_one(oracle, ds, es):
    xq, xs, w, ws, wc, n = models.crafted_q8r(ds, es)
    return oracle.matmul_q8r(xq, xs, w, ws, wc, n)[0]


def test_q8r_lanes_are_g_mod_4(oracle):
    """relaxed/int8.ts:26-39: lane k adds groups 4j + k.  p0 = 2^24, p1 = 1, p4 = -2^24 (12 groups): lane 0 is
    2^24 - 2^24 = 0 and lane 1 keeps the 1 -> 1.  One accumulator in group order gives 0 (2^24 + 1 -> 2^24), and
    lanes of consecutive blocks (g // 3) give 0 too."""
    ds = [1, 1, 0, 0, -1, 0, 0, 0, 0, 0, 0, 0]
    es = [BIG, 0, 0, 0, BIG, 0, 0, 0, 0, 0, 0, 0]
    assert q8r_one(oracle, ds, es) == F(1.0)


def test_q8r_lane_chain_in_order(oracle):
    """lane 0 takes groups 0, 4, 8 in that order: (2^24 + 1) + -2^24 = 0, where (2^24 + -2^24) + 1 would be 1."""
    ds = [1, 0, 0, 0, 1, 0, 0, 0, -1, 0, 0, 0]
    es = [BIG, 0, 0, 0, 0, 0, 0, 0, BIG, 0, 0, 0]
    assert q8r_one(oracle, ds, es) == F(0.0)


def test_q8r_hsum_order(oracle):
    """math.ts:7-9: ((l0 + l1) + l2) + l3.  l0 = 2^24, l1 = 1, l2 = 1, l3 = -2^24: ((2^24 + 1) + 1) - 2^24 = 0,
    where (l0 + l1) + (l2 + l3) = 2^24 + (1 - 2^24) = 1."""
    ds = [1, 1, 1, -1]
    es = [BIG, 0, 0, BIG]
    assert q8r_one(oracle, ds, es) == F(0.0)


def test_q8r_tail_after_hsum(oracle):
    """relaxed/int8.ts:40-47: groups past the fours are added one at a time after hsum.  5 groups: p0 = 2^24,
    p1 = -2^24, p4 = 1: hsum 0, then + 1 = 1.  Folding group 4 into lane 0 would give (2^24 + 1) - 2^24 = 0."""
    ds = [1, -1, 0, 0, 1]
    es = [BIG, BIG, 0, 0, 0]
    assert q8r_one(oracle, ds, es) == F(1.0)
    # the tail groups one at a time, in order: ng = 7 -> groups 4, 5, 6: (0 + 2^24) + 1 + -2^24 = 0
    ds = [0, 0, 0, 0, 1, 1, -1]
    es = [0, 0, 0, 0, BIG, 0, BIG]
    assert q8r_one(oracle, ds, es) == F(0.0)


def test_q8r_scale_product_rounded_first(oracle):
    """f(d * f(ws * xs)): the scales' product is rounded before the integer meets it.  d = 3, ws = xs = 1 + 2^-12:
    ws * xs = 1 + 2^-11 + 2^-24 rounds (a tie, to even) to 1 + 2^-11, and 3 (1 + 2^-11) is exact; multiplying the
    unrounded product would give 3 + 3 * 2^-11 + 2^-22 instead."""
    xq, xs, w, ws, wc, n = models.crafted_q8r([3], [0])
    ws[0] = xs[0] = F(1 + 2.0 ** -12)
    got = oracle.matmul_q8r(xq, xs, w, ws, wc, n)[0]
    assert got == F(3 + 3 * 2.0 ** -11)
    assert got != F(3 + 3 * 2.0 ** -11 + 2.0 ** -22)


def test_q8r_no_fused_multiply_add(oracle):
    """f(lane + f(d * s)): the product is rounded before it is added.  Lane 0 takes group 0 (-3) then group 4
    (d = 3, s = 1 + 2^-23): 3 s = 3 + 1.5 ulp rounds to 3 + 2^-21, and -3 + that = 2^-21; a fused multiply-add would
    give 3 * 2^-23."""
    ds = [-3, 0, 0, 0, 3, 0, 0, 0]
    xq, xs, w, ws, wc, n = models.crafted_q8r(ds, [0] * 8)
    ws[4] = F(1 + 2.0 ** -23)
    got = oracle.matmul_q8r(xq, xs, w, ws, wc, n)[0]
    assert got == F(2.0 ** -21)
    assert got != F(3 * 2.0 ** -23)


def test_q8r_wc_enters_the_integer(oracle):
    """relaxed/int8.ts:37, 45: the correction is added to the group's integer before it is scaled: with wc = 0 the
    integer is dot(w, q) itself (here 65 * d), with int8_sums' wc it is dot(w, q - 64) (= d)."""
    xq, xs, w, ws, wc, n = models.crafted_q8r([5, -7, 2, 1, 3], [0, 0, 0, 0, 0])
    assert oracle.matmul_q8r(xq, xs, w, ws, wc, n)[0] == F(5 - 7 + 2 + 1 + 3)
    assert oracle.matmul_q8r(xq, xs, w, ws, np.zeros_like(wc), n)[0] == F(65 * (5 - 7 + 2 + 1 + 3))


# ---- matmul_q8: lane membership and order ---------------------------------------------------------------------
def q8_groups(ds_by_pos, es):
    """one row; group g holds a single nonzero product ds_by_pos[g] = (position, d) (activation 1 there), scale 2^e"""
    ng = len(ds_by_pos)
    n = ng * 32
    w = np.zeros(n, np.int8)
    xq = np.zeros(n, np.int8)
    for g, (pos, d) in enumerate(ds_by_pos):
        if d:
            w[g * 32 + pos] = d
            xq[g * 32 + pos] = 1
    ws = np.array([F(2.0 ** e) for e in es], F)
    return xq, np.ones(ng, F), w, ws, n


def test_q8_lane_membership(oracle):
    """kernel/matmul.ts:60-66: lane k holds products 2k, 2k+1, 2k+8, 2k+9 of each half.  Group 0 puts 2^24 at
    position 0 (lane 0), group 1 puts 1 at position p, group 2 puts -2^24 at position 0: the 1 is lost exactly when
    position p is in lane 0's chain."""
    lane0 = {0, 1, 8, 9, 16, 17, 24, 25}
    for p in range(32):
        xq, xs, w, ws, n = q8_groups([(0, 1), (p, 1), (0, -1)], [BIG, 0, BIG])
        got = oracle.matmul_q8(xq, xs, w, ws, n)[0]
        assert got == (F(0.0) if p in lane0 else F(1.0)), p


def test_q8_lane_of_each_position(oracle):
    """and which lane: with 2^24 in lane k0 and -2^24 in lane k1 != k0 after it, a 1 in lane L survives unless
    L == k0 ((2^24 + 1) - 2^24 in one lane is 0; in two lanes 2^24 + (1 - 2^24)... the hsum order decides)."""
    lane_of = lambda p: (p % 8) // 2
    for p in range(32):
        for k0 in range(4):
            pos0 = 2 * k0
            xq, xs, w, ws, n = q8_groups([(pos0, 1), (p, 1), (pos0, -1)], [BIG, 0, BIG])
            got = oracle.matmul_q8(xq, xs, w, ws, n)[0]
            assert got == (F(0.0) if lane_of(p) == k0 else F(1.0)), (p, k0)


def test_q8_all_groups_in_lanes(oracle):
    """kernel/matmul.ts:84-95: matmul_q8 has no tail rule: group 4 (of 5) goes into the lanes like the others.
    p0 = 2^24 (lane 0), p4 = 1 (lane 0), p1 = -2^24 (lane 0): 2^24 + (-2^24) + 1 in lane 0's order 0, 1, 4 = 1;
    lane 0 order is groups 0, 1, 4: ((2^24 - 2^24) + 1) = 1."""
    xq, xs, w, ws, n = q8_groups([(0, 1), (0, -1), (0, 0), (0, 0), (0, 1)], [BIG, BIG, 0, 0, 0])
    assert oracle.matmul_q8(xq, xs, w, ws, n)[0] == F(1.0)
    # and groups 0, 4, 1 would differ: put the 1 first among the big ones
    xq, xs, w, ws, n = q8_groups([(0, 1), (0, 1), (0, 0), (0, 0), (0, -1)], [BIG, 0, 0, 0, BIG])
    assert oracle.matmul_q8(xq, xs, w, ws, n)[0] == F(0.0)


def test_q8_int16_pairs(oracle):
    """dot32 adds products 2k and 2k+8 in int16 before widening (matmul.ts:60-72): -128 * -128 twice wraps to
    -32768 (only where quantize_x's scale is 0: the reference's note); -128 * 127 + -128 * -128 stays exact."""
    n = 32
    w = np.zeros(n, np.int8)
    xq = np.zeros(n, np.int8)
    w[0], xq[0], w[8], xq[8] = -128, -128, -128, -128
    got = oracle.matmul_q8(xq, np.ones(1, F), w, np.ones(1, F), n)[0]
    assert got == F(-32768.0)
    xq[8] = 127
    assert oracle.matmul_q8(xq, np.ones(1, F), w, np.ones(1, F), n)[0] == F(16384 - 16256)


# ---- matmul_t2r: order-revealing inputs --------------------------------------------------------------------
def t2_crafted(terms, groups):
    """one ternary row: terms[(g, k)] = (w, e): sub-group k of group g holds one weight w (code w + 1) against an
    activation 1, and the activation scale xs[4g + k] = 2^e; every group scale d = 1 (half 0x3c00)."""
    n = groups * 128
    codes = np.ones(n, np.uint8)
    a = np.zeros(n, np.int8)
    xs = np.ones(n // 32, F)
    for (g, k), (wv, e) in terms.items():
        j = g * 128 + k * 32
        codes[j] = wv + 1
        a[j] = 1
        xs[4 * g + k] = F(2.0 ** e)
    wq = pack_ternary(codes)
    ws = np.full(groups, 0x3C00, np.uint16)
    return a, xs, wq, ws, n


def t2_run(oracle, a, xs, wq, ws, n):
    xq, area = oracle.interleave(a, xs)
    return oracle.matmul_t2r(xq, area, wq, ws, n)[0]


def test_t2r_lane_is_subgroup(oracle):
    """relaxed/signs.ts:28-55: lane k adds sub-group k (activations 32k..32k+31) of every group in order.
    2^24 (g0 k0), 1 (g0 k1), -2^24 (g1 k0): lane 0 cancels, lane 1 keeps 1."""
    a, xs, wq, ws, n = t2_crafted({(0, 0): (1, BIG), (0, 1): (1, 0), (1, 0): (-1, BIG)}, 2)
    assert t2_run(oracle, a, xs, wq, ws, n) == F(1.0)
    a, xs, wq, ws, n = t2_crafted({(0, 0): (1, BIG), (1, 0): (1, 0), (2, 0): (-1, BIG)}, 3)
    assert t2_run(oracle, a, xs, wq, ws, n) == F(0.0)


def test_t2r_hsum_order(oracle):
    a, xs, wq, ws, n = t2_crafted({(0, 0): (1, BIG), (0, 1): (1, 0), (0, 2): (1, 0), (0, 3): (-1, BIG)}, 1)
    assert t2_run(oracle, a, xs, wq, ws, n) == F(0.0)


def test_t2r_scales_twice_rounded(oracle):
    """f(f(whole * xs) * d): two roundings.  whole = 1 (a weight 1 against 1), xs = 1 + 2^-23, d = half 1 + 2^-10
    (0x3c01): f(1 + 2^-23) * (1 + 2^-10) = 1 + 2^-10 + 2^-23 + 2^-33 -> 1 + 2^-10 + 2^-23 (one rounding of the
    product, which the double product's exact value also rounds to here); the second rounding is what matters for
    a larger whole: whole = 3: f(3 + 3 * 2^-23) = 3 + 2^-21 (1.5 ulp rounds to even: 2 ulp), times (1 + 2^-10)."""
    n = 128
    codes = np.ones(n, np.uint8)
    a = np.zeros(n, np.int8)
    codes[0], a[0] = 2, 3
    xs = np.ones(4, F)
    xs[0] = F(1 + 2.0 ** -23)
    wq = pack_ternary(codes)
    ws = np.array([0x3C01], np.uint16)
    got = t2_run(oracle, a, xs, wq, ws, n)
    first = F(F(3.0) * xs[0])
    assert first == F(3 + 2.0 ** -21)
    assert got == F(first * F(1 + 2.0 ** -10))


def test_t2r_fourth_code(oracle):
    """ternary.ts:23-27 / ternary-check.ts:7-10: code 3 (PQ2_0's fourth, weight 2) passes the mask."""
    n = 128
    codes = np.ones(n, np.uint8)
    a = np.zeros(n, np.int8)
    codes[5], a[5] = 3, 7
    a[6] = -1
    got = t2_run(oracle, a, np.ones(4, F), pack_ternary(codes), np.array([0x3C00], np.uint16), n)
    assert got == F(14.0)


# ---- exact sums, power-of-two scales, float64 bound ----------------------------------------------------------
def test_q8r_power_of_two_scales_exact(oracle):
    """With every scale a power of two and small integers, every partial sum is exact: the result is the exact
    integer sum, whatever the order (pins the indexing of w, q, ws, wc over rows and groups)."""
    rng = np.random.default_rng(6)
    rows, ng = 7, 13
    n = ng * 32
    # |dot| <= 32 * 4 * 8 = 1024 and scale products 2^-6..2^0: every partial sum is a multiple of 2^-6 below
    # 2^14, exact in float32
    w = rng.integers(-4, 5, rows * n).astype(np.int8)
    xq = rng.integers(56, 73, n).astype(np.uint8)
    ws = (2.0 ** rng.integers(-3, 1, rows * ng)).astype(F)
    xs = (2.0 ** rng.integers(-3, 1, ng)).astype(F)
    wc = oracle.int8_sums(w)
    got = oracle.matmul_q8r(xq, xs, w, ws, wc, n)
    dots = (w.reshape(rows, ng, 32).astype(np.int64) * (xq.reshape(ng, 32).astype(np.int64) - 64)).sum(-1)
    want = (dots * ws.reshape(rows, ng).astype(np.float64) * xs.astype(np.float64)).sum(-1)
    assert np.array_equal(got.astype(np.float64), want)


def test_q8r_float64_bound(oracle):
    rng = np.random.default_rng(7)
    rows, n = 64, 4096
    ng = n // 32
    x = rng.standard_normal(n).astype(F)
    xq, xs = oracle.quantize_x(x, 64)
    w = rng.integers(-127, 128, rows * n).astype(np.int8)
    ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
    got = oracle.matmul_q8r(xq, xs, w, ws, oracle.int8_sums(w), n)
    dots = (w.reshape(rows, ng, 32).astype(np.int64) * (xq.reshape(ng, 32).astype(np.int64) - 64)).sum(-1)
    exact = (dots * (ws.reshape(rows, ng).astype(np.float64) * xs.astype(np.float64))).sum(-1)
    assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))


def test_q6_is_q8_on_widened_weights(oracle):
    """relaxed/six.ts:10-39, kernel/matmul.ts:226-244: the int6 products are the int8 ones on the widened
    groups (six.ts:1-11), scale and order alike."""
    rng = np.random.default_rng(8)
    rows, ng = 9, 11
    n = ng * 32
    v = (4 * rng.integers(-32, 32, rows * n)).astype(np.int8)
    packed = pack6(v)
    ws = rng.random(rows * ng).astype(F)
    x = rng.standard_normal(n).astype(F)
    xq, xs = oracle.quantize_x(x, 64)
    assert np.array_equal(oracle.matmul_q6r(xq, xs, packed, ws, oracle.six_sums(packed), n),
                          oracle.matmul_q8r(xq, xs, v, ws, oracle.int8_sums(v), n))
    xq0, xs0 = oracle.quantize_x(x, 0)
    assert np.array_equal(oracle.matmul_q6(xq0, xs0, packed, ws, n), oracle.matmul_q8(xq0, xs0, v, ws, n))


def test_t2r_float64_bound_and_identity(oracle):
    """The integer of sub-group k is dot(code - 1, a) exactly (ternary.ts:37-43): power-of-two scales give the
    exact float64 sum; random scales stay within 1e-5 of max |y|."""
    rng = np.random.default_rng(9)
    rows, groups = 6, 5
    n = groups * 128
    codes = rng.integers(0, 4, rows * n).astype(np.uint8)
    a = rng.integers(-128, 128, n).astype(np.int8)
    wq = pack_ternary(codes)
    for power in (True, False):
        if power:
            xs = (2.0 ** rng.integers(-6, 0, n // 32)).astype(F)
            d = (2.0 ** rng.integers(-6, 0, rows * groups)).astype(np.float16)
        else:
            xs = (rng.random(n // 32) * 0.01).astype(F)
            d = (rng.random(rows * groups) * 0.01).astype(np.float16)
        got = t2_run_all(oracle, a, xs, wq, d.view(np.uint16), n)
        whole = ((codes.reshape(rows, n // 32, 32).astype(np.int64) - 1) * a.reshape(n // 32, 32)).sum(-1)
        exact = (whole * xs.astype(np.float64) * np.repeat(d.astype(np.float64).reshape(rows, groups), 4, axis=1)).sum(-1)
        if power:
            assert np.array_equal(got.astype(np.float64), exact)
        else:
            assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))


def t2_run_all(oracle, a, xs, wq, ws, n):
    xq, area = oracle.interleave(a, xs)
    return oracle.matmul_t2r(xq, area, wq, ws, n)


# ---- the reference tests' own models on their streams ---------------------------------------------------------
def int8_check_case(ng, rows=13, tokens=4):
    """tests/int8-check.ts:129-171's inputs for one group count (tokens 0..2 the fixed patterns, 3 random)."""
    rng = LCG(644 + ng)
    n = ng * 32
    w8 = np.array([(rng.next() & 255) - 128 for _ in range(rows * n)], np.int8)
    w8[:n], w8[n:2 * n] = 127, -128
    w8[2 * n:3 * n] = np.where(np.arange(n) & 1, 127, -128)
    wsv = np.array([scale_rule(rng, i) for i in range(rows * ng)], F)
    acts, scales = [], []
    for t in range(tokens):
        if t < 3:
            q = [127, 0, None][t]
            u = np.full(n, q, np.uint8) if q is not None else np.where(np.arange(n) & 1, 127, 0).astype(np.uint8)
        else:
            u = np.array([rng.next() & 127 for _ in range(n)], np.uint8)
        acts.append(u)
        scales.append(np.array([scale_rule(rng, g + t) for g in range(ng)], F))
    return w8, wsv, acts, scales, n


@pytest.mark.parametrize("ng", [1, 2, 3, 4, 5, 7, 9, 12, 13, 80, 81])
def test_q8r_reference_model(oracle, ng):
    w8, wsv, acts, scales, n = int8_check_case(ng)
    rows = w8.size // n
    wc = oracle.int8_sums(w8)
    for q, xs in zip(acts, scales):
        got = oracle.matmul_q8r(q, xs, w8, wsv, wc, n)
        for i in range(rows):
            want = models.q8r_model(w8[i * n:(i + 1) * n], q, wsv[i * ng:(i + 1) * ng], xs, ng)
            assert got[i].view(np.uint32) == want.view(np.uint32), (ng, i)


@pytest.mark.parametrize("ng", [1, 3, 4, 9, 13])
def test_q8_reference_model(oracle, ng):
    rng = LCG(77 + ng)
    n, rows = ng * 32, 5
    w8 = np.array([(rng.next() & 255) - 128 for _ in range(rows * n)], np.int8)
    q = np.array([(rng.next() % 255) - 127 for _ in range(n)], np.int8)
    wsv = np.array([scale_rule(rng, i) for i in range(rows * ng)], F)
    xs = np.array([scale_rule(rng, g + 1) for g in range(ng)], F)
    got = oracle.matmul_q8(q, xs, w8, wsv, n)
    for i in range(rows):
        want = models.q8_model(w8[i * n:(i + 1) * n], q, wsv[i * ng:(i + 1) * ng], xs, ng)
        assert got[i].view(np.uint32) == want.view(np.uint32)


@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 7, 9])
def test_t2r_reference_model(oracle, groups):
    """tests/ternary-check.ts:108-139, its stream and fixed rows (row 0's first group all +1, row 1's second all
    -1, activations at int8's ends)."""
    rng = LCG(231 + groups)
    rows, n = 13, groups * 128
    codes = np.array([rng.next() & 3 for _ in range(rows * n)], np.uint8)
    codes[:128] = 2
    if groups > 1:
        codes[n + 128:n + 256] = 0
    halves = []
    for g in range(rows * groups):
        v = 2.0 ** -20 * (1 + rng.next() % 1000) if g % 11 == 7 else (0 if g % 13 == 5 else 1e-3 * (1 + rng.next() % 1000))
        halves.append(np.float16(v))
    hs = np.array(halves, np.float16)
    a = np.array([(rng.next() & 255) - 128 for _ in range(n)], np.int8)
    a[:64], a[64:128] = 127, -128
    if groups > 1:
        a[128:256] = -128
    xs = np.array([F(1e-2 * (1 + rng.next() % 1000)) for _ in range(n // 32)], F)
    got = t2_run_all(oracle, a, xs, pack_ternary(codes), hs.view(np.uint16), n)
    for i in range(rows):
        want = models.t2_model(codes[i * n:(i + 1) * n], a, xs, hs[i * groups:(i + 1) * groups].astype(F), groups)
        assert got[i].view(np.uint32) == want.view(np.uint32), (groups, i)


# ---- binary weights: kernels/binary.ts, relaxed/signs.ts:123-128, kernel/matmul.ts:222-224 -------------------------
@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 7, 9])
def test_b1r_is_ternary_for_the_same_signs(oracle, groups):
    """tests/ternary-check.ts:286-341: the binary kernel's numbers are the ternary kernel's to the bit for the same
    signs (ternary code 2 b = the weight + 1), scales and activations.  Rows of all +1 and all -1, activations at
    int8's ends and random, scales with subnormal and zero groups; row ranges anywhere.  The two packings are written
    independently (pack_binary: bit 4 h + p of byte c; pack_ternary: 2 bits a weight), so a wrong bit or byte in
    either kernel's unpacking gives a different integer."""
    rows, n = 11, groups * 128
    rng = np.random.default_rng(634 + groups)
    bits = rng.integers(0, 2, rows * n).astype(np.uint8)
    bits[:n], bits[n:2 * n] = 1, 0
    bw = pack_binary(bits, n)
    tw = pack_ternary(2 * bits)
    halves = np.where(np.arange(rows * groups) % 11 == 7, 2.0 ** -20 * (1 + rng.integers(0, 1000, rows * groups)),
                      np.where(np.arange(rows * groups) % 13 == 5, 0.0, 1e-3 * (1 + rng.integers(0, 1000, rows * groups))))
    ws = halves.astype(np.float16).view(np.uint16)
    for t in range(3):
        a = np.where(np.arange(n) & 1, 127, -128) if t == 0 else (np.full(n, -128) if t == 1 else
                                                                  rng.integers(-128, 128, n))
        q = a.astype(np.int8)
        s = (1e-2 * (1 + rng.integers(0, 1000, n // 32))).astype(F)
        xi, area = oracle.interleave(q, s)
        for r0, r1 in [(0, rows), (0, 1), (rows - 1, rows), (3, 8), (5, 5)]:
            got = oracle.matmul_b1r(xi, area, bw, ws, n, r0, r1)
            want = oracle.matmul_t2r(xi, area, tw, ws, n, r0, r1)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, r0, r1)
    # and a float64 bound against the signs themselves (no shared arithmetic with either kernel)
    q = rng.integers(-128, 128, n).astype(np.int8)
    s = (1e-2 * (1 + rng.integers(0, 1000, n // 32))).astype(F)
    xi, area = oracle.interleave(q, s)
    got = oracle.matmul_b1r(xi, area, bw, ws, n).astype(np.float64)
    w = (2.0 * bits.reshape(rows, n) - 1.0)
    d = np.array([oracle.half(h) for h in ws], np.float64).reshape(rows, groups)
    exact = np.zeros(rows)
    for g in range(groups):
        for k in range(4):
            lo = 128 * g + 32 * k
            exact += (w[:, lo:lo + 32] @ q[lo:lo + 32].astype(np.float64)) * float(s[4 * g + k]) * d[:, g]
    scale = np.abs(w).sum(1) * 128 * float(s.max()) * d.max(1) + 1e-30
    assert np.all(np.abs(got - exact) <= 1e-5 * scale)


def test_b1r_tile_is_the_token_kernel(oracle):
    groups, rows, count = 3, 7, 5
    n = 128 * groups
    rng = np.random.default_rng(11)
    bw = pack_binary(rng.integers(0, 2, rows * n), n)
    ws = (rng.random(rows * groups) * 0.01).astype(np.float16).view(np.uint16)
    frame, os_ = 2 * n, 4 * (rows + 1)
    buf = np.zeros(count * frame, np.uint8)
    toks = []
    for t in range(count):
        q = rng.integers(-128, 128, n).astype(np.int8)
        s = (rng.random(n // 32) * 0.01).astype(F)
        xi, area = oracle.interleave(q, s)
        buf[t * frame:t * frame + n] = xi.view(np.uint8)
        buf[t * frame + n:t * frame + n + area.nbytes] = area.view(np.uint8)
        toks.append((xi, area))
    out = np.full(count * os_ // 4, -7, F)
    lib = oracle.lib()
    lib.o_matmul_b1r_tile(out.ctypes.data, buf.ctypes.data, buf[n:].ctypes.data, bw.ctypes.data, ws.ctypes.data, n,
                          1, rows, count, os_, frame, 2)
    got = out.reshape(count, -1)
    for t, (xi, area) in enumerate(toks):
        want = oracle.matmul_b1r(xi, area, bw, ws, n)
        assert np.array_equal(got[t, 1:rows].view(np.uint32), want[1:rows].view(np.uint32))
        assert got[t, 0] == -7 and got[t, rows] == -7


def binary_x_case(rng, groups=40):
    """tests/ternary-check.ts:343-352: groups of +-d, d of every size (1e-30 to 65504), a group of zeros, one of -0"""
    x = np.zeros(groups * 128, F)
    for g in range(groups):
        d = 0.0 if g == 3 else float(F([1, 0.0078125, 3.0000002, 1e-30, 65504, 1.5e-5][g % 6] * (1 + rng.integers(0, 7))))
        x[g * 128:(g + 1) * 128] = -0.0 if g == 5 else np.where(rng.integers(0, 2, 128) == 1, d, -d)
    return x


def test_binary_x_bytes_scales_and_refusals(oracle):
    """tests/ternary-check.ts:343-376: pack_binary's bytes (bit 4 h + p of byte c set where value 64 h + 4 c + p is not
    below 0: -0 counts as 0), the largest |value| a group, and 1 for a value that is not plus or minus it"""
    rng = np.random.default_rng(634)
    x = binary_x_case(rng)
    out, xs, bad = oracle.binary_x(x)
    assert bad == 0
    groups = x.size // 128
    assert np.array_equal(xs, np.abs(x.reshape(groups, 128)).max(1))
    assert np.array_equal(out, pack_binary((~(x < 0)).astype(np.uint8), x.size))
    for at, spoil in [(0, 0.5), (127, 1.0000001), (128 + 63, 2), (128 * 39 + 127, np.nan), (128 * 7 + 5, -0.999999),
                      (128 * 9 + 64 + 3, 0), (128 * 9 + 32 + 1, 0.5), (128 * 9 + 64 + 6, 0.5), (128 * 9 + 96 + 11, 0.5),
                      (128 * 9 + 14, 0.5), (128 * 39 + 127, 0.5)]:
        y = binary_x_case(rng)
        g = at >> 7
        y[g * 128:(g + 1) * 128] = np.where(np.arange(128) % 2 == 1, 3.0, -3.0)
        y[at] = F(spoil * 3)
        assert oracle.binary_x(y)[2] == 1, (at, spoil)
    # a NaN makes its group's scale NaN (f32x4.max keeps it)
    y = binary_x_case(rng)
    y[130] = np.nan
    assert np.isnan(oracle.binary_x(y)[1][1])


# ---- llama.cpp's blocks: kernels/blocks/types.ts, token.ts, row.ts ------------------------------------------------
import blocks_model as bm  # noqa: E402


@pytest.fixture(scope="module")
def sb_setup(oracle):
    rng = np.random.default_rng(363)
    row = bm.codebooks(rng)
    return row, bm.grids(row), oracle.sb_tables(row)


def test_sb_tables(oracle, sb_setup):
    """types.ts:323-348: the grids as given (IQ1_S's plus one), the signs of a 7-bit index with an even count of
    minus signs, IQ4_XS's values / magnitudes / signs, the vectors"""
    row, _, tab = sb_setup
    assert np.array_equal(tab[:17408], row[:17408])
    assert np.array_equal(tab[17408:33792], (row[17408:33792].astype(np.int32) + 1).astype(np.uint8))
    signs = tab[33792:34816].reshape(128, 8)
    assert set(np.unique(signs)) <= {0, 255}
    assert np.all((signs == 255).sum(1) % 2 == 0)
    assert np.array_equal(signs[:, :7] == 255, bm.bits_of(np.arange(128))[:, :7] == 1)
    v = row[33792:].view(np.int8)
    assert np.array_equal(tab[34816:34832].view(np.int8), v)
    assert np.array_equal(tab[34832:34848], np.abs(v.astype(np.int32)).astype(np.uint8))
    assert np.array_equal(tab[34848:34864], np.where(v < 0, 255, 0).astype(np.uint8))


def test_sums_x_closed_form(oracle):
    rng = np.random.default_rng(5)
    n = 512
    q = rng.integers(-127, 128, n).astype(np.int8)
    s = rng.random(n // 32).astype(F)
    area = oracle.sums_x(q, s)
    assert np.array_equal(area[:4 * (n // 32)].view(F), s)
    s16 = area[4 * (n // 32):4 * (n // 32) + 2 * (n // 16)].view(np.int16)
    s8 = area[4 * (n // 32) + 2 * (n // 16):].view(np.int16)
    assert np.array_equal(s16, q.astype(np.int32).reshape(-1, 16).sum(1))
    assert np.array_equal(s8, q.astype(np.int32).reshape(-1, 8).sum(1))


@pytest.mark.parametrize("name", sorted(bm.TYPES))
def test_sb_row_is_the_reader(oracle, sb_setup, name):
    """row.ts: a row as float32 is the converter's reader's (superblocks.py), to the bit: here against a model
    written from the blocks' forms, for random blocks with ordinary and with subnormal scales"""
    _, g, tab = sb_setup
    t = bm.TYPES[name]
    rng = np.random.default_rng(t)
    for tiny in (False, True):
        blocks = bm.random_blocks(rng, t, 12, tiny)
        got = oracle.sb_row(blocks.reshape(-1), tab, 256 * len(blocks), t)
        want = bm.read_floats(t, blocks, g).reshape(-1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, tiny, np.nonzero(got != want)[0][:5])


@pytest.mark.parametrize("name", ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S"])
def test_grid_bytes_are_signed(oracle, name):
    """Outside the converter's grids (magnitudes 0..127): the plain kernel multiplies a grid's bytes as int8
    (types.ts:171-173, extmul_*_i8x16_s), so a byte of 128..255 is a negative magnitude, and sb_row puts the signs on
    with a wrapping byte subtraction (row.ts:32-37, types.ts:163-165: -(-128) is -128)"""
    rng = np.random.default_rng(77)
    row = bm.codebooks(rng)
    row[:17408] = rng.integers(0, 256, 17408, dtype=np.uint8)
    tab = oracle.sb_tables(row)
    g = bm.grids(row)
    for key, (at, count, k) in bm.GRIDS.items():
        if key != "IQ1S":
            g[key] = row[at:at + count * k].view(np.int8).reshape(count, k).astype(np.int32)
    t = bm.TYPES[name]
    nb, rows = 3, 4
    n = 256 * nb
    blocks = bm.random_blocks(rng, t, rows * nb)
    q, s = oracle.quantize_x(rng.standard_normal(n).astype(F), 0)
    q = q.view(np.int8)
    got = oracle.matmul_sbr(q, oracle.sums_x(q, s), blocks.reshape(-1), tab, n, t)
    for r in range(rows):
        want = bm.matmul(t, blocks[r * nb:(r + 1) * nb], q, s, g)
        assert got[r].view(np.uint32) == np.float32(want).view(np.uint32), (name, r)
    # every magnitude -128: with its sign a weight is -(-128) = -128 too, so every weight of the row is -128 S d
    row[:17408] = 0x80
    tab = oracle.sb_tables(row)
    g = {key: np.full((count, k), -128, np.int32) for key, (at, count, k) in bm.GRIDS.items() if key != "IQ1S"}
    g.update({key: value for key, value in bm.grids(row).items() if key not in g})
    got = oracle.sb_row(blocks[:nb].reshape(-1), tab, n, t)
    model = bm.read_floats(t, blocks[:nb], g).reshape(-1)
    assert np.array_equal(got, -np.abs(model)) and np.any(model > 0), name


@pytest.mark.parametrize("name", sorted(bm.TYPES))
def test_matmul_sbr_order_and_integers(oracle, sb_setup, name):
    """token.ts / types.ts:48-57: the exact integers of every group and the kernels' float32 order, to the bit against
    the model; rows cut anywhere; the tile is the token kernel's; and a float64 bound from the reader's weights"""
    _, g, tab = sb_setup
    t = bm.TYPES[name]
    rng = np.random.default_rng(100 + t)
    rows, nb = 7, 3
    n = 256 * nb
    blocks = bm.random_blocks(rng, t, rows * nb)
    w = blocks.reshape(-1)
    for trial in range(3):
        x = rng.standard_normal(n).astype(F) * (1 + 3 * trial)
        q, s = oracle.quantize_x(x, 0)
        q = q.view(np.int8)
        area = oracle.sums_x(q, s)
        got = oracle.matmul_sbr(q, area, w, tab, n, t)
        for r in range(rows):
            want = bm.matmul(t, blocks[r * nb:(r + 1) * nb], q, s, g)
            assert got[r].view(np.uint32) == np.float32(want).view(np.uint32), (name, trial, r, got[r], want)
        part = oracle.matmul_sbr(q, area, w, tab, n, t, 2, 5)
        assert np.array_equal(part[2:5].view(np.uint32), got[2:5].view(np.uint32))
        assert not part[:2].any() and not part[5:].any()
        weights = bm.read_floats(t, blocks, g).reshape(rows, n).astype(np.float64)
        exact = weights @ (q.astype(np.float64) * np.repeat(s.astype(np.float64), 32))
        bound = np.abs(weights) @ (np.abs(q.astype(np.float64)) * np.repeat(s.astype(np.float64), 32))
        assert np.all(np.abs(got - exact) <= 1e-5 * bound + 1e-30), name
    # the tile: three tokens a frame apart
    count, frame = 3, 2 * n + 64
    buf = np.zeros(count * frame, np.uint8)
    toks = []
    for tk in range(count):
        q, s = oracle.quantize_x(rng.standard_normal(n).astype(F), 0)
        area = oracle.sums_x(q.view(np.int8), s)
        buf[tk * frame:tk * frame + n] = q
        buf[tk * frame + n:tk * frame + n + area.size] = area
        toks.append((q.view(np.int8), area))
    out = np.full(count * (rows + 1), -7, F)
    oracle.lib().o_matmul_sbr_tile(out.ctypes.data, buf.ctypes.data, buf[n:].ctypes.data, w.ctypes.data, tab.ctypes.data,
                                   n, 0, rows, count, 4 * (rows + 1), frame, t)
    for tk, (q, area) in enumerate(toks):
        want = oracle.matmul_sbr(q, area, w, tab, n, t)
        assert np.array_equal(out[tk * (rows + 1):tk * (rows + 1) + rows].view(np.uint32), want.view(np.uint32))


# ---- the CPU baseline's vectorised kernel (fast.c) gives the oracle's numbers -----------------------------------
@pytest.mark.parametrize("ng", [1, 3, 4, 7, 13, 128, 448])
def test_fast_q8r_is_the_oracle(oracle, ng):
    """fast.c's AVX2 matmul_q8r (bench.py's CPU baseline) against oracle.c's scalar one, to the bit: random groups
    and the extremes of the relaxed form's pairs (activation 127 by weight -128, twice, in every pair: 2^15 - 256,
    no saturation of the 16-bit pair sums), rows past the quads, the groups past the fours"""
    rng = np.random.default_rng(ng)
    n, rows = 32 * ng, 11
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    w[:n] = -128
    xq, xs = oracle.quantize_x(rng.standard_normal(n).astype(F), 64)
    xq[: min(n, 64)] = 127
    ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
    wc = oracle.int8_sums(w)
    want = oracle.matmul_q8r(xq, xs, w, ws, wc, n)
    got = oracle.fast_matmul_q8r(xq, xs, w, ws, wc, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("count, rows", [(1, 4), (4, 8), (6, 13), (9, 3)])
def test_fast_q8r_tile_is_the_oracle(oracle, count, rows):
    """the tile's 4 x 4 quads, the rows and tokens past them: every (row, token) the oracle's matmul_q8r"""
    rng = np.random.default_rng(100 * count + rows)
    ng = 13
    n = 32 * ng
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
    wc = oracle.int8_sums(w)
    qs = [oracle.quantize_x(rng.standard_normal(n).astype(F), 64) for _ in range(count)]
    got = oracle.fast_matmul_q8r_tile(np.stack([q for q, _ in qs]), np.stack([s for _, s in qs]), w, ws, wc, n, count)
    for t, (q, s) in enumerate(qs):
        want = oracle.matmul_q8r(q, s, w, ws, wc, n)
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), t


# ---- the converters' packers: quantize6_x and ternary_x (kernels/kernel/quantize.ts:153-225) ----------------------
def numpy_quantize6(x):
    """src/python/engine/packing.py:73-80 (quantize6, the converter's NumPy form the reference's smoke test holds the
    kernel to, tests/smoke.ts:800-811), with pack6 (tests/streams.py): 24 bytes and scale / 4 a group"""
    groups = np.asarray(x, np.float32).reshape(-1, 32)
    scales = (np.abs(groups).max(axis=1) / np.float32(31.0)).astype(np.float32)
    inverse = np.divide(np.float32(1.0), scales, out=np.zeros_like(scales), where=scales > 0)
    six = np.clip(np.rint(groups * inverse[:, None]), -32, 31).astype(np.int8)
    return pack6((six * 4).astype(np.int8)), scales / np.float32(4)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantize6_x_is_the_converters_quantize6(oracle, seed):
    """random groups of every magnitude, a group of zeros, and smoke.ts:802-804's ties (halves that round to even
    with a scale of exactly 1), against packing.py's NumPy quantize6 + pack6 to the byte"""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((24, 32)) * np.exp(rng.uniform(-20, 20, (24, 1)))).astype(F)
    x[3] = 0.0
    x[5] = np.arange(32, dtype=F) - F(15.5)
    x[5, 31] = 31.0
    x[6] = -x[5]
    x[7, 0] = 1e-38  # a subnormal scale
    got_bytes, got_scales = oracle.quantize6_x(x.reshape(-1))
    want_bytes, want_scales = numpy_quantize6(x)
    assert np.array_equal(got_bytes, want_bytes)
    assert np.array_equal(got_scales.view(np.uint32), want_scales.view(np.uint32))
    assert not got_bytes[3 * 24:4 * 24].any() and got_scales[3] == 0
    # the ties: value j - 15.5 over scale 1 rounds to the even neighbour (np.rint), so the six bits of -15.5 are -16
    values = oracle.six_unpack(got_bytes[5 * 24:6 * 24]).astype(np.int32) // 4
    assert values.tolist() == np.rint(x[5]).astype(np.int32).tolist() and got_scales[5] == 0.25


def test_quantize6_x_round_trip_and_nan(oracle):
    """six_unpack (kernels/six.ts, pinned separately) of quantize6_x's bytes gives 4 v; v times 4 xs is the value to
    half a scale; a NaN in lane 1..3 of groupMax is passed over (the scale is lane 0's or the others'), one in lane 0
    makes the scale NaN and every code 0 (trunc_sat of NaN)"""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 32)).astype(F)
    b, s = oracle.quantize6_x(x.reshape(-1))
    v = oracle.six_unpack(b).astype(np.float64).reshape(16, 32)  # 4 v
    assert np.all(np.abs(v * s[:, None].astype(np.float64) - x) <= 2 * s[:, None] * (1 + 1e-6))
    y = np.ones((2, 32), F)
    y[0, 1] = np.nan  # lane 1 of the first four: passed over
    y[1, 0] = np.nan  # lane 0: the scale is NaN
    b, s = oracle.quantize6_x(y.reshape(-1))
    assert s[0] == F(1.0 / 31.0) * F(0.25) and np.isnan(s[1])
    assert oracle.six_unpack(b[24:]).tolist() == [0] * 32


def numpy_ternary(x):
    """src/python/engine/packing.py:117-130 (ternary, without its float16 check): the sign + 1 of each value packed
    four to a byte (tests/streams.py), the largest |value| of each group of 128, and whether every value is its sign
    times that"""
    groups = np.asarray(x, np.float32).reshape(-1, 128)
    scales = np.abs(groups).max(axis=1)
    signs = np.sign(groups)
    codes = (np.nan_to_num(signs) + 1).astype(np.uint8)  # (a NaN is refused below; its code is not compared)
    return pack_ternary(codes.reshape(-1)), scales, int(not np.array_equal(signs * scales[:, None], groups))


def ternary_case(rng):
    """tests/ternary-check.ts:252-258: 40 groups, scales of every size, a group of zeros, one of -0 alone"""
    x = np.zeros((40, 128), F)
    for g in range(40):
        d = 0.0 if g == 3 else F([1, 0.0078125, 3.0000002, 1e-30, 65504, 1.5e-5][g % 6] * (1 + rng.integers(0, 7)))
        x[g] = -0.0 if g == 5 else (rng.integers(0, 3, 128) - 1) * F(d)
    return x.reshape(-1)


def test_ternary_x_is_the_converters_ternary(oracle):
    rng = np.random.default_rng(6)
    x = ternary_case(rng)
    got = oracle.ternary_x(x)
    want = numpy_ternary(x)
    assert got[2] == 0 and want[2] == 0
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    assert (got[0][5 * 32:6 * 32] == 0x55).all()  # -0: code 1 (neither above nor below 0)


@pytest.mark.parametrize("at, spoil", [(0, 0.5), (127, 1.0000001), (128 + 63, 2), (128 * 39 + 127, np.nan),
                                       (128 * 7 + 5, -0.999999), (128 * 9 + 33, 0.5), (128 * 9 + 38, 0.5),
                                       (128 * 9 + 43, 0.5), (128 * 9 + 46, 0.5)])
def test_ternary_x_refusals(oracle, at, spoil):
    """tests/ternary-check.ts:276-283: one value of one place that is not ternary (half the scale, a little more
    than it, twice it, not a number; in each of the four vectors of sixteen values) is refused; the codes and scales
    are still written"""
    rng = np.random.default_rng(7)
    x = ternary_case(rng)
    g = at >> 7
    x[g * 128:(g + 1) * 128] = np.where(np.arange(128) % 2 == 1, 3.0, -3.0)
    x[at] = F(spoil * 3)
    got = oracle.ternary_x(x)
    assert got[2] == 1
    assert numpy_ternary(x)[2] == 1
    if not np.isnan(spoil):
        want = numpy_ternary(x)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    else:
        assert np.isnan(got[1][g])
