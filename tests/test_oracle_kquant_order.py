"""Order pins for the oracle's K-quant dots — CPU only.

The integer sub-dots of Q4_K / Q6_K are exact, so only the f32 steps around
them can differ between a faithful restatement and a regrouped one. Each test
here builds blocks whose value under the reference's documented f32 order is
derived by hand in the docstring (every intermediate is an exact power-of-two
sum or a stated round-to-nearest-even tie), asserts the oracle returns exactly
that, and evaluates the plausible regroupings on the same blocks to show that
each gives another value. Reference steps:

  dot_q4k_scalar  kquant.rs:192-218  sum_q f32 chain over j, then ONE
                                     `sumf += d_all*sum_q - dmin_all*sum_m`
  dot_q6k_scalar  kquant.rs:220-250  ONE `sum` chain over both halves' 16 groups,
                                     then `sumf += d_all*sum`
  dot_q4k_avx2    kquant.rs:260-305  integer sumi, fma per block into 8 lanes,
                                     acc_min kept apart, `hsum256(acc) - acc_min`
  dot_q6k_avx2    kquant.rs:454-510  integer sumi over both halves, fma per
                                     block, hsum256 (kquant.rs:512-522)

The float64 closed-form checks at the end use an error bound counted from the
number of f32 roundings on the reference's longest chain, tight enough that an
f16-rounded Q8_K scale fails them.
"""
from fractions import Fraction

import numpy as np
import pytest

F32 = np.float32
U = 2.0 ** -24  # unit roundoff of f32


# ---- block builders (layouts: kquant.rs:26-52) -----------------------------------


def q8k_block(d: float, qs) -> np.ndarray:
    """Q8_K: d f32 @0, qs i8[256] @4, bsums i16[16] @260 (group sums of 16)."""
    qs = np.asarray(qs, dtype=np.int64)
    assert qs.shape == (256,) and qs.min() >= -128 and qs.max() <= 127
    b = np.zeros(292, dtype=np.uint8)
    b[0:4] = np.array([d], dtype=np.float32).view(np.uint8)
    b[4:260] = qs.astype(np.int8).view(np.uint8)
    b[260:292] = qs.reshape(16, 16).sum(axis=1).astype(np.int16).view(np.uint8)
    return b


def pack_q4k_scales(sc, m) -> np.ndarray:
    """The 12-byte 6-bit packing that q4k_scale_min (kquant.rs:83-92) unpacks."""
    s = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return s


def q4k_block(d_bits: int, dmin_bits: int, sc, m, q4) -> np.ndarray:
    """Q4_K: d f16 @0, dmin f16 @2, scales @4, qs @16; sub-block j holds
    elements 32j..32j+31 in the low (even j) or high (odd j) nibbles of
    qs[32*(j//2) ..]."""
    q4 = np.asarray(q4, dtype=np.int64)
    assert q4.shape == (256,) and q4.min() >= 0 and q4.max() <= 15
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    b[2:4] = np.array([dmin_bits], dtype=np.uint16).view(np.uint8)
    b[4:16] = pack_q4k_scales(sc, m)
    for c in range(4):
        lo, hi = q4[64 * c:64 * c + 32], q4[64 * c + 32:64 * c + 64]
        b[16 + 32 * c:16 + 32 * c + 32] = (lo | (hi << 4)).astype(np.uint8)
    return b


def q6k_block(d_bits: int, scales, q) -> np.ndarray:
    """Q6_K: ql @0, qh @128, scales i8 @192, d f16 @208; element 128h + 32p + l
    (plane p, l < 32) is ql nibble + 2 qh bits as kquant.rs:233-236 reads it."""
    q = np.asarray(q, dtype=np.int64)
    assert q.shape == (256,) and q.min() >= 0 and q.max() <= 63
    b = np.zeros(210, dtype=np.uint8)
    for h in range(2):
        e = q[128 * h:128 * h + 128]
        for l in range(32):
            q1, q2, q3, q4 = e[l], e[l + 32], e[l + 64], e[l + 96]
            b[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * h + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    return b


F16_ONE, F16_1024 = 0x3C00, 0x6400


def test_block_builders_match_the_oracle_unpackers(oracle):
    """The builders above are the inverse of the oracle's (already pinned)
    unpack and dequant: every scale/min slot and quant position lands where
    the oracle reads it."""
    O = oracle
    rng = np.random.default_rng(3)
    for _ in range(20):
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q4 = rng.integers(0, 16, 256)
        b = q4k_block(F16_ONE, F16_ONE, sc, m, q4)
        for j in range(8):
            assert O.q4k_scale_min(b[4:16], j) == (sc[j], m[j])
        want = np.array([sc[e // 32] * q4[e] - m[e // 32] for e in range(256)], dtype=np.float32)
        assert np.array_equal(O.dequant_q4k(b), want)
        s6, q = rng.integers(-128, 128, 16), rng.integers(0, 64, 256)
        b6 = q6k_block(F16_ONE, s6, q)
        want6 = np.array([s6[e // 16] * (q[e] - 32) for e in range(256)], dtype=np.float32)
        assert np.array_equal(O.dequant_q6k(b6), want6)


# ---- f32 helpers for the regroupings (numpy float32, one rounding per op) ------------


def chain(vals):
    s = F32(0)
    for v in vals:
        s = F32(s + F32(v))
    return s


def hsum256(a):
    """((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) in f32 (kquant.rs:512-522)."""
    a = [F32(v) for v in a]
    return F32(F32(F32(a[0] + a[4]) + F32(a[2] + a[6])) + F32(F32(a[1] + a[5]) + F32(a[3] + a[7])))


def round_f32(x: Fraction) -> float:
    """x rounded to the nearest f32, ties to even (exact rational input)."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    q = x / Fraction(2) ** (e - 23)  # 2^23 <= q < 2^24
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(Fraction(n) * Fraction(2) ** (e - 23))


def q4k_sub(b4, bx, j):
    """Exact integer sub-dot of Q4_K sub-block j (kquant.rs:200-211)."""
    q8 = bx[4:260].view(np.int8).astype(np.int64)
    qs = b4[16:144].astype(np.int64)
    c = qs[32 * (j // 2):32 * (j // 2) + 32]
    nib = (c >> 4) if j % 2 else (c & 15)
    return int((nib * q8[32 * j:32 * j + 32]).sum())


# ---- Q4_K scalar -----------------------------------------------------------------


def q4k_chain_case():
    """Sub-blocks 0-4 and 6-7 have scale 63 and sub-dot 32*15*(+-127); sub-block 5
    has scale 1 and sub-dot 1; d = 1, dmin = 0, x.d = 1 (the case below)."""
    q4 = np.zeros(256, dtype=np.int64)
    q8 = np.zeros(256, dtype=np.int64)
    for j in (0, 1, 2, 3, 4, 6, 7):
        q4[32 * j:32 * j + 32] = 15
        q8[32 * j:32 * j + 32] = 127 if j < 5 else -127
    q4[32 * 5], q8[32 * 5] = 1, 1
    sc = [63, 63, 63, 63, 63, 1, 63, 63]
    w = q4k_block(F16_ONE, 0, sc, [0] * 8, q4).reshape(1, 144)
    x = q8k_block(1.0, q8).reshape(1, 292)
    return w, x, sc


def test_q4k_scalar_sum_q_is_an_f32_chain_in_subblock_order(oracle):
    """sum_q += sc*sub for j = 0..7 in f32 (kquant.rs:212). With sc = 63 and
    sub = 32*15*127 = 60960, T = sc*sub = 3840480. Sub-blocks 0-4 give +T,
    sub-block 5 gives +1, sub-blocks 6-7 give -T; d = dmin-free, x.d = 1.
    5T = 19202400 lies in [2^24, 2^25) where the f32 spacing is 2; 5T + 1 is a
    tie between 19202400 and 19202402 and goes to the even significand,
    19202400; minus 2T is exact: 11521440. The exact integer sum (or any order
    that adds the 1 below 2^24) gives 11521441."""
    O = oracle
    T = 63 * 60960
    w, x, sc = q4k_chain_case()
    terms = [sc[j] * q4k_sub(w[0], x[0], j) for j in range(8)]
    assert terms == [T] * 5 + [1, -T, -T]
    got = O.dot(O.Q4K, O.ORDER_SCALAR, w, x)
    assert got == 11521440.0
    # regroupings: exact integer sum, reversed chain, pairwise halves
    assert float(F32(sum(terms))) != got
    assert float(chain(terms[::-1])) != got
    assert float(F32(chain(terms[:4]) + chain(terms[4:]))) != got


def test_q4k_scalar_one_sumf_update_per_block(oracle):
    """`sumf += d_all*sum_q - dmin_all*sum_m as f32` is one update per block
    (kquant.rs:215). Block 0 adds exactly 1 (sc = 1, sub = 1, dmin = 0).
    Block 1 has d = dmin = 1024, x.d = 1, sum_q = 32*1024 and
    sum_m = 8*32*128 = 32768, so both products are 2^25 and its contribution
    is exactly 0: the reference returns 1. Two updates (sumf += a; sumf -= b)
    absorb the 1 into 2^25 and return 0; keeping the min term apart and
    subtracting it after the block loop does the same."""
    O = oracle
    q4a, q8a = np.zeros(256, np.int64), np.zeros(256, np.int64)
    q4a[0], q8a[0] = 1, 1
    b0 = q4k_block(F16_ONE, 0, [1, 0, 0, 0, 0, 0, 0, 0], [0] * 8, q4a)
    q4b = np.zeros(256, np.int64)
    q4b[0:32] = 8
    b1 = q4k_block(F16_1024, F16_1024, [32, 0, 0, 0, 0, 0, 0, 0], [32] * 8, q4b)
    w = np.stack([b0, b1])
    x = np.stack([q8k_block(1.0, q8a), q8k_block(1.0, np.full(256, 4))])
    got = O.dot(O.Q4K, O.ORDER_SCALAR, w, x)
    assert got == 1.0
    a = [F32(1.0), F32(2.0 ** 25)]  # d_all * sum_q per block
    b = [F32(0.0), F32(2.0 ** 25)]  # dmin_all * sum_m per block
    two = F32(0)
    for ai, bi in zip(a, b):
        two = F32(F32(two + ai) - bi)
    assert two != got
    apart = F32(chain(a) - chain(b))
    assert apart != got


# ---- Q6_K scalar -----------------------------------------------------------------


def _q6k_chain_case():
    """Half 0: all 8 groups have scale 64 and group sum 16*(-32)*(-128) = 65536,
    so each term is 2^22 and the running sum reaches 2^25 exactly after the
    half. Half 1: groups 8, 9, 10 have scale 1 and group sum 1 (one quant 33
    against q8 = 1); the rest are zero. d = x.d = 1."""
    q = np.full(256, 32, dtype=np.int64)
    q8 = np.zeros(256, dtype=np.int64)
    q[0:128] = 0
    q8[0:128] = -128
    for g in (8, 9, 10):
        e = 16 * g
        q[e], q8[e] = 33, 1
    scales = [64] * 8 + [1] * 8
    return q6k_block(F16_ONE, scales, q).reshape(1, 210), q8k_block(1.0, q8).reshape(1, 292), scales


def test_q6k_scalar_sum_runs_across_both_halves(oracle):
    """`sum += sc[g] * group_sums[g]` is one f32 chain over both halves
    (kquant.rs:228-246, `sum` declared outside the half loop). After half 0 the
    chain holds 2^25, where the f32 spacing is 4, so each of the three +1 of
    half 1 rounds away: the reference returns 2^25. A sum per half added at the
    end (2^25 + 3 -> 2^25 + 4), or an integer sum, returns 33554436."""
    O = oracle
    w, x, scales = _q6k_chain_case()
    got = O.dot(O.Q6K, O.ORDER_SCALAR, w, x)
    assert got == 2.0 ** 25
    terms = [2 ** 22] * 8 + [1, 1, 1] + [0] * 5
    per_half = F32(chain(terms[:8]) + chain(terms[8:]))
    assert per_half == 2.0 ** 25 + 4 and per_half != got
    assert F32(sum(terms)) != got


def test_q6k_avx2_integer_sum_over_both_halves_then_one_fma(oracle):
    """dot_q6k_avx2 keeps the whole block in i32 lanes (kquant.rs:470-503), one
    fma per block, then hsum256. Lane k takes bytes 4k..4k+3 of each 32-byte
    plane; plane bytes 0-15 use scale 2n, bytes 16-31 scale 2n+1. Half 0 puts
    4*64*4*4096 = 2^22 in every lane. Half 1's three unit groups start at
    element 0 (group 8, lane 0), 16 (group 9, lane 4) and 32 (group 10, lane 0):
    a0 = 2^22 + 2, a4 = 2^22 + 1, other lanes 2^22, all exact. hsum:
    a0 + a4 = 2^23 + 3; + (a2 + a6) = 2^24 + 3, a tie at spacing 2 that goes to
    the even significand 2^24 + 4; + 2^24 = 2^25 + 4 = 33554436 (not the scalar
    order's 2^25, which the reference's tolerance allows)."""
    O = oracle
    w, x, _ = _q6k_chain_case()
    got = O.dot(O.Q6K, O.ORDER_AVX2, w, x)
    assert got == 2.0 ** 25 + 4
    lanes = [2 ** 22 + 2, 2 ** 22, 2 ** 22, 2 ** 22, 2 ** 22 + 1, 2 ** 22, 2 ** 22, 2 ** 22]
    assert hsum256(lanes) == got
    # an f32 chain over groups (the scalar order) or an adjacent-pair lane tree differ
    assert F32(chain([2 ** 22] * 8 + [1, 1, 1])) != got
    pairs = [F32(F32(lanes[i]) + F32(lanes[i + 1])) for i in range(0, 8, 2)]
    assert F32(F32(pairs[0] + pairs[1]) + F32(pairs[2] + pairs[3])) != got
    # the 4-wide kernel reproduces it per lane (kquant.rs:376-377)
    assert np.array_equal(O.dot_x4(O.Q6K, w, [x] * 4), np.full(4, got, np.float32))


# ---- Q4_K AVX2 ------------------------------------------------------------------


def test_q4k_avx2_min_term_kept_apart_and_subtracted_after_hsum(oracle):
    """dot_q4k_avx2 accumulates `acc_min += dmin * min_sum` in a scalar kept
    apart from the 8 lane accumulators and returns hsum256(acc) - acc_min
    (kquant.rs:279-280, 303). Block 0: quant 1 at sub-block element 8 (lane 2)
    against q8 = 1, sc = 1, d = 1, dmin = 0: a2 = 1. Block 1: elements 0-3 of
    sub-block 0 (lane 0) are 8 against q8 = 32 (the whole sub-block is 32),
    sc = 32, d = 1024: a0 = 1024*32*1024 = 2^25; dmin = 1024, m0 = 32,
    bsum pair 1024: acc_min = 2^25. hsum = (2^25 + 1) -> 2^25 at spacing 4,
    minus 2^25 = 0. Subtracting the min per block (a scalar-style sum), or
    from lane 0 before the hsum, keeps the 1 and returns 1."""
    O = oracle
    q4a, q8a = np.zeros(256, np.int64), np.zeros(256, np.int64)
    q4a[8], q8a[8] = 1, 1
    b0 = q4k_block(F16_ONE, 0, [1, 0, 0, 0, 0, 0, 0, 0], [0] * 8, q4a)
    q4b, q8b = np.zeros(256, np.int64), np.zeros(256, np.int64)
    q4b[0:4] = 8
    q8b[0:32] = 32
    b1 = q4k_block(F16_1024, F16_1024, [32, 0, 0, 0, 0, 0, 0, 0], [32, 0, 0, 0, 0, 0, 0, 0], q4b)
    w = np.stack([b0, b1])
    x = np.stack([q8k_block(1.0, q8a), q8k_block(1.0, q8b)])
    got = O.dot(O.Q4K, O.ORDER_AVX2, w, x)
    assert got == 0.0
    lanes = [F32(2.0 ** 25), 0, F32(1.0), 0, 0, 0, 0, 0]
    assert F32(hsum256(lanes) - F32(2.0 ** 25)) == got
    # regroupings
    per_block = F32(F32(F32(1.0) - F32(0.0)) + F32(F32(2.0 ** 25) - F32(2.0 ** 25)))
    assert per_block != got
    lane0 = list(lanes)
    lane0[0] = F32(lane0[0] - F32(2.0 ** 25))
    assert hsum256(lane0) != got
    assert np.array_equal(O.dot_x4(O.Q4K, w, [x] * 4), np.full(4, got, np.float32))
    # the scalar order on the same blocks is one update per block: 1
    assert O.dot(O.Q4K, O.ORDER_SCALAR, w, x) == 1.0


def _split4(n, wmax):
    """Four (w, x) pairs, |w| <= wmax, |x| <= 127, with sum w*x == n: three
    pairs (wmax, t) and the remainder over a (1, r) pair."""
    t = int(n / (3 * wmax))
    r = n - 3 * wmax * t
    assert abs(t) <= 127 and abs(r) <= 127, n
    return [(wmax, t)] * 3 + [(1, r)]


def _lane0_blocks(oracle, dtype, n, d_bits, xd):
    """One weight block and one activation block whose AVX2 lane 0 (bytes 0-3
    of every 32-byte vector) holds the integer sum n and every other lane 0;
    d_bits is the weight's f16 scale, xd the activation's."""
    O = oracle
    if dtype == O.Q8_0:
        pairs = _split4(n, 127)
        qw = [p[0] for p in pairs] + [0] * 28
        qx = [p[1] for p in pairs] + [0] * 28
        w = np.zeros(34, np.uint8)
        w[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
        w[2:] = np.array(qw, np.int8).view(np.uint8)
        x = np.zeros(34, np.uint8)
        x[0:2] = np.array([O.f32_to_f16(xd)], np.uint16).view(np.uint8)
        x[2:] = np.array(qx, np.int8).view(np.uint8)
        assert O.f16_to_f32(O.f32_to_f16(xd)) == xd
        return w, x
    # K-quants: sub-block / plane 0 carries 63*S0 (Q4_K) or 127*S0 (Q6_K), a
    # second one with scale 1 carries the rest; elements 0-3 of each only
    big = 63 if dtype == O.Q4K else 127
    s0 = int(n / big)
    rest = n - big * s0
    q8 = np.zeros(256, np.int64)
    if dtype == O.Q4K:
        q4 = np.zeros(256, np.int64)
        for base, s in ((0, s0), (64, rest)):  # sub-blocks 0 and 2 (low nibbles)
            for e, (a, b) in enumerate(_split4(s, 15)):
                q4[base + e], q8[base + e] = a, b
        return q4k_block(d_bits, 0, [big, 0, 1, 0, 0, 0, 0, 0], [0] * 8, q4), q8k_block(xd, q8)
    q = np.full(256, 32, np.int64)
    for base, s in ((0, s0), (128, rest)):  # plane 0 of each half
        for e, (a, b) in enumerate(_split4(s, 31)):
            q[base + e], q8[base + e] = 32 + a, b
    scales = [0] * 16
    scales[0], scales[8] = big, 1
    return q6k_block(d_bits, scales, q), q8k_block(xd, q8)


@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_avx2_dots_accumulate_with_fused_multiply_add(oracle, dtype):
    """The AVX2 dots accumulate `acc = _mm256_fmadd_ps(d, cvt(sumi), acc)`, one
    rounding per block (kernels.rs:277, kquant.rs:301, 505). Block 0 puts the
    integer -round(p) in lane 0 with d = 1, where p = d1*s is block 1's lane-0
    product (d1 = f16 scale times activation scale). fma(d1, s, -round(p)) is
    the rounding error of p, rounded once (computed here exactly with
    rationals); a separate multiply and add give 0."""
    O = oracle
    rng = np.random.default_rng(11 + dtype)
    for _ in range(200):
        dw = 1.0 + int(rng.integers(1, 64)) * 2.0 ** -10  # f16-exact, below 1.0625
        if dtype == O.Q8_0:
            dx = 1.0 + int(rng.integers(1, 64)) * 2.0 ** -10  # the activation scale is f16 too
            s = int(rng.integers(10000, 28000))
        else:
            dx = float(F32(1.0 + int(rng.integers(1, 2 ** 16)) * 2.0 ** -20))
            s = int(rng.integers(50000, 150000))
        d1 = float(F32(F32(dw) * F32(dx)))
        p = Fraction(d1) * s
        n0 = -round(p)
        fused = round_f32(p + n0)
        unfused = round_f32(Fraction(round_f32(p)) + n0)
        if fused != unfused and fused != 0.0:
            break
    else:
        raise AssertionError("no distinguishing case found")
    b0 = _lane0_blocks(O, dtype, n0, F16_ONE, 1.0)
    b1 = _lane0_blocks(O, dtype, s, O.f32_to_f16(dw), dx)
    w, x = np.stack([b0[0], b1[0]]), np.stack([b0[1], b1[1]])
    got = O.dot(dtype, O.ORDER_AVX2, w, x)
    assert got == fused and got != unfused
    assert np.array_equal(O.dot_x4(dtype, w, [x] * 4), np.full(4, got, np.float32))


# ---- float64 closed forms with an op-count error bound -------------------------------


def _exact_and_magnitude(O, dtype, w, x):
    """The dot in exact arithmetic over the block fields (integer sub-dots,
    f32 scale products as the reference forms them), and the sum of the
    magnitudes of every term the f32 steps round."""
    d, qs, bs = O.q8k_fields(x)
    exact, mag = Fraction(0), Fraction(0)
    for b in range(w.shape[0]):
        if dtype == O.Q4K:
            dw = O.f16_to_f32(int(w[b, 0:2].view(np.uint16)[0]))
            dm = O.f16_to_f32(int(w[b, 2:4].view(np.uint16)[0]))
            d_all, dmin_all = Fraction(float(F32(F32(dw) * d[b]))), Fraction(float(F32(F32(dm) * d[b])))
            sc_sub = []
            sum_m = 0
            for j in range(8):
                sc, m = O.q4k_scale_min(w[b, 4:16], j)
                sc_sub.append(sc * q4k_sub(w[b], x[b], j))
                sum_m += m * (int(bs[b, 2 * j]) + int(bs[b, 2 * j + 1]))
            exact += d_all * sum(sc_sub) - dmin_all * sum_m
            mag += abs(d_all) * sum(abs(t) for t in sc_sub) + abs(dmin_all) * abs(sum_m)
        else:
            dw = O.f16_to_f32(int(w[b, 208:210].view(np.uint16)[0]))
            d_all = Fraction(float(F32(F32(dw) * d[b])))
            sums = O.block_sums(O.Q6K, w[b:b + 1], x[b:b + 1])
            scales = w[b, 192:208].view(np.int8).astype(np.int64)
            terms = [int(scales[g]) * int(sums[g]) for g in range(16)]
            exact += d_all * sum(terms)
            mag += abs(d_all) * sum(abs(t) for t in terms)
    return exact, mag


@pytest.mark.parametrize("dtype,seed", [(2, 141), (3, 151)])
@pytest.mark.parametrize("order", [0, 1])
def test_kquant_dot_within_op_count_bound_of_exact(oracle, dtype, seed, order):
    """Against the exact value, the f32 result errs by at most gamma_k * M,
    where M sums the magnitudes of the rounded terms and k counts the roundings
    on the longest chain: the block's own steps (Q4_K: 8 chain adds, 3 products,
    1 subtraction, the int->f32 of sum_m; Q6_K: 16 chain adds, 1 product; AVX2:
    1 fma, 3 hsum levels, the acc_min chain) plus one add per block. The bound
    is ~1e-6 relative for these sizes; an f16-rounded Q8_K scale (relative
    error up to 2^-11) breaks it, as the planted copy below shows."""
    O = oracle
    rng = O.Rng(seed)
    for blocks in (1, 3, 12, 38):
        w = O.quantize_weights_ref(dtype, rng.adversarial(blocks * 256))
        x = O.quantize_q8k(rng.vec(blocks * 256))
        got = Fraction(O.dot(dtype, order, w, x))
        exact, mag = _exact_and_magnitude(O, dtype, w, x)
        k = blocks + (16 if dtype == O.Q4K else 18) + 4
        bound = Fraction(k) * Fraction(U) / (1 - k * Fraction(U)) * mag
        assert abs(got - exact) <= bound, (blocks, float(abs(got - exact) / mag))
        # the same bound fails for a Q8_K whose scale was stored as f16 (up to 12
        # blocks; over 38 the per-block errors of random sign partly cancel)
        xf = x.copy()
        d16 = np.float32(np.float16(xf[:, 0:4].copy().view(np.float32).ravel()))
        xf[:, 0:4] = d16.reshape(-1, 1).view(np.uint8)
        planted = Fraction(O.dot(dtype, order, w, xf))
        if blocks <= 12:
            assert abs(planted - exact) > bound, blocks


def test_q4k_scalar_block_step_is_not_contracted(oracle):
    """`d_all * sum_q - dmin_all * sum_m as f32` rounds both products before the
    subtraction (Rust never fuses). With one block, sumf = 0 + that value
    exactly. The case below is searched so that a fused form,
    fma(d_all, sum_q, -(dmin_all * sum_m)), rounds differently (computed with
    rationals)."""
    O = oracle
    rng = np.random.default_rng(29)
    while True:
        dw = 1.0 + int(rng.integers(1, 1024)) * 2.0 ** -10
        dm = 1.0 + int(rng.integers(1, 1024)) * 2.0 ** -10
        xd = float(F32(1.0 + int(rng.integers(1, 2 ** 20)) * 2.0 ** -20))
        sub = int(rng.integers(1000, 15 * 127 * 32))
        sm = int(rng.integers(1000, 63 * 127 * 32))
        d_all, dmin_all = float(F32(F32(dw) * F32(xd))), float(F32(F32(dm) * F32(xd)))
        a = round_f32(Fraction(d_all) * sub)
        b = round_f32(Fraction(dmin_all) * sm)
        plain = round_f32(Fraction(a) - Fraction(b))
        fused = round_f32(Fraction(d_all) * sub - Fraction(b))
        if plain != fused:
            break
    q4, q8 = np.zeros(256, np.int64), np.zeros(256, np.int64)
    # sub-block 0: sub = sum of q4*q8 over its 32 elements (sc0 = 1)
    q4[0:31] = 15
    per = sub // (15 * 30)
    q8[0:30] = per
    left = sub - 15 * 30 * per  # 0 <= left < 450
    q8[30] = left // 15
    q4[31], q8[31] = 1, left % 15
    assert abs(int(q8[31])) <= 127 and int((q4[0:32] * q8[0:32]).sum()) == sub
    # sub-block 1 (q4 = 0) carries the mins: m1 = 63, bsum pair = sm / 63 rounded,
    # with the rest of sum_m taken by sub-block 2 (m2 = 1)
    pair = sm // 63
    rest = sm - 63 * pair
    vals = np.zeros(32, np.int64)
    vals[:] = pair // 32
    vals[0] += pair - 32 * (pair // 32)
    q8[32:64] = vals
    q8[64] = rest
    assert np.abs(q8).max() <= 127
    w = q4k_block(O.f32_to_f16(dw), O.f32_to_f16(dm), [1, 0, 0, 0, 0, 0, 0, 0], [0, 63, 1, 0, 0, 0, 0, 0], q4)
    x = q8k_block(xd, q8)
    got = O.dot(O.Q4K, O.ORDER_SCALAR, w.reshape(1, 144), x.reshape(1, 292))
    assert got == plain and got != fused
