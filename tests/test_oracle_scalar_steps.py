"""Step pins for the oracle's Q8_0 / Q6_K scalar dots and both activation
quantizers -- CPU only.

Each test builds a block whose result under the reference's f32 steps is
derived by hand in its docstring (exact rationals, every rounding stated),
checks the derivation with exact rational arithmetic (``round_f32``, an
f32 round-to-nearest-even written from the definition), asserts the oracle
returns exactly that, and evaluates the plausible slips on the same block to
show that each gives another value. Reference steps:

  dot_q8_scalar  kernels.rs:72-82   `sum += acc as f32 * bw.scale() * bx.scale()`,
                                    left to right: ((acc * dw) * dx)
  dot_q6k_scalar kquant.rs:220-250  `d_all = f16_to_f32(d) * x.d` first, then
                                    `sumf += d_all * sum`
  q8::quantize   q8.rs:27-44        `d = f16(amax / 127.0)`, `inv = 1/d`,
                                    `x = v * inv`, `(x +- 0.5) as i32` (trunc),
                                    `clamp(-127, 127)`
  quantize_q8k   kquant.rs:145-187  `iscale = -128/max`, `nearest_int(iscale*v)`
                                    ((v +- 0.5) as i32, ties away from zero),
                                    `.min(127)`, `d = 1/iscale`
  dot_f16_f16c   kernels.rs:174-201 lane i takes elements 8c + i, one fmadd per
                                    chunk, hsum ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7)),
                                    tail added after in scalar
  axpy_f16_f16c  kernels.rs:203-220 one fmadd per element of whole chunks, tail
                                    `out += a * v` (two roundings)
"""
from fractions import Fraction as Fr

import numpy as np

from tests.test_oracle_kquant_order import q6k_block, q8k_block, round_f32

F32 = np.float32


def f32(x) -> float:
    return float(F32(x))


def q8_0_block(d_bits: int, qs) -> np.ndarray:
    """Q8_0: d f16 @0, qs i8[32] @2 (q8.rs:9-17)."""
    qs = list(qs) + [0] * (32 - len(qs))
    b = np.zeros(34, dtype=np.uint8)
    b[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    b[2:] = np.array(qs, dtype=np.int8).view(np.uint8)
    return b


def trunc_q(r: float, lo: int, hi: int) -> int:
    """`r as i32` (toward zero), then clamp."""
    return max(lo, min(hi, int(np.trunc(r))))


def round_half(x: float) -> float:
    """`if x >= 0 { x + 0.5 } else { x - 0.5 }` in f32."""
    x = F32(x)
    return f32(x + F32(0.5)) if x >= 0 else f32(x - F32(0.5))


# ---- dot_q8_scalar ------------------------------------------------------------------


def test_q8_scalar_contribution_is_acc_times_dw_then_dx(oracle):
    """One block, acc = 127*127 + 127*2 = 16383, dw = 1 + 2^-10 (f16 0x3C01),
    dx = 1 + 2^-9 (0x3C02).
    Reference, (acc*dw)*dx:
      acc*dw = 16383 + 16383/1024 = 16398 + 1023/1024. In [2^14, 2^15) the
      f32 spacing is 2^-9, and 1023/1024 is 511.5 spacings: a tie between
      16398 + 511/512 (odd significand) and 16399 (even) -> 16399.
      16399*dx = 16399 + 16399/512 = 16431 + 15/512, exact -> 16431.029296875.
    Slips:
      acc*(dw*dx): dw*dx = 1 + 3*2^-10 + 2^-19 (exact); times 16383 is
      16431 + 14.4990...*2^-9 -> 16431 + 14/512 = 16431.02734375.
      (acc*dx)*dw: 16383*dx = 16414 + 511/512 (exact); times dw is the same
      real number as above -> 16431.02734375."""
    O = oracle
    w = q8_0_block(0x3C01, [127, 127]).reshape(1, 34)
    x = q8_0_block(0x3C02, [127, 2]).reshape(1, 34)
    acc, dw, dx = Fr(16383), Fr(1) + Fr(1, 1024), Fr(1) + Fr(1, 512)
    assert O.f16_to_f32(0x3C01) == float(dw) and O.f16_to_f32(0x3C02) == float(dx)
    step1 = round_f32(acc * dw)
    assert step1 == 16399.0
    ref = round_f32(Fr(step1) * dx)
    assert ref == 16431 + 15 / 512
    got = O.dot(O.Q8_0, O.ORDER_SCALAR, w, x)
    assert got == ref
    slip_a = round_f32(acc * Fr(round_f32(dw * dx)))
    slip_b = round_f32(Fr(round_f32(acc * dx)) * dw)
    assert slip_a == slip_b == 16431 + 14 / 512
    assert slip_a != got
    # the same slips in numpy float32
    assert f32(F32(16383) * F32(F32(dw) * F32(dx))) != got
    assert f32(F32(F32(16383) * F32(dx)) * F32(dw)) != got


def test_q8_scalar_contributions_chain_with_dx_not_one(oracle):
    """Two blocks: block 0 is the block above (16431 + 15/512); block 1 has
    acc = 1, dw = dx = 1 + 2^-10, so its contribution is
    f32(f32(1 + 2^-10) * (1 + 2^-10)) = 1 + 2^-9 + 2^-20 (exact).
    sum = 16431 + 15/512 + 1 + 2^-9 + 2^-20 = 16432 + 16/512 + 2^-20; the
    2^-20 is below half the 2^-9 spacing -> 16432.03125. With the slip
    acc*(dw*dx) in block 0 the sum is 16432 + 15/512 + 2^-20 -> 16432.029296875."""
    O = oracle
    w = np.stack([q8_0_block(0x3C01, [127, 127]), q8_0_block(0x3C01, [1])])
    x = np.stack([q8_0_block(0x3C02, [127, 2]), q8_0_block(0x3C01, [1])])
    got = O.dot(O.Q8_0, O.ORDER_SCALAR, w, x)
    assert got == 16432.03125
    slip = f32(F32(16431 + 14 / 512) + F32(1 + 2.0 ** -9 + 2.0 ** -20))
    assert slip == 16432 + 15 / 512 and slip != got


# ---- dot_q6k_scalar -------------------------------------------------------------------


def test_q6k_scalar_d_all_is_formed_before_the_sum(oracle):
    """One block: group 0 has scale 127 and group sum (q-32)*q8 = 1*127 + 1*2
    = 129; every other quant is 32 (zero) -> sum = 16383 exactly.
    d = 1 + 2^-10 (f16 0x3C01), x.d = 1 + 2^-10 (f32).
    Reference: d_all = (1 + 2^-10)^2 = 1 + 2^-9 + 2^-20 (exact);
      d_all*16383 = 16383 + 16383/512 + 16383/2^20 = 16415 + 6.9992*2^-9
      -> 16415 + 7/512 = 16415.013671875; sumf = 0 + that.
    Slips:
      d*(x.d*sum): x.d*16383 = 16398 + 1023/1024 -> tie -> 16399 (even);
      times d: 16399 + 16399/1024 = 16415 + 7.5*2^-9, a tie between 7/512
      (odd) and 8/512 (even) -> 16415.015625.
      (d*sum)*x.d: the same by symmetry -> 16415.015625."""
    O = oracle
    q = np.full(256, 32, dtype=np.int64)
    q8 = np.zeros(256, dtype=np.int64)
    q[0], q8[0] = 33, 127
    q[1], q8[1] = 33, 2
    xd = 1 + 2.0 ** -10
    w = q6k_block(0x3C01, [127] + [0] * 15, q).reshape(1, 210)
    x = q8k_block(xd, q8).reshape(1, 292)
    d = Fr(1) + Fr(1, 1024)
    d_all = round_f32(d * Fr(xd))
    assert d_all == 1 + 2.0 ** -9 + 2.0 ** -20
    ref = round_f32(Fr(d_all) * 16383)
    assert ref == 16415 + 7 / 512
    got = O.dot(O.Q6K, O.ORDER_SCALAR, w, x)
    assert got == ref
    slip_a = round_f32(d * Fr(round_f32(Fr(xd) * 16383)))
    slip_b = round_f32(Fr(round_f32(d * 16383)) * Fr(xd))
    assert slip_a == slip_b == 16415 + 8 / 512
    assert slip_a != got
    assert f32(F32(d) * F32(F32(xd) * F32(16383))) != got


# ---- q8::quantize ---------------------------------------------------------------------


def test_q8_0_quantize_rounds_ties_away_and_adds_half_in_f32(oracle):
    """amax = 127 -> d = f16(127/127) = 1.0 (0x3C00), inv = 1.
      v = 2.5:   x + 0.5 = 3.0 -> 3  (round-half-even, rintf, gives 2)
      v = -2.5:  x - 0.5 = -3.0 -> -3 (rintf: -2)
      v = 0.5 - 2^-25 (largest f32 below 0.5): x + 0.5 = 1 - 2^-25, which is
                 a tie between 1 - 2^-24 (odd) and 1.0 (even) -> 1.0 -> 1
                 (roundf and any correctly rounded x -> 0)
      v = -(0.5 - 2^-25): -> -1.
      v = 1.5 - 2^-23: x + 0.5 = 2 - 2^-23, exact -> 1."""
    O = oracle
    near = 0.5 - 2.0 ** -25
    src = np.zeros(32, dtype=np.float32)
    src[:6] = [127.0, 2.5, -2.5, near, -near, 1.5 - 2.0 ** -23]
    assert F32(near) == near and round_half(near) == 1.0
    blk = O.quantize_q8_0(src).reshape(-1)
    assert int(blk[0]) | int(blk[1]) << 8 == 0x3C00
    qs = blk[2:].view(np.int8)
    assert list(qs[:6]) == [127, 3, -3, 1, -1, 1]
    assert not qs[6:].any()
    # slips: rintf and roundf
    assert [int(np.rint(v)) for v in src[1:5]] != [3, -3, 1, -1]
    assert int(np.round(near)) == 0 and int(np.floor(near + 0.5)) == 0


def test_q8_0_quantize_clamps_at_minus_127_with_a_subnormal_scale(oracle):
    """amax = 177*2^-24 (the element is negative). amax/127 = 1.394*2^-24 in
    f32, a subnormal f16 of 1.394 units of 2^-24, which rounds (half-up rule
    of f16.rs:43-47) to one unit: d = 2^-24 (0x0001), inv = 2^24 exactly.
    x = -177, x - 0.5 = -177.5, as i32 = -177, clamp -> -127.
    A -128 clamp gives -128 (0x80)."""
    O = oracle
    src = np.zeros(32, dtype=np.float32)
    src[3] = -177 * 2.0 ** -24
    assert O.f32_to_f16(f32(F32(src[3]) / F32(-127))) & 0x7FFF == 0x0001
    blk = O.quantize_q8_0(src).reshape(-1)
    assert int(blk[0]) | int(blk[1]) << 8 == 0x0001
    qs = blk[2:].view(np.int8)
    assert qs[3] == -127 and not np.delete(qs, 3).any()
    assert trunc_q(round_half(-177.0), -128, 127) == -128  # the slip


def test_q8_0_quantize_multiplies_by_the_inverse_scale(oracle):
    """amax = 127*33/32 = 130.96875 -> amax/127 = 33/32 exactly -> d = 1.03125
    (f16 0x3C20). inv = f32(32/33): 2^24*32/33 = 16268815.515..., rounded up
    to 16268816, so inv = 32/33 + (16/33)*2^-24.
    v = 15.984375 - 2^-20 (15.5*d less one f32 spacing):
      reference x = v*inv = 15.5 - (32/33)*2^-20 + 15.98*(16/33)*2^-24
                 = 15.5 - 0.485*2^-20 -> 15.5 (spacing 2^-20 in [8, 16));
                 x + 0.5 = 16 -> 16.
      slip x = v/d = 15.5 - 0.970*2^-20 -> 15.5 - 2^-20; + 0.5 = 16 - 2^-20
                 (exact) -> 15."""
    O = oracle
    d = Fr(33, 32)
    v = Fr(15984375, 10 ** 6) - Fr(1, 2 ** 20)
    assert Fr(f32(float(v))) == v
    src = np.zeros(32, dtype=np.float32)
    src[0], src[1] = 130.96875, float(v)
    inv = round_f32(1 / d)
    assert Fr(inv) == Fr(32, 33) + Fr(16, 33) / 2 ** 24
    x_ref = round_f32(v * Fr(inv))
    assert x_ref == 15.5
    blk = O.quantize_q8_0(src).reshape(-1)
    assert int(blk[0]) | int(blk[1]) << 8 == 0x3C20
    qs = blk[2:].view(np.int8)
    assert qs[0] == 127 and qs[1] == 16
    x_slip = round_f32(v / d)
    assert x_slip == 15.5 - 2.0 ** -20
    assert trunc_q(round_half(x_slip), -127, 127) == 15


def test_q8_0_quantize_scale_is_amax_divided_by_127(oracle):
    """amax = 127*(1 + 2^-11) + 2^-17 (one f32 spacing above 127*(1 + 2^-11)).
    Reference: amax/127 = 1 + 2^-11 + (64/127)*2^-23 -> rounds up (0.504 of a
    spacing) to 1 + 2^-11 + 2^-23, just above the f16 midpoint between
    0x3C00 and 0x3C01 -> d = 0x3C01.
    Slip amax*f32(1/127): f32(1/127) = 8454660*2^-30 = 1/127 - 0.0315*2^-30,
    so the product is 1 + 2^-11 + 0.473*2^-23 -> 1 + 2^-11 exactly, the
    midpoint itself, which rounds to the even f16 0x3C00."""
    O = oracle
    amax = Fr(127) * (1 + Fr(1, 2048)) + Fr(1, 2 ** 17)
    assert Fr(f32(float(amax))) == amax
    q = round_f32(amax / 127)
    assert q == 1 + 2.0 ** -11 + 2.0 ** -23
    r127 = round_f32(Fr(1, 127))
    assert Fr(r127) == Fr(8454660, 2 ** 30)
    slip = round_f32(amax * Fr(r127))
    assert slip == 1 + 2.0 ** -11
    assert O.f32_to_f16(q) == 0x3C01 and O.f32_to_f16(slip) == 0x3C00
    src = np.zeros(32, dtype=np.float32)
    src[7] = float(amax)
    blk = O.quantize_q8_0(src).reshape(-1)
    assert int(blk[0]) | int(blk[1]) << 8 == 0x3C01


# ---- quantize_q8k ---------------------------------------------------------------------


def test_q8k_nearest_int_ties_away_and_adds_half_in_f32(oracle):
    """max = -128 (the first largest |v|) -> iscale = -128/-128 = 1, d = 1/1 = 1.
      v = 2.5 -> nearest_int(2.5) = 3 (rintf: 2); v = -2.5 -> -3 (rintf: -2);
      v = 0.5 - 2^-25 -> (v + 0.5) = 1.0 in f32 (tie to even) -> 1 (roundf: 0);
      v = -(0.5 - 2^-25) -> -1."""
    O = oracle
    near = 0.5 - 2.0 ** -25
    src = np.zeros(256, dtype=np.float32)
    src[:5] = [-128.0, 2.5, -2.5, near, -near]
    blk = O.quantize_q8k(src).reshape(-1)
    d, qs, bsums = O.q8k_fields(blk.reshape(1, 292))
    assert float(d[0]) == 1.0
    assert list(qs[0, :5]) == [-128, 3, -3, 1, -1]
    assert not qs[0, 5:].any()
    assert bsums[0, 0] == -128
    assert [int(np.rint(v)) for v in src[1:5]] != [3, -3, 1, -1]
    assert int(np.round(near)) == 0


def test_q8k_scale_and_quants_come_from_iscale(oracle):
    """max = 7 -> iscale = f32(-128/7): 128/7 * 2^19 = 9586980.571..., rounded
    to 9586981, so |iscale| = 128/7 + (3/7)*2^-19.
    d = 1/iscale = -(7/128)*(1 - 4.47e-8) = -(7/128 - 0.656*2^-28) ->
    -(7/128 - 2^-28) = -0.0546874962747097 (spacing 2^-28 in [2^-5, 2^-4)).
    The slip d = max/-128 is -7/128 = -0.0546875 exactly.
    v = -(6.91796875 - 2^-21) (126.5*7/128 less one f32 spacing):
      iscale*v = 126.5 - (128/7)*2^-21 + 6.918*(3/7)*2^-19
               = 126.5 - 1.606*2^-19 -> 126.5 (spacing 2^-17);
               nearest_int -> 127.
      slip v/(max/-128) = 126.5 - 4.571*2^-19 -> 126.5 - 2^-17;
               + 0.5 = 127 - 2^-17 (exact) -> 126.
    The max itself: iscale*7 = -128 - 3*2^-19 -> -128 -> -128."""
    O = oracle
    isc = round_f32(Fr(-128, 7))
    assert Fr(isc) == -Fr(9586981, 2 ** 19)
    d_ref = round_f32(1 / Fr(isc))
    assert d_ref == -(7 / 128 - 2.0 ** -28)
    v = -(Fr(88550, 12800) - Fr(1, 2 ** 21))
    assert v == -(Fr(1265, 10) * 7 / 128 - Fr(1, 2 ** 21)) and Fr(f32(float(v))) == v
    assert round_f32(Fr(isc) * v) == 126.5
    slip_x = round_f32(v / Fr(-7, 128))
    assert slip_x == 126.5 - 2.0 ** -17
    assert trunc_q(round_half(slip_x), -1000, 127) == 126
    src = np.zeros(256, dtype=np.float32)
    src[0], src[1] = 7.0, float(v)
    blk = O.quantize_q8k(src).reshape(1, 292)
    d, qs, _ = O.q8k_fields(blk)
    assert float(d[0]) == d_ref and float(d[0]) != -7 / 128
    assert qs[0, 0] == -128 and qs[0, 1] == 127


# ---- dot_f16_f16c / axpy_f16_f16c (the x86 host's attention kernels) ---------------


def f16_bits(vals):
    import oracle as O

    out = np.array([O.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert all(O.f16_to_f32(int(b)) == float(v) for b, v in zip(out, vals)), "values must be exact f16"
    return out


def test_dot_f16_f16c_lanes_and_hsum_tree(oracle):
    """kernels.rs:174-201: lane i of the accumulator takes elements 8c + i; the
    halves are added (lane i + lane i+4), then movehl and add_ss:
    ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). Elements: k0*q0 = 2^15 * 2^10 = 2^25
    (lane 0), k1*q1 = 1 (lane 1), k4*q4 = -2^25 (lane 4). The tree cancels
    a0 + a4 first and returns 1. The scalar kernel (element order) reaches
    2^25 + 1, which rounds to 2^25 (spacing 4), and returns 0; a sequential
    lane sum does the same."""
    O = oracle
    k = f16_bits([2.0 ** 15, 1, 0, 0, -(2.0 ** 15), 0, 0, 0])
    q = np.array([1024, 1, 0, 0, 1024, 0, 0, 0], np.float32)
    assert O.dot_f16(O.ORDER_AVX2, k, q) == 1.0
    assert O.dot_f16(O.ORDER_SCALAR, k, q) == 0.0
    lanes = [2.0 ** 25, 1, 0, 0, -(2.0 ** 25), 0, 0, 0]
    seq = F32(0)
    for v in lanes:
        seq = F32(seq + F32(v))
    assert float(seq) == 0.0


def test_dot_f16_f16c_fuses_each_chunk_and_adds_the_tail_after(oracle):
    """One fmadd per 8-element chunk and lane: lane 0 holds k0*q0 = -1 after
    chunk 0, then fma(k8, q8, -1) with k8 = 1 + 2^-10 (f16 0x3C01) and
    q8 = 1 + 2^-14: the exact product is 1 + 2^-10 + 2^-14 + 2^-24, and one
    rounding of the sum leaves 2^-10 + 2^-14 + 2^-24 (15 significant bits,
    exact). Multiply-then-add first rounds the product to 1 + 2^-10 + 2^-14
    (2^-24 is half a spacing, tie to even) and returns 2^-10 + 2^-14: the
    scalar kernel's value. With n = 17 the tail element 16 (k = 2^-10,
    q = -1) is added after the hsum, in scalar: 2^-14 + 2^-24."""
    O = oracle
    k = np.zeros(16, np.uint16)
    q = np.zeros(16, np.float32)
    k[0], q[0] = f16_bits([-1.0])[0], 1.0
    k[8], q[8] = 0x3C01, 1 + 2.0 ** -14
    fused = 2.0 ** -10 + 2.0 ** -14 + 2.0 ** -24
    assert O.dot_f16(O.ORDER_AVX2, k, q) == fused
    assert O.dot_f16(O.ORDER_SCALAR, k, q) == 2.0 ** -10 + 2.0 ** -14
    k17 = np.concatenate([k, f16_bits([2.0 ** -10])])
    q17 = np.concatenate([q, np.array([-1.0], np.float32)])
    assert O.dot_f16(O.ORDER_AVX2, k17, q17) == 2.0 ** -14 + 2.0 ** -24


def test_axpy_f16_f16c_fuses_whole_chunks_only(oracle):
    """kernels.rs:203-220: out = fmadd(a, f32(v), out) for each element of the
    whole 8-element chunks, the tail out += a * f32(v) in scalar. With
    a = 1 + 2^-14, v = 1 + 2^-10 (0x3C01) and out = -1: fused
    2^-10 + 2^-14 + 2^-24, unfused 2^-10 + 2^-14 (see above). Nine elements:
    the first eight are fused, the ninth (the tail) is not."""
    O = oracle
    a = 1 + 2.0 ** -14
    v = np.full(9, 0x3C01, np.uint16)
    out = np.full(9, -1.0, np.float32)
    got = O.axpy_f16(O.ORDER_AVX2, out, a, v)
    fused, unfused = 2.0 ** -10 + 2.0 ** -14 + 2.0 ** -24, 2.0 ** -10 + 2.0 ** -14
    assert list(got[:8]) == [fused] * 8 and got[8] == unfused
    assert np.all(O.axpy_f16(O.ORDER_SCALAR, out, a, v) == unfused)


def test_f16c_kernels_within_the_reference_tolerance(oracle):
    """On random rows both orders agree with the float64 closed form well
    inside f32 accuracy (the reference's attention tests are tolerance-only,
    tests/kernels.rs:130-226)."""
    O = oracle
    rng = np.random.default_rng(9)
    for n in (8, 64, 67, 128):
        kf = rng.normal(0, 1, n).astype(np.float32)
        k = np.array([O.f32_to_f16(float(x)) for x in kf], np.uint16)
        kd = O.f16_to_f32_array(k).astype(np.float64)
        q = rng.normal(0, 1, n).astype(np.float32)
        want = float(np.dot(kd, q.astype(np.float64)))
        bound = 4 * n * 2.0 ** -24 * float(np.dot(np.abs(kd), np.abs(q.astype(np.float64))))
        for order in (O.ORDER_SCALAR, O.ORDER_AVX2):
            assert abs(O.dot_f16(order, k, q) - want) <= bound
        out = rng.normal(0, 1, n).astype(np.float32)
        a = float(rng.normal())
        want_o = out.astype(np.float64) + a * kd
        for order in (O.ORDER_SCALAR, O.ORDER_AVX2):
            got = O.axpy_f16(order, out, np.float32(a), k).astype(np.float64)
            assert np.all(np.abs(got - want_o) <= 2.0 ** -22 * (np.abs(out) + np.abs(a * kd)) + 1e-30)
