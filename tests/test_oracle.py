"""Pins of the CPU oracle (oracle/nrq_oracle.c) — CPU only.

The reference (Rust) cannot be built or run here, so the oracle is pinned by
(1) the reference tests' own known values and properties, restated with the
same seeds and tolerances (crates/nr-tensor/tests/kernels.rs, tests/kquant.rs),
(2) independent references the mathematics fixes (IEEE f16 via numpy,
brute-force integer dots, f64 closed forms), and (3) order-sensitive inputs
that only the reference's documented f32 order passes.
"""
import numpy as np
import pytest

# ---- f16 (f16.rs) ------------------------------------------------------------


def test_f16_known_values(oracle):
    """tests/kernels.rs:43-58"""
    O = oracle
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0xC000) == -2.0
    assert O.f16_to_f32(0x3800) == 0.5
    assert O.f16_to_f32(0x7BFF) == 65504.0
    assert O.f16_to_f32(0x0001) == np.float32(5.9604645e-8)
    assert O.f16_to_f32(0x0000) == 0.0
    assert np.isinf(O.f16_to_f32(0x7C00))
    assert np.isnan(O.f16_to_f32(0x7E00))
    assert O.f32_to_f16(1.0) == 0x3C00
    assert O.f32_to_f16(-2.0) == 0xC000
    assert O.f32_to_f16(65504.0) == 0x7BFF
    assert O.f32_to_f16(1e30) == 0x7C00


def test_f16_roundtrip_normals(oracle):
    """tests/kernels.rs:60-69: every normal finite f16 round-trips."""
    for bits in range(0x0400, 0x7C00):
        for sign in (0, 0x8000):
            b = bits | sign
            assert oracle.f32_to_f16(oracle.f16_to_f32(b)) == b, hex(b)


def test_f16_to_f32_matches_ieee_all_patterns(oracle):
    """f16_to_f32 equals IEEE binary16 decoding (numpy) for all 65536 patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32_array(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rounding(oracle):
    """Normals round to nearest even (== IEEE/numpy); subnormals round half up
    (f16.rs:43-47), which differs from IEEE only on exact ties."""
    rng = np.random.default_rng(5)
    # normal range: random f32 in [2^-14, 65504]
    v = (rng.uniform(-14, 15.99, 4000)).astype(np.float32)
    vals = (np.float32(2.0) ** v) * rng.choice([-1, 1], 4000).astype(np.float32)
    for x in vals:
        assert oracle.f32_to_f16(float(x)) == int(np.float32(x).astype(np.float16).view(np.uint16)), x
    # subnormal non-ties agree with IEEE
    sub = (rng.uniform(0.01, 1023.99, 2000) * 2.0 ** -24).astype(np.float32)
    for x in sub:
        k = float(x) / 2.0 ** -24
        if abs(k - round(k) - 0.5) < 1e-3 or abs(k - int(k) - 0.5) < 1e-6:
            continue
        assert oracle.f32_to_f16(float(x)) == int(np.float32(x).astype(np.float16).view(np.uint16)), x
    # subnormal exact ties round up (away from zero in magnitude)
    for k in (0, 1, 2, 3, 100, 1022):
        x = (k + 0.5) * 2.0 ** -24
        assert oracle.f32_to_f16(x) == k + 1
        assert oracle.f32_to_f16(-x) == 0x8000 | (k + 1)
    # below 2^-25 flushes to signed zero; NaN keeps the quiet bit
    assert oracle.f32_to_f16(2.0 ** -26) == 0
    assert oracle.f32_to_f16(-(2.0 ** -26)) == 0x8000
    assert oracle.f32_to_f16(float("nan")) & 0x7E00 == 0x7E00


# ---- activation quantizers ----------------------------------------------------


def test_quantize_error_bound(oracle):
    """tests/kernels.rs:71-82"""
    x = oracle.Rng(7).vec(1024)
    blocks = oracle.quantize_q8_0(x)
    back = oracle.dequantize_q8_0(blocks)
    d = oracle.f16_to_f32_array(blocks[:, 0:2].copy().view(np.uint16).ravel())
    scale = np.repeat(d, 32)
    assert np.all(np.abs(x - back) <= scale * 0.5 + 1e-6)


def test_quantize_q8_0_max_element_hits_127(oracle):
    """amax / d = 127 up to f16 rounding: the largest element lands on +-127."""
    rng = np.random.default_rng(1)
    x = rng.normal(size=32 * 64).astype(np.float32)
    blocks = oracle.quantize_q8_0(x)
    qs = blocks[:, 2:].view(np.int8)
    for b in range(64):
        i = np.argmax(np.abs(x[b * 32:(b + 1) * 32]))
        assert abs(int(qs[b, i])) >= 126
        assert np.sign(qs[b, i]) == np.sign(x[b * 32 + i])
    assert np.abs(qs).max() <= 127


def test_q8k_quantization_properties(oracle):
    """tests/kquant.rs:54-76: bsums are exact group sums; error <= d/2."""
    rng = oracle.Rng(11)
    for src in (rng.vec(512), rng.adversarial(512)):
        blocks = oracle.quantize_q8k(src)
        d, qs, bsums = oracle.q8k_fields(blocks)
        for b in range(blocks.shape[0]):
            q = qs[b].astype(np.int32)
            assert np.array_equal(q.reshape(16, 16).sum(axis=1), bsums[b].astype(np.int32))
            back = q.astype(np.float32) * d[b]
            assert np.all(np.abs(back - src[b * 256:(b + 1) * 256]) <= abs(d[b]) * 0.5 + 1e-6)


def test_q8k_first_max_maps_to_minus_128(oracle):
    """iscale = -128/max at the first largest |v| (kquant.rs:162-176)."""
    x = np.zeros(256, dtype=np.float32)
    x[3], x[9] = -2.0, 2.0  # equal |v|: the first one (index 3) is `max`
    blocks = oracle.quantize_q8k(x)
    d, qs, _ = oracle.q8k_fields(blocks)
    assert qs[0, 3] == -128 and qs[0, 9] == 127  # 128 clamps to 127 (upper clamp only)
    assert d[0] == np.float32(1.0) / (np.float32(-128.0) / np.float32(-2.0))
    zero = oracle.quantize_q8k(np.zeros(256, dtype=np.float32))
    assert not zero.any()


# ---- K-quant packing --------------------------------------------------------------


def test_q4k_scale_min_packer_roundtrip(oracle):
    """The unpacker (kquant.rs:83-92) inverts the packer of quantize_q4k_ref
    (kquant.rs:679-684) for every 6-bit (scale, min)."""
    rng = np.random.default_rng(3)
    for _ in range(300):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        s = np.zeros(12, dtype=np.uint8)
        for j in range(4):
            s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
            s[j + 8] = (sc[j + 4] & 0x0F) | ((mn[j + 4] & 0x0F) << 4)
        for j in range(8):
            assert oracle.q4k_scale_min(s, j) == (sc[j], mn[j])


def test_q4k_dequant_roundtrip(oracle):
    """tests/kquant.rs:78-101"""
    rng = oracle.Rng(21)
    for src in (rng.vec(256), rng.adversarial(256)):
        block = oracle.quantize_q4k_ref(src)[0]
        back = oracle.dequant_q4k(block)
        d = oracle.f16_to_f32(int(block[0:2].view(np.uint16)[0]))
        for j in range(8):
            sc, _ = oracle.q4k_scale_min(block[4:16], j)
            step = np.float32(d) * np.float32(sc)
            tol = step * 0.75 + max(step, 1e-3)
            assert np.all(np.abs(back[j * 32:(j + 1) * 32] - src[j * 32:(j + 1) * 32]) <= tol)


def test_q6k_dequant_roundtrip(oracle):
    """tests/kquant.rs:106-136: exact plane packing and scale indexing."""
    rng = oracle.Rng(31)
    for src in (rng.vec(256), rng.adversarial(256)):
        block = oracle.quantize_q6k_ref(src)[0]
        d = np.float32(oracle.f16_to_f32(int(block[208:210].view(np.uint16)[0])))
        scales = block[192:208].view(np.int8)
        back = oracle.dequant_q6k(block)
        for i in range(256):
            sc = d * np.float32(scales[i // 16])
            if sc != 0:
                r = np.float32(src[i]) / sc
                r = int(r + np.float32(0.5)) if r >= 0 else int(r - np.float32(0.5))
                q = min(max(r + 32, 0), 63) - 32
            else:
                q = 0
            expect = sc * np.float32(q)
            assert abs(back[i] - expect) <= abs(expect) * 1e-6 + 1e-7


def _q4k_ints(block):
    """Quants of a Q4_K block by the layout (kquant.rs:26-31, 102-117)."""
    qs = block[16:144]
    q = np.zeros(256, dtype=np.int32)
    for c in range(4):
        q[64 * c:64 * c + 32] = qs[32 * c:32 * c + 32] & 0x0F
        q[64 * c + 32:64 * c + 64] = qs[32 * c:32 * c + 32] >> 4
    return q


def _q6k_ints(block):
    """Quants (minus 32) of a Q6_K block by the layout (kquant.rs:37-42, 125-141)."""
    ql, qh = block[0:128].astype(np.int32), block[128:192].astype(np.int32)
    q = np.zeros(256, dtype=np.int32)
    for h in range(2):
        a, b, hh = ql[64 * h:64 * h + 32], ql[64 * h + 32:64 * h + 64], qh[32 * h:32 * h + 32]
        q[128 * h + 0:128 * h + 32] = (a & 15) | ((hh & 3) << 4)
        q[128 * h + 32:128 * h + 64] = (b & 15) | (((hh >> 2) & 3) << 4)
        q[128 * h + 64:128 * h + 96] = (a >> 4) | (((hh >> 4) & 3) << 4)
        q[128 * h + 96:128 * h + 128] = (b >> 4) | (((hh >> 6) & 3) << 4)
    return q - 32


def test_block_sums_brute_force(oracle):
    """Integer sub-dots equal brute force over the unpacked quants."""
    O = oracle
    rng = np.random.default_rng(9)
    x8 = O.quantize_q8_0(rng.normal(size=32 * 5).astype(np.float32))
    w8 = rng.integers(0, 256, (5, 34), dtype=np.uint8)
    got = O.block_sums(O.Q8_0, w8, x8)
    want = [int((w8[b, 2:].view(np.int8).astype(np.int32) * x8[b, 2:].view(np.int8).astype(np.int32)).sum())
            for b in range(5)]
    assert list(got) == want
    xk = O.quantize_q8k(rng.normal(size=256 * 3).astype(np.float32))
    _, xq, bsums = O.q8k_fields(xk)
    w4 = rng.integers(0, 256, (3, 144), dtype=np.uint8)
    got = O.block_sums(O.Q4K, w4, xk).reshape(3, 9)
    for b in range(3):
        q = _q4k_ints(w4[b])
        sub = (q * xq[b].astype(np.int32)).reshape(8, 32).sum(axis=1)
        mins = [O.q4k_scale_min(w4[b, 4:16], j)[1] for j in range(8)]
        pair = bsums[b].astype(np.int32).reshape(8, 2).sum(axis=1)
        assert list(got[b, :8]) == list(sub)
        assert got[b, 8] == int(np.dot(mins, pair))
    w6 = rng.integers(0, 256, (3, 210), dtype=np.uint8)
    got = O.block_sums(O.Q6K, w6, xk).reshape(3, 16)
    for b in range(3):
        gs = (_q6k_ints(w6[b]) * xq[b].astype(np.int32)).reshape(16, 16).sum(axis=1)
        assert list(got[b]) == list(gs)


# ---- dots -----------------------------------------------------------------------


def test_matvec_matches_f32_reference(oracle):
    """tests/kernels.rs:102-128"""
    O = oracle
    rng = O.Rng(1234)
    rows, cols = 48, 128
    w = O.quantize_q8_0(rng.vec(rows * cols))
    x = O.quantize_q8_0(rng.vec(cols))
    wd = O.dequantize_q8_0(w).reshape(rows, cols)
    xd = O.dequantize_q8_0(x)
    for order in (O.ORDER_SCALAR, O.ORDER_AVX2):
        y = O.matvec(O.Q8_0, order, w, x, rows, cols)
        for r in range(rows):
            expect = np.float32(0)
            for a, b in zip(wd[r], xd):
                expect = np.float32(expect + a * b)
            assert abs(y[r] - expect) <= 1e-4 * max(abs(expect), 1.0)


@pytest.mark.parametrize("dtype,seed", [(2, 41), (3, 51)])
def test_kquant_dot_matches_dequant_reference(oracle, dtype, seed):
    """tests/kquant.rs:138-166 (Q4_K) and 269-295 (Q6_K)"""
    O = oracle
    rng = O.Rng(seed)
    for blocks in (1, 3, 10):
        w = O.quantize_weights_ref(dtype, rng.adversarial(blocks * 256))
        x = O.quantize_q8k(rng.vec(blocks * 256))
        got = O.dot(dtype, O.ORDER_SCALAR, w, x)
        d, qs, _ = O.q8k_fields(x)
        expect = 0.0
        for b in range(blocks):
            wd = O.dequant_q4k(w[b]) if dtype == O.Q4K else O.dequant_q6k(w[b])
            xv = (qs[b].astype(np.float32) * d[b]).astype(np.float64)
            expect += float(np.dot(wd.astype(np.float64), xv))
        assert abs(got - expect) <= 1e-3 * max(abs(expect), 1.0)


def test_avx2_matches_scalar(oracle):
    """tests/kernels.rs:84-100"""
    O = oracle
    rng = O.Rng(42)
    for blocks in (1, 3, 64, 65):
        w = O.quantize_q8_0(rng.vec(blocks * 32))
        x = O.quantize_q8_0(rng.vec(blocks * 32))
        s = O.dot(O.Q8_0, O.ORDER_SCALAR, w, x)
        v = O.dot(O.Q8_0, O.ORDER_AVX2, w, x)
        tol = 1e-5 * max(blocks, 1.0) + 1e-6
        assert abs(s - v) <= tol * max(abs(s), 1.0)


@pytest.mark.parametrize("dtype,seed", [(2, 61), (3, 71)])
def test_avx2_matches_scalar_kquant(oracle, dtype, seed):
    """tests/kquant.rs:168-208"""
    O = oracle
    rng = O.Rng(seed)
    for blocks in (1, 5, 16):
        w = O.quantize_weights_ref(dtype, rng.adversarial(blocks * 256))
        x = O.quantize_q8k(rng.vec(blocks * 256))
        s = O.dot(dtype, O.ORDER_SCALAR, w, x)
        v = O.dot(dtype, O.ORDER_AVX2, w, x)
        assert abs(s - v) <= 1e-4 * max(abs(s), 1.0)


def saturated_blocks(oracle):
    """tests/kquant.rs:215-228"""
    O = oracle
    q4 = np.zeros(144, dtype=np.uint8)
    q4[0:2] = np.array([O.f32_to_f16(0.9)], dtype=np.uint16).view(np.uint8)
    q4[2:4] = np.array([O.f32_to_f16(1.7)], dtype=np.uint16).view(np.uint8)
    q4[4:] = 0xFF
    q6 = np.full(210, 0xFF, dtype=np.uint8)
    q6[192:208] = np.array([-128] * 16, dtype=np.int8).view(np.uint8)
    q6[208:210] = np.array([O.f32_to_f16(1.3)], dtype=np.uint16).view(np.uint8)
    return q4.reshape(1, 144), q6.reshape(1, 210)


def test_avx2_matches_scalar_saturated_blocks(oracle):
    """tests/kquant.rs:210-245"""
    O = oracle
    q4, q6 = saturated_blocks(O)
    x = O.quantize_q8k(O.Rng(81).adversarial(256))
    for dtype, w in ((O.Q4K, q4), (O.Q6K, q6)):
        s = O.dot(dtype, O.ORDER_SCALAR, w, x)
        v = O.dot(dtype, O.ORDER_AVX2, w, x)
        assert abs(s - v) <= 1e-4 * max(abs(s), 1.0)


@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_x4_bit_equals_1wide(oracle, dtype):
    """dot_*_avx2_x4 is bit-identical per lane to dot_*_avx2 (kernels.rs:222-223,
    kquant.rs:307-310, 376-377)."""
    O = oracle
    rng = O.Rng(5 + dtype)
    qk = O.QK[dtype]
    blocks = 7
    w = O.quantize_weights_ref(dtype, rng.adversarial(blocks * qk))
    xs = [O.quantize_act(dtype, rng.vec(blocks * qk)) for _ in range(4)]
    v4 = O.dot_x4(dtype, w, xs)
    for i in range(4):
        assert v4[i].view(np.uint32) == np.float32(O.dot(dtype, O.ORDER_AVX2, w, xs[i])).view(np.uint32)


@pytest.mark.parametrize("dtype", [1, 2, 3])
@pytest.mark.parametrize("order", [0, 1])
def test_matmul_bit_equals_matvec(oracle, dtype, order):
    """tests/kernels.rs:277-292, tests/kquant.rs:297-329 (batch 4 and 5: x4
    tile + remainder)."""
    O = oracle
    rng = O.Rng(202 + dtype)
    qk = O.QK[dtype]
    rows, cols = 32, 2 * qk
    bpr = cols // qk
    w = O.quantize_weights_ref(dtype, rng.vec(rows * cols))
    for batch in (4, 5):
        xs = O.quantize_act(dtype, rng.vec(batch * cols))
        ym = O.matmul(dtype, order, w, xs, rows, cols, batch)
        for b in range(batch):
            yv = O.matvec(dtype, order, w, xs[b * bpr:(b + 1) * bpr], rows, cols)
            assert np.array_equal(ym[b * rows:(b + 1) * rows].view(np.uint32), yv.view(np.uint32))


@pytest.mark.parametrize("order", [0, 1])
def test_row_pool_is_bit_identical(oracle, order):
    """The parallel.rs-style pool only splits rows: any thread count gives the
    same bits."""
    O = oracle
    w = O.gen_weights(O.Q6K, 3, 600, 1024)
    x = O.quantize_q8k(O.Rng(4).normal(1024))
    y1 = O.matvec(O.Q6K, order, w, x, 600, 1024, threads=1)
    y8 = O.matvec(O.Q6K, order, w, x, 600, 1024, threads=8)
    assert np.array_equal(y1.view(np.uint32), y8.view(np.uint32))


# ---- f32 order pins: inputs only the reference's documented order passes --------


def _q8_block(d_bits: int, qs):
    b = np.zeros(34, dtype=np.uint8)
    b[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    b[2:] = np.array(qs, dtype=np.int8).view(np.uint8)
    return b


def test_scalar_order_is_sequential_over_blocks(oracle):
    """dot_q8_scalar adds block contributions left to right (kernels.rs:74-80):
    contributions (2^25, 1, -2^25) give (2^25 + 1) - 2^25 = 0 in f32, while
    any reassociation that pairs +-2^25 first gives 1."""
    O = oracle
    one = [1] + [0] * 31
    # contribution = (acc * dw) * dx with dx = 1.0 and acc = 1
    big = O.f32_to_f16(2.0 ** 15)  # 32768; acc = 1024 gives 2^25
    w = np.stack([_q8_block(big, [32] * 32), _q8_block(0x3C00, one), _q8_block(big, [-32] * 32)])
    x = np.stack([_q8_block(0x3C00, one * 0 + [1] * 32)] * 3)
    x[1] = _q8_block(0x3C00, one)
    s = O.dot(O.Q8_0, O.ORDER_SCALAR, w, x)
    assert s == 0.0
    # the same three contributions in another block order keep the small term
    s2 = O.dot(O.Q8_0, O.ORDER_SCALAR, w[[0, 2, 1]], x[[0, 2, 1]])
    assert s2 == 1.0


def test_avx2_order_hsum_tree(oracle):
    """dot_q8_avx2 keeps 8 lane accumulators (bytes 4k..4k+3) and reduces them
    as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) (kernels.rs:280-285).
    Block 0 (d = 4096) puts a0 = 2^25, a4 = -2^25; block 1 (d = 1) puts
    a1 = 1. The tree cancels a0 + a4 first and returns 1; a sequential lane sum
    or adjacent-pair tree absorbs the 1 into 2^25 and returns 0."""
    O = oracle
    qs0 = [0] * 32
    qs0[0:4] = [64] * 4
    qs0[16:20] = [-64] * 4
    xq0 = [0] * 32
    xq0[0:4] = [32] * 4
    xq0[16:20] = [32] * 4
    qs1 = [0] * 32
    qs1[4] = 1
    w = np.stack([_q8_block(O.f32_to_f16(4096.0), qs0), _q8_block(0x3C00, qs1)])
    x = np.stack([_q8_block(0x3C00, xq0), _q8_block(0x3C00, qs1)])
    assert O.dot(O.Q8_0, O.ORDER_AVX2, w, x) == 1.0
    # the lane-sequential sum the tree replaces would lose the 1
    a = np.float32(2.0 ** 25) + np.float32(1.0)
    assert a - np.float32(2.0 ** 25) == 0.0


def test_golden_fixtures(oracle):
    """The oracle still reproduces the committed fixtures (tests/golden/)."""
    import os

    from tests.golden import make_golden

    path = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
    g = np.load(path, allow_pickle=False)
    fresh = make_golden.build(oracle)
    assert sorted(g.files) == sorted(fresh.keys())
    for k in g.files:
        assert np.array_equal(g[k], fresh[k]), k
