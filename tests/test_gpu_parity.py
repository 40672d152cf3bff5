"""GPU parity: libnrq's gfx950 kernels against the CPU oracle, bit for bit.

Every comparison here is exact (f32 outputs compared as bit patterns, integer
sums and quantized blocks byte for byte) in the f32 order under test; the
reference's own tolerance (1e-5 relative) is never needed because both
orders are reproduced exactly. Calls go through the C ABI (host-slice mirror
of nr-tensor, or the device entry points over torch tensors).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DTYPES = [1, 2, 3]
NAMES = {1: "q8_0", 2: "q4k", 3: "q6k"}
ORDERS = [0, 1]
ONAMES = {0: "scalar", 1: "avx2"}
THREADS = min(16, os.cpu_count() or 1)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitwise(got, want, what=""):
    got, want = bits(got), bits(want)
    if not np.array_equal(got, want):
        bad = np.nonzero(got != want)[0]
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {got.size} differ; first at {i}: "
                             f"{got[i:i + 1].view(np.float32)} vs {want[i:i + 1].view(np.float32)}")


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_matvec(dtype, order, w, x, rows, cols):
    import torch

    from nightrun_amd import device

    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    device.matvec(dtype, order, y, dev(w), dev(x), rows, cols)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def gpu_matmul(dtype, order, w, xs, rows, cols, batch):
    import torch

    from nightrun_amd import device

    y = torch.empty(rows * batch, dtype=torch.float32, device="cuda")
    device.matmul(dtype, order, y, dev(w), dev(xs), rows, cols, batch)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.fixture(scope="module")
def golden():
    path = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
    return dict(np.load(path, allow_pickle=False))


# ---- committed fixtures --------------------------------------------------------


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_golden_matvec_host_api(gpu, golden, dtype, order):
    """nr-tensor mirror (host slices, synchronous) reproduces the fixtures."""
    from nightrun_amd.nr_tensor import kernels, kquant

    n = NAMES[dtype]
    w, x = golden[f"{n}_w"], golden[f"{n}_x"]
    rows, cols = 37, (160 if dtype == 1 else 768)
    gpu.set_order(order)
    try:
        y = np.zeros(rows, dtype=np.float32)
        fn = {1: kernels.matvec_q8, 2: kquant.matvec_q4k, 3: kquant.matvec_q6k}[dtype]
        fn(y, w, x, rows, cols)
        assert_bitwise(y, golden[f"{n}_y_{ONAMES[order]}"], f"{n} {ONAMES[order]}")
        ym = np.zeros(rows * 5, dtype=np.float32)
        fm = {1: kernels.matmul_q8, 2: kquant.matmul_q4k, 3: kquant.matmul_q6k}[dtype]
        fm(ym, w, golden[f"{n}_xs"], rows, cols, 5)
        assert_bitwise(ym, golden[f"{n}_ym_{ONAMES[order]}"], f"{n} matmul {ONAMES[order]}")
    finally:
        gpu.set_order(0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_golden_block_sums(gpu, golden, dtype):
    """Per-block integer dot products are bit-exact (kernels.rs:75-78,
    kquant.rs:200-214, 232-242)."""
    import torch

    from nightrun_amd import device

    n = NAMES[dtype]
    rows, cols = 37, (160 if dtype == 1 else 768)
    want = golden[f"{n}_sums"]
    out = torch.zeros(want.size, dtype=torch.int32, device="cuda")
    device.block_sums(dtype, out, dev(golden[f"{n}_w"]), dev(golden[f"{n}_x"]), rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", DTYPES)
def test_golden_quantize(gpu, golden, dtype):
    from nightrun_amd.nr_tensor import kquant, q8

    n = NAMES[dtype]
    for src_key, q_key in ((f"{n}_xf", f"{n}_x"), (f"{n}_xsf", f"{n}_xs")):
        src, want = golden[src_key], golden[q_key]
        out = np.zeros_like(want)
        (q8.quantize if dtype == 1 else kquant.quantize_q8k)(src, out)
        assert np.array_equal(out, want), src_key


# ---- quantizers -------------------------------------------------------------------


def quant_inputs(oracle, n):
    rng = oracle.Rng(77)
    f = np.finfo(np.float32)
    cases = [rng.vec(n), rng.adversarial(n), rng.normal(n), np.zeros(n, np.float32), rng.vec(n) * np.float32(1e-30),
             rng.vec(n) * np.float32(3e38)]
    ties = ((np.arange(n) % 1023) + 0.5).astype(np.float32) * np.float32(2.0 ** -24) * np.float32(127.0)
    cases.append(ties)
    special = rng.normal(n)
    special[::37] = np.nan
    special[5::41] = np.inf
    special[9::43] = -np.inf
    special[11::47] = f.tiny / 4
    cases.append(special)
    # the largest |v| twice with opposite signs: the first index sets the
    # scale's sign (kquant.rs:162-167); positions in one lane, across quads,
    # 16-lane rows and half-waves of a 256-value block, and the same with +-inf
    pairs = [(0, 1), (1, 0), (7, 8), (8, 7), (31, 32), (32, 31), (100, 200), (200, 100), (255, 0), (0, 255),
             (128, 127), (127, 128)]
    for big in (np.float32(2.0), np.float32(np.inf)):
        tie = rng.vec(n) * np.float32(0.5)
        for k in range(n // 256):
            p1, p2 = pairs[k % len(pairs)]
            tie[256 * k + p1] = -big
            tie[256 * k + p2] = big
        cases.append(tie)
    return cases


def test_quantize_q8_0_bitexact(gpu, oracle):
    """q8::quantize (q8.rs:27-44) incl. the softfloat f16 scale and Rust's
    saturating float->int cast, over random, adversarial, zero, tiny, huge,
    subnormal-tie and NaN/inf inputs."""
    from nightrun_amd.nr_tensor import q8

    for i, src in enumerate(quant_inputs(oracle, 32 * 96)):
        out = np.zeros((96, 34), dtype=np.uint8)
        q8.quantize(src, out)
        assert np.array_equal(out, oracle.quantize_q8_0(src)), f"case {i}"


def test_quantize_q8k_bitexact(gpu, oracle):
    """kquant::quantize_q8k (kquant.rs:157-187)."""
    from nightrun_amd.nr_tensor import kquant

    for i, src in enumerate(quant_inputs(oracle, 256 * 12)):
        out = np.zeros((12, 292), dtype=np.uint8)
        kquant.quantize_q8k(src, out)
        assert np.array_equal(out, oracle.quantize_q8k(src)), f"case {i}"


def test_quantize_device_entry_points(gpu, oracle):
    import torch

    from nightrun_amd import device

    src = oracle.Rng(5).normal(256 * 40)
    o8 = torch.zeros(40 * 8 * 34, dtype=torch.uint8, device="cuda")
    device.quantize_q8_0(dev(src), o8)
    ok = torch.zeros(40 * 292, dtype=torch.uint8, device="cuda")
    device.quantize_q8k(dev(src), ok)
    torch.cuda.synchronize()
    assert np.array_equal(o8.cpu().numpy().reshape(-1, 34), oracle.quantize_q8_0(src))
    assert np.array_equal(ok.cpu().numpy().reshape(-1, 292), oracle.quantize_q8k(src))


def test_hand_derived_step_pins_on_device(gpu):
    """The blocks of tests/test_oracle_scalar_steps.py, whose results under the
    reference's f32 steps are derived by hand there, through the device
    quantizers, the decode matvec and both prefill tiles (16 x 16 under 1024
    rows, 32 x 32 from 1024), compared with the hand-derived literals."""
    import torch

    from nightrun_amd import device
    from tests.test_oracle_kquant_order import q6k_block, q8k_block
    from tests.test_oracle_scalar_steps import q8_0_block

    near = 0.5 - 2.0 ** -25
    srcs = np.zeros((5, 32), dtype=np.float32)
    srcs[0, :6] = [127.0, 2.5, -2.5, near, -near, 1.5 - 2.0 ** -23]
    srcs[1, 3] = -177 * 2.0 ** -24
    srcs[2, :2] = [130.96875, 15.984375 - 2.0 ** -20]
    srcs[3, 7] = 127 * (1 + 2.0 ** -11) + 2.0 ** -17
    o8 = torch.zeros(5 * 34, dtype=torch.uint8, device="cuda")
    device.quantize_q8_0(dev(srcs.reshape(-1)), o8)
    torch.cuda.synchronize()
    b = o8.cpu().numpy().reshape(5, 34)
    d = b[:, 0].astype(np.int64) | b[:, 1].astype(np.int64) << 8
    qs = b[:, 2:].view(np.int8)
    assert list(d[:4]) == [0x3C00, 0x0001, 0x3C20, 0x3C01]
    assert list(qs[0, :6]) == [127, 3, -3, 1, -1, 1]
    assert qs[1, 3] == -127 and list(qs[2, :2]) == [127, 16]

    k = np.zeros((2, 256), dtype=np.float32)
    k[0, :5] = [-128.0, 2.5, -2.5, near, -near]
    k[1, :2] = [7.0, -(6.91796875 - 2.0 ** -21)]
    ok = torch.zeros(2 * 292, dtype=torch.uint8, device="cuda")
    device.quantize_q8k(dev(k.reshape(-1)), ok)
    torch.cuda.synchronize()
    kb = ok.cpu().numpy().reshape(2, 292)
    kd = kb[:, 0:4].copy().view(np.float32).ravel()
    kq = kb[:, 4:260].view(np.int8)
    assert kd[0] == 1.0 and list(kq[0, :5]) == [-128, 3, -3, 1, -1]
    assert kd[1] == -(7 / 128 - 2.0 ** -28) and list(kq[1, :2]) == [-128, 127]

    # dot_q8_scalar: ((acc*dw)*dx), two blocks chained
    w8 = np.stack([q8_0_block(0x3C01, [127, 127]), q8_0_block(0x3C01, [1])]).reshape(1, 68)
    x8 = np.stack([q8_0_block(0x3C02, [127, 2]), q8_0_block(0x3C01, [1])]).reshape(-1)
    # dot_q6k_scalar: d_all before the sum
    q = np.full(256, 32, dtype=np.int64)
    q8 = np.zeros(256, dtype=np.int64)
    q[0], q8[0], q[1], q8[1] = 33, 127, 33, 2
    w6 = q6k_block(0x3C01, [127] + [0] * 15, q).reshape(1, 210)
    x6 = q8k_block(1 + 2.0 ** -10, q8).reshape(-1)
    for dtype, w, x, cols, want in ((1, w8, x8, 64, 16432.03125), (3, w6, x6, 256, 16415 + 7 / 512)):
        assert gpu_matvec(dtype, 0, w, x, 1, cols)[0] == want
        for rows in (40, 1056):
            wr = np.ascontiguousarray(np.repeat(w, rows, axis=0))
            xs = np.ascontiguousarray(np.tile(x, 5))
            assert np.all(gpu_matvec(dtype, 0, wr, x, rows, cols) == want)
            assert np.all(gpu_matmul(dtype, 0, wr, xs, rows, cols, 5) == want)


@pytest.mark.parametrize("dtype", [2, 3])
def test_scale_chain_past_2p24_on_device(gpu, oracle, dtype):
    """The K-quant scale chains whose partial sums pass 2^24 and round
    (tests/test_oracle_kquant_order.py: Q4_K 11521440, Q6_K 2^25, where the
    exact integer sums are 11521441 and 2^25 + 3), in every third row beside
    random blocks, so that the lanes of a wave take both the integer and the
    f32 form of the chain; decode matvec and prefill tiles."""
    from tests.test_oracle_kquant_order import _q6k_chain_case, q4k_chain_case

    if dtype == 2:
        wc, xc, _ = q4k_chain_case()
        want = 11521440.0
    else:
        wc, xc, _ = _q6k_chain_case()
        want = 2.0 ** 25
    assert gpu_matvec(dtype, 0, wc, xc, 1, 256)[0] == want
    cols = 512
    xr = oracle.quantize_act(dtype, oracle.Rng(17).normal(256))
    x = np.ascontiguousarray(np.concatenate([xc.reshape(-1), xr.reshape(-1)]))
    for rows in (40, 1056):
        w = oracle.gen_weights(dtype, 90 + rows, rows, cols).reshape(rows, 2, -1).copy()
        w[::3, 0] = wc[0]
        w = np.ascontiguousarray(w.reshape(rows, -1))
        ref = oracle.matvec(dtype, 0, w, x, rows, cols)
        assert_bitwise(gpu_matvec(dtype, 0, w, x, rows, cols), ref, f"{NAMES[dtype]} {rows} rows")
        xs = np.ascontiguousarray(np.tile(x, 5))
        got = gpu_matmul(dtype, 0, w, xs, rows, cols, 5).reshape(5, rows)
        for t in range(5):
            assert_bitwise(got[t], ref, f"{NAMES[dtype]} {rows} rows, token {t}")


# ---- f16 scale decode --------------------------------------------------------------


@pytest.mark.parametrize("order", ORDERS)
def test_f16_scale_decode_all_patterns(gpu, oracle, order):
    """Every f16 weight-scale bit pattern decodes like f16_to_f32 (f16.rs:3-23):
    row r of a Q8_0 matrix has d = r and one unit quant, against x = e0 with
    dx = 1, so y[r] = (1 * f16(r)) * 1."""
    rows = 65536
    w = np.zeros((rows, 34), dtype=np.uint8)
    w[:, 0:2] = np.arange(rows, dtype=np.uint32).astype(np.uint16).view(np.uint8).reshape(rows, 2)
    w[:, 2] = 1
    x = np.zeros((1, 34), dtype=np.uint8)
    x[0, 0:2] = np.array([0x3C00], dtype=np.uint16).view(np.uint8)
    x[0, 2] = 1
    y = gpu_matvec(1, order, w, x, rows, 32)
    want = oracle.matvec(1, order, w, x, rows, 32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(y), nan)
    assert_bitwise(y[~nan], want[~nan], "f16 decode")


# ---- shapes ------------------------------------------------------------------------

SHAPES = {
    1: [(1, 32), (7, 64), (64, 2048), (1000, 256), (513, 8192), (4099, 2048)],
    2: [(1, 256), (5, 512), (64, 3072), (777, 2560), (300, 4096), (2049, 3072)],
    3: [(1, 256), (5, 768), (64, 3072), (777, 2560), (301, 9728), (2049, 3072)],
}


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matvec_shapes_bitexact(gpu, oracle, dtype, order):
    """Ragged row counts, 1..256 blocks per row, rows that are not 16-byte
    multiples (Q6_K 210-byte and Q8_0 34-byte blocks), both orders."""
    for i, (rows, cols) in enumerate(SHAPES[dtype]):
        w = oracle.gen_weights(dtype, 1000 + i, rows, cols)
        x = oracle.quantize_act(dtype, oracle.Rng(2000 + i).normal(cols))
        want = oracle.matvec(dtype, order, w, x, rows, cols, threads=THREADS)
        assert_bitwise(gpu_matvec(dtype, order, w, x, rows, cols), want, f"{NAMES[dtype]} {rows}x{cols}")


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matvec_adversarial_weights(gpu, oracle, dtype, order):
    """Weights from the reference's test quantizers over adversarial data,
    and the saturated blocks of tests/kquant.rs:210-245."""
    qk = oracle.QK[dtype]
    rows, cols = 40, 4 * qk
    rng = oracle.Rng(300 + dtype)
    w = oracle.quantize_weights_ref(dtype, rng.adversarial(rows * cols))
    x = oracle.quantize_act(dtype, rng.adversarial(cols))
    assert_bitwise(gpu_matvec(dtype, order, w, x, rows, cols), oracle.matvec(dtype, order, w, x, rows, cols))
    if dtype != 1:
        from tests.test_oracle import saturated_blocks

        q4, q6 = saturated_blocks(oracle)
        blk = q4 if dtype == 2 else q6
        ws = np.repeat(blk, rows * 4, axis=0)
        assert_bitwise(gpu_matvec(dtype, order, ws, x, rows, cols), oracle.matvec(dtype, order, ws, x, rows, cols))


@pytest.mark.parametrize("dtype", DTYPES)
def test_w_longer_than_rows_times_bpr(gpu, oracle, dtype):
    """`w.len() >= rows * bpr` (kernels.rs:40): trailing blocks are ignored."""
    from nightrun_amd.nr_tensor import kernels, kquant

    qk = oracle.QK[dtype]
    rows, cols = 9, 3 * qk
    w = oracle.gen_weights(dtype, 7, rows + 2, cols)
    x = oracle.quantize_act(dtype, oracle.Rng(8).normal(cols))
    y = np.zeros(rows, dtype=np.float32)
    fn = {1: kernels.matvec_q8, 2: kquant.matvec_q4k, 3: kquant.matvec_q6k}[dtype]
    fn(y, w, x, rows, cols)
    assert_bitwise(y, oracle.matvec(dtype, 0, w, x, rows, cols))


# ---- matmul == matvec ----------------------------------------------------------------


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_bit_equals_matvec(gpu, oracle, dtype, order):
    """Batched output equals per-token matvecs bit for bit (tests/kernels.rs:277-292,
    tests/kquant.rs:297-329), at batch 1, 4, 5, 17, 63 and 64 (MAX_BATCH,
    crates/nr-model/src/infer.rs:101)."""
    qk = oracle.QK[dtype]
    rows, cols = 96, 8 * qk
    bpr = cols // qk
    w = oracle.gen_weights(dtype, 55, rows, cols)
    for batch in (1, 4, 5, 17, 63, 64):
        xs = oracle.quantize_act(dtype, oracle.Rng(60 + batch).normal(batch * cols))
        ym = gpu_matmul(dtype, order, w, xs, rows, cols, batch)
        assert_bitwise(ym, oracle.matmul(dtype, order, w, xs, rows, cols, batch, threads=THREADS), f"batch {batch}")
        for b in (0, batch - 1):
            yv = gpu_matvec(dtype, order, w, xs[b * bpr:(b + 1) * bpr], rows, cols)
            assert_bitwise(ym[b * rows:(b + 1) * rows], yv, f"batch {batch} row {b}")


# ---- boundary behaviour -----------------------------------------------------------------


def test_shape_assertions_panic(gpu):
    """Shape mismatches raise with the reference assertion's text
    (kernels.rs:38-40, kquant.rs:541-543, q8.rs:28)."""
    from nightrun_amd import NrPanic
    from nightrun_amd.nr_tensor import kernels, kquant, q8

    w = np.zeros((8, 34), dtype=np.uint8)
    x = np.zeros((2, 34), dtype=np.uint8)
    with pytest.raises(NrPanic, match=r"y.len\(\) == rows"):
        kernels.matvec_q8(np.zeros(3, np.float32), w, x, 4, 64)
    with pytest.raises(NrPanic, match=r"x.len\(\) == bpr"):
        kernels.matvec_q8(np.zeros(4, np.float32), w, x[:1], 4, 64)
    with pytest.raises(NrPanic, match=r"w.len\(\) >= rows \* bpr"):
        kernels.matvec_q8(np.zeros(5, np.float32), w, x, 5, 64)
    with pytest.raises(NrPanic, match=r"xs.len\(\) == batch \* bpr"):
        kernels.matmul_q8(np.zeros(8, np.float32), w, x, 4, 64, 2)
    with pytest.raises(NrPanic):
        kquant.matvec_q4k(np.zeros(2, np.float32), np.zeros((2, 144), np.uint8), np.zeros((2, 292), np.uint8), 2, 256)
    with pytest.raises(NrPanic):
        q8.quantize(np.zeros(33, np.float32), np.zeros((1, 34), np.uint8))


def test_empty_and_zero_width(gpu):
    """rows = 0 is a no-op; cols < QK gives empty dots (+0.0)."""
    from nightrun_amd.nr_tensor import kernels

    kernels.matvec_q8(np.zeros(0, np.float32), np.zeros((0, 34), np.uint8), np.zeros((0, 34), np.uint8), 0, 0)
    y = np.full(3, 7.0, dtype=np.float32)
    kernels.matvec_q8(y, np.zeros((0, 34), np.uint8), np.zeros((0, 34), np.uint8), 3, 31)
    assert_bitwise(y, np.zeros(3, np.float32))


def test_registered_weights_match_unregistered(gpu, oracle):
    from nightrun_amd import nr_tensor
    from nightrun_amd.nr_tensor import kquant

    rows, cols = 300, 3072
    w = oracle.gen_weights(3, 99, rows, cols)
    x = oracle.quantize_q8k(oracle.Rng(3).normal(cols))
    y0 = np.zeros(rows, np.float32)
    kquant.matvec_q6k(y0, w, x, rows, cols)
    nr_tensor.register_weights(w)
    try:
        y1 = np.zeros(rows, np.float32)
        kquant.matvec_q6k(y1, w, x, rows, cols)
        # a slice of the registered region: rows 10.. (2520-byte rows, 8-byte aligned only)
        y2 = np.zeros(rows - 16, np.float32)
        kquant.matvec_q6k(y2, w[16 * 12:], x, rows - 16, cols)
    finally:
        nr_tensor.unregister_weights(w)
    assert_bitwise(y1, y0)
    assert_bitwise(y2, y0[16:])


# ---- full benchmark shapes ------------------------------------------------------------------

CONFIGS = {
    "cfg1_q8_0_8192x2048": (1, 8192, 2048, 0x5EED0001),
    "cfg2_q4k_8192x3072": (2, 8192, 3072, 0x5EED0002),
    "cfg3_q6k_128256x3072": (3, 128256, 3072, 0x5EED0003),
}


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_benchmark_configs_bitexact(gpu, oracle, cfg, order):
    dtype, rows, cols, seed = CONFIGS[cfg]
    w = oracle.gen_weights(dtype, seed, rows, cols)
    x = oracle.quantize_act(dtype, oracle.Rng(seed ^ 0xABCDEF).normal(cols))
    want = oracle.matvec(dtype, order, w, x, rows, cols, threads=THREADS)
    assert_bitwise(gpu_matvec(dtype, order, w, x, rows, cols), want, cfg)


# ---- prefill matmul (int8 MFMA tiles, both orders) ---------------------------------------

# Qwen3-4B layer at M = 64 tokens: hidden 2560, attention width 4096, ffn 9728,
# 8 KV heads x 128 (kv width 1024); Q/K/V/O/gate/up Q4_K, down Q6_K.
QWEN3_4B_LAYER = {
    "wq": (2, 4096, 2560), "wk": (2, 1024, 2560), "wv": (2, 1024, 2560), "wo": (2, 2560, 4096),
    "w_gate": (2, 9728, 2560), "w_up": (2, 9728, 2560), "w_down": (3, 2560, 9728),
}


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("name", list(QWEN3_4B_LAYER))
def test_prefill_qwen3_4b_layer_bitexact(gpu, oracle, name, order):
    """Batched M = 64 matmul on the layer's real shapes equals the oracle's
    matmul (== 64 matvecs, tests/kquant.rs:297-329) bit for bit, in the
    scalar order and in the AVX2 order (the 4-wide x4 tiles of
    kquant.rs:566-639)."""
    dtype, rows, cols = QWEN3_4B_LAYER[name]
    seed = 0x5EED0004 + list(QWEN3_4B_LAYER).index(name)
    w = oracle.gen_weights(dtype, seed, rows, cols)
    xs = oracle.quantize_act(dtype, oracle.Rng(seed ^ 0x77).normal(64 * cols))
    want = oracle.matmul(dtype, order, w, xs, rows, cols, 64, threads=THREADS)
    assert_bitwise(gpu_matmul(dtype, order, w, xs, rows, cols, 64), want, f"{name} {ONAMES[order]}")


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_batches_past_64(gpu, oracle, dtype, order):
    """The reference's matmul takes any batch; a launch covers it in 32-token
    tiles (batch 65 and 130: a one-token tile and a partial tile)."""
    qk = oracle.QK[dtype]
    rows, cols = 50, 3 * qk
    w = oracle.gen_weights(dtype, 91, rows, cols)
    for batch in (65, 130):
        xs = oracle.quantize_act(dtype, oracle.Rng(92 + batch).normal(batch * cols))
        assert_bitwise(gpu_matmul(dtype, order, w, xs, rows, cols, batch),
                       oracle.matmul(dtype, order, w, xs, rows, cols, batch, threads=THREADS), f"batch {batch}")


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_long_rows_and_odd_block_counts(gpu, oracle, dtype, order):
    """Rows longer than a split holds (70 blocks, 5 tokens: one split, idle
    token tiles), an odd block count at a full 64-token batch (Q6_K blocks of
    one row then alternate their 4-byte alignment), and a row count that is
    not a multiple of 16."""
    qk = oracle.QK[dtype]
    for rows, bpr, batch in ((20, 70, 5), (40, 37, 64)):
        cols = bpr * qk
        w = oracle.gen_weights(dtype, 700 + bpr, rows, cols)
        xs = oracle.quantize_act(dtype, oracle.Rng(701 + bpr).normal(batch * cols))
        assert_bitwise(gpu_matmul(dtype, order, w, xs, rows, cols, batch),
                       oracle.matmul(dtype, order, w, xs, rows, cols, batch, threads=THREADS),
                       f"rows {rows} bpr {bpr} batch {batch}")


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_adversarial_and_saturated(gpu, oracle, dtype, order):
    """Adversarial activations, the reference quantizers' weights, and the
    saturated blocks of tests/kquant.rs:210-245 through the MFMA path."""
    qk = oracle.QK[dtype]
    rows, cols, batch = 33, 4 * qk, 19
    rng = oracle.Rng(400 + dtype)
    w = oracle.quantize_weights_ref(dtype, rng.adversarial(rows * cols))
    xs = oracle.quantize_act(dtype, rng.adversarial(batch * cols))
    assert_bitwise(gpu_matmul(dtype, order, w, xs, rows, cols, batch),
                   oracle.matmul(dtype, order, w, xs, rows, cols, batch))
    if dtype != 1:
        from tests.test_oracle import saturated_blocks

        q4, q6 = saturated_blocks(oracle)
        ws = np.repeat(q4 if dtype == 2 else q6, rows * 4, axis=0)
        assert_bitwise(gpu_matmul(dtype, order, ws, xs, rows, cols, batch),
                       oracle.matmul(dtype, order, ws, xs, rows, cols, batch))


def _q8k_raw(d, qs):
    """Q8_K blocks from raw fields (bsums consistent with qs)."""
    qs = np.asarray(qs, dtype=np.int8).reshape(-1, 256)
    out = np.zeros((qs.shape[0], 292), dtype=np.uint8)
    out[:, 0:4] = np.full((qs.shape[0], 1), d, dtype=np.float32).view(np.uint8)
    out[:, 4:260] = qs.view(np.uint8)
    out[:, 260:292] = qs.astype(np.int16).reshape(-1, 16, 16).sum(axis=2).astype(np.int16).view(np.uint8)
    return out


@pytest.mark.parametrize("dtype", [2, 3])
def test_matmul_avx2_extreme_integer_sums(gpu, oracle, dtype):
    """The AVX2 order's per-lane integer sums at their extremes, where the
    MFMA tile splits each scaled weight into two int8 operands: Q6_K scale
    -128 against quants 0 (sc * (q - 32) = 4096) and activations -128, a lane
    sum of -2^24 (kquant.rs:495-499); Q4_K scale 63 against nibbles 15; and
    mixed signs and scales. Batches of 2 and 33 (the smallest MFMA batch, and
    a one-token second tile), 37 rows (a partial row tile), 3 blocks a row."""
    rows, bpr = 37, 3
    cols = 256 * bpr
    rng = np.random.default_rng(1234 + dtype)
    if dtype == 3:
        w = np.zeros((rows * bpr, 210), dtype=np.uint8)
        w[:, 192:208] = np.array(-128, dtype=np.int8).view(np.uint8)
        w[:, 208:210] = np.array([oracle.f32_to_f16(1.0)], dtype=np.uint16).view(np.uint8)
        mixed = rng.integers(0, 256, size=(rows * bpr, 208), dtype=np.uint8)
        w[1::2, :208] = mixed[1::2]  # odd blocks: random quants and signed scales
    else:
        w = np.zeros((rows * bpr, 144), dtype=np.uint8)
        w[:, 0:2] = np.array([oracle.f32_to_f16(1.0)], dtype=np.uint16).view(np.uint8)
        w[:, 2:4] = np.array([oracle.f32_to_f16(0.5)], dtype=np.uint16).view(np.uint8)
        w[:, 4:] = 0xFF  # every 6-bit scale and min 63, every nibble 15
        mixed = rng.integers(0, 256, size=(rows * bpr, 140), dtype=np.uint8)
        w[1::2, 4:] = mixed[1::2]
    for batch in (2, 33):
        qs = np.full((batch * bpr, 256), -128, dtype=np.int8)
        qs[1::2] = rng.integers(-128, 128, size=qs[1::2].shape, dtype=np.int8)
        xs = _q8k_raw(1.0, qs)
        assert_bitwise(gpu_matmul(dtype, 1, w, xs, rows, cols, batch),
                       oracle.matmul(dtype, 1, w, xs, rows, cols, batch), f"batch {batch}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_avx2_small_shapes(gpu, oracle, dtype):
    """AVX2-order matmul at the small cases of the MFMA tiles: one block a
    row, fewer rows than a tile (1, 7, 9), one token (the decode kernel), two
    tokens, and rows just past one and two 32-row tiles."""
    qk = oracle.QK[dtype]
    for rows, bpr, batch in ((1, 1, 2), (7, 2, 3), (9, 1, 1), (33, 2, 2), (65, 5, 31)):
        cols = bpr * qk
        w = oracle.gen_weights(dtype, 1300 + rows, rows, cols)
        xs = oracle.quantize_act(dtype, oracle.Rng(1301 + rows).normal(batch * cols))
        assert_bitwise(gpu_matmul(dtype, 1, w, xs, rows, cols, batch),
                       oracle.matmul(dtype, 1, w, xs, rows, cols, batch), f"rows {rows} bpr {bpr} batch {batch}")


@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_matmul_every_split_count(gpu, oracle, dtype, monkeypatch):
    """The 32 x 32 prefill kernel (Q8_0, Q4_K, Q6_K) splits a tile's blocks over 1, 2, 4 or
    8 waves and holds one, two or (Q8_0) four blocks of loads in registers
    (chosen by shape; NRQ_MMT_SPLITS and NRQ_MMT_NB force them). Every combination gives the
    oracle's bits: odd block counts (the last round partly empty), a
    partial token tile, batches past 64 and fewer than 32 tokens."""
    qk = oracle.QK[dtype]
    cases = []
    shapes = ((96, 8, 64), (40, 37, 33), (50, 3, 130), (20, 11, 5))
    if dtype == 1:  # Q8_0 takes these tiles from 1024 rows
        shapes = ((1024, 8, 64), (1100, 37, 33), (1030, 3, 130), (1056, 11, 5))
    for rows, bpr, batch in shapes:
        cols = bpr * qk
        w = oracle.gen_weights(dtype, 800 + bpr, rows, cols)
        xs = oracle.quantize_act(dtype, oracle.Rng(801 + bpr).normal(batch * cols))
        cases.append((rows, cols, batch, w, xs, oracle.matmul(dtype, 0, w, xs, rows, cols, batch, threads=THREADS)))
    # register buffers of block loads: 1 or 2, a ring of 4 for Q8_0, and Q8_0's
    # 8-block spans through LDS (whole rows of 8-block multiples only, else 1)
    for nb in ("1", "2", "4", "8") if dtype == 1 else ("1", "2"):
        monkeypatch.setenv("NRQ_MMT_NB", nb)
        for ks in ("1", "2", "4", "8"):
            monkeypatch.setenv("NRQ_MMT_SPLITS", ks)
            for rows, cols, batch, w, xs, want in cases:
                assert_bitwise(gpu_matmul(dtype, 0, w, xs, rows, cols, batch), want,
                               f"splits {ks} buffers {nb} rows {rows} cols {cols} batch {batch}")


def test_matmul_q8_0_spans(gpu, oracle, monkeypatch):
    """Q8_0 tiles of whole rows past 64 tokens read 8-block spans of their rows
    and tokens into LDS: ragged row and token tiles, one span and several, and
    the span path forced below 64 tokens, all with the oracle's bits."""
    cases = []
    for rows, bpr, batch in ((1024, 8, 65), (1100, 16, 130), (1030, 64, 200), (1056, 24, 5), (1024, 8, 33)):
        cols = bpr * 32
        w = oracle.gen_weights(1, 810 + bpr, rows, cols)
        xs = oracle.quantize_act(1, oracle.Rng(811 + batch).normal(batch * cols))
        cases.append((rows, cols, batch, w, xs, oracle.matmul(1, 0, w, xs, rows, cols, batch, threads=THREADS)))
    for forced in (False, True):
        if forced:
            monkeypatch.setenv("NRQ_MMT_NB", "8")
            monkeypatch.setenv("NRQ_MMT_SPLITS", "1")
        for rows, cols, batch, w, xs, want in cases:
            assert_bitwise(gpu_matmul(1, 0, w, xs, rows, cols, batch), want,
                           f"spans forced {forced} rows {rows} cols {cols} batch {batch}")


@pytest.mark.parametrize("dtype", [1, 2, 3])
def test_matmul_group(gpu, oracle, dtype):
    """nrq_dev_matmul_group (Acts::matmul_group, infer.rs:180-228): every
    matrix of a group over one activation equals the oracle's matmul bit for
    bit, whether the group runs as one launch of the 32 x 32 kernel (ragged
    rows, partial tiles, batches past 64) or as separate launches (Q8_0 below
    1024 rows in all, one matrix)."""
    import torch

    from nightrun_amd import device

    qk = oracle.QK[dtype]
    big = (1100, 300, 40) if dtype == 1 else (96, 40, 33)
    small = (300, 200) if dtype == 1 else (50,)
    for rows_list, bpr, batch in ((big, 8, 64), (big, 3, 70), (small, 5, 17)):
        cols = bpr * qk
        xs = oracle.quantize_act(dtype, oracle.Rng(900 + bpr).normal(batch * cols))
        ws = [oracle.gen_weights(dtype, 910 + i + bpr, r, cols) for i, r in enumerate(rows_list)]
        ys = [torch.empty(batch * r, dtype=torch.float32, device="cuda") for r in rows_list]
        device.matmul_group(dtype, ys, [torch.from_numpy(w).cuda() for w in ws], list(rows_list),
                            torch.from_numpy(xs).cuda(), cols, batch)
        torch.cuda.synchronize()
        for i, r in enumerate(rows_list):
            want = oracle.matmul(dtype, 0, ws[i], xs, r, cols, batch, threads=THREADS)
            assert_bitwise(ys[i].cpu().numpy(), want, f"matrix {i} rows {r} bpr {bpr} batch {batch}")
