"""nrq_dev_rmsnorm on the GPU: the rmsnorm of vec.rs:4-14 (the sum of squares
in element order, then scale = 1/sqrtf(ss/n + eps), out = x * scale * w)
bit-exact against the oracle's sequential loop, on rows built to stress the
ordered sum.

The rows include exact ties at every scale, squares across 240 binades,
subnormal and overflowing squares, zeros, NaN, and widths from 256 to 8192.
The decode and prefill steps run the same kernel."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_same(got, want, what):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), what
    d = np.nonzero(bits(got)[~nan] != bits(want)[~nan])[0]
    assert d.size == 0, f"{what}: {d.size} of {want.size} differ; first at {d[0]}: {got[~nan][d[0]]} vs {want[~nan][d[0]]}"


def rows_for(n, rng):
    out = []
    out.append(("normal", rng.normal(0, 1, n)))
    out.append(("small_ints_pow2", rng.integers(-15, 16, n) * 2.0 ** rng.integers(-6, 6, n)))
    out.append(("wide_range", rng.choice([-1, 1], n) * 2.0 ** rng.uniform(-60, 60, n)))
    out.append(("subnormal_squares", rng.normal(0, 1, n) * 1e-23))
    out.append(("overflowing", rng.normal(0, 1, n) * 1e20))
    out.append(("zeros", np.zeros(n)))
    lz = rng.normal(0, 1, n)
    lz[: n // 3] = 0.0
    out.append(("leading_zeros", lz))
    big = rng.normal(0, 1e-2, n)
    big[0] = 3e3
    out.append(("one_big_first", big))
    asc = np.sort(np.abs(rng.normal(0, 1, n))) ** 3
    out.append(("ascending", asc))
    nan = rng.normal(0, 1, n)
    nan[n // 2] = np.nan
    out.append(("nan", nan))
    ties = np.full(n, 2.0 ** -12)  # squares 2^-24: halves of the running sum's unit past 1
    ties[0] = 1.0
    out.append(("ties_after_one", ties))
    # past the first 128 terms: the sum sits at 2^20 (unit 2^-3) and every square
    # 1/16 is an exact tie, so each term ends a parallel run early
    flat = np.full(n, 0.25)
    flat[0] = 1024.0
    out.append(("all_ties_steady", flat))
    # squares m^2/16 against the unit 2^-3: odd m is a tie, even m exact
    mix = 0.25 * rng.integers(1, 8, n) * rng.choice([-1, 1], n)
    mix[0] = 1024.0
    out.append(("mixed_ties_steady", mix))
    # a slow ramp: the sum crosses binades at scattered positions late in the row
    out.append(("late_crossings", np.sqrt(np.linspace(1e-3, 4.0, n)) * rng.choice([-1, 1], n)))
    spikes = rng.normal(0, 1e-3, n)
    spikes[rng.integers(128, n, 6)] = rng.normal(0, 30, 6)
    out.append(("late_spikes", spikes))
    return out


@pytest.mark.parametrize("n", [256, 512, 768, 2048, 2560, 4096, 6144, 8192])
def test_rmsnorm_bitexact_on_hard_rows(gpu, oracle, n):
    import torch

    from nightrun_amd import _lib

    rng = np.random.default_rng(n)
    cases = rows_for(n, rng)
    x = np.stack([c[1] for c in cases]).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32)
    eps = np.float32(1e-5)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    out = torch.empty_like(xd)
    _lib.check(_lib.lib().nrq_dev_rmsnorm(xd.data_ptr(), wd.data_ptr(), out.data_ptr(), x.shape[0], n, C.c_float(eps),
                                          None))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, (name, _) in enumerate(cases):
        want = oracle.rmsnorm(x[i], w, float(eps))
        assert_same(got[i], want, f"n={n} {name}")


def test_rmsnorm_rejects_bad_shapes(gpu):
    import torch

    from nightrun_amd import _lib

    x = torch.zeros(300, device="cuda")
    rc = _lib.lib().nrq_dev_rmsnorm(x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 300, C.c_float(1e-5), None)
    assert rc != 0
