"""The workgroup-parallel exact sum behind the decode norms (wg_chain_pass and
wg_chain_nonneg in nightrun_amd/csrc/nrq_device.h), restated lane for lane
in numpy float32 and checked bit-exact against the sequential f32 chain, the
reference's `ss += v * v` loop (crates/nr-tensor/src/vec.rs:4-14).

The restatement follows the device code: four waves of 64 lanes, 4, 8 or 16
consecutive terms per lane, an f32 prediction of each term's binade (wave
totals added in wave order across the waves), terms rounded to the unit of
their predicted binade, special terms (binade crossings, ties) resolved in
order by plain f32 adds, and every check that makes a pass fall back to the
plain chain (more than 48 special terms in one pass among them). The cases are
built to reach each of those checks; the fast path must also be the one taken
on ordinary rows, or the device code would only ever run its fallback. On the
GPU, tests/test_gpu_rmsnorm.py runs the kernel itself."""
import numpy as np
import pytest

F32 = np.float32
U32 = np.uint32
NW = 4  # waves of the norm kernels' workgroups
MAX_SPECIAL = 48


def bits(x):
    return np.asarray(x, F32).view(U32)


def f32(u):
    return np.asarray(u, U32).view(F32)


def serial(a, s):
    """The sequential chain s + a[0] + ... + a[n-1], one rounding per add."""
    s = F32(s)
    for v in np.asarray(a, F32):
        s = F32(s + v)
    return s


def chain_pass(a, s, rl):
    """(ok, s + a[0] + ... + a[m-1]) for m = len(a) <= 64 * NW * rl, as wg_chain_pass<NW, rl>."""
    m = len(a)
    lanes = 64 * NW
    assert m <= lanes * rl
    sb = int(bits(s))
    if not (0x0D800000 <= sb < 0x7F000000):
        return False, s
    av = np.zeros(lanes * rl, F32)
    av[:m] = a
    av = av.reshape(lanes, rl)
    if int(bits(av).max()) >= 0x7F800000:
        return False, s
    tot = np.zeros(lanes, F32)
    for j in range(rl):
        tot = (tot + av[:, j]).astype(F32)
    # in-wave scans (any association: a prediction), wave totals added in wave order
    incl_w = np.concatenate([np.cumsum(tot[64 * w:64 * w + 64], dtype=F32) for w in range(NW)]).astype(F32)
    excl_w = np.concatenate([np.concatenate([[F32(0)], incl_w[64 * w:64 * w + 63]]) for w in range(NW)]).astype(F32)
    off = [F32(0)]
    for w in range(NW):
        off.append(F32(off[-1] + incl_w[64 * w + 63]))
    p0 = np.array([F32(F32(s) + F32(off[g // 64] + excl_w[g])) for g in range(lanes)], F32)
    ef = np.zeros((lanes, rl + 1), U32)
    p = p0.copy()
    for j in range(rl):
        ef[:, j] = bits(p) & 0x7F800000
        p = (p + av[:, j]).astype(F32)
    ef[:lanes - 1, rl] = bits(p0[1:]) & 0x7F800000
    for w in range(NW):  # a wave's last lane: the next wave's first prediction
        ef[64 * w + 63, rl] = int(bits(F32(F32(s) + off[w + 1]))) & 0x7F800000
    assert all(ef[64 * w + 63, rl] == ef[64 * w + 64, 0] for w in range(NW - 1))
    inv_u = f32((0x8A800000 - ef[:, :rl].astype(np.int64)).astype(U32))
    with np.errstate(over="ignore", invalid="ignore"):
        q = (av * inv_u).astype(F32)
        r = np.rint(np.clip(q, 0, 4294967040)).astype(np.uint64).astype(U32)
        frac = (q - np.floor(q)).astype(F32)
    sp = (ef[:, :rl] != ef[:, 1:]) | (frac == F32(0.5))
    sp[(np.arange(lanes)[:, None] * rl + np.arange(rl)[None, :]) >= m] = False  # only real terms (as the device code)
    r = np.where(sp, U32(0), r)
    racc = np.sum(r, axis=1, dtype=U32)
    cum = (np.cumsum(r, axis=1, dtype=U32) - r).astype(U32)  # before term j
    incl = np.cumsum(racc, dtype=U32)
    excl = (incl - racc).astype(U32)
    total = int(incl[-1])
    S = (sb & 0x7FFFFF) | 0x800000
    Ef = sb & 0x7F800000
    bstart = 0
    specials = list(zip(*np.nonzero(sp)))  # lane-major, term order within a lane
    if len(specials) > MAX_SPECIAL:  # the plain chain is cheaper than more special terms
        return False, s
    # the binade predicted before each special term is the one predicted after
    # the previous (s's own for the first): the device code relies on it
    for k, (L, J) in enumerate(specials):
        assert int(ef[L, J]) == (Ef if k == 0 else int(ef[specials[k - 1][0], specials[k - 1][1] + 1]))
    ok = True
    for L, J in specials:  # only the f32 adds are sequential; the checks could run after
        before = (int(excl[L]) + int(cum[L, J])) & 0xFFFFFFFF
        pre = (before - bstart) & 0xFFFFFFFF
        X = S + pre
        se = F32(F32(X & 0xFFFFFFFF) * f32((Ef - (23 << 23)) & 0xFFFFFFFF))
        nb = int(bits(F32(se + F32(a[rl * L + J]))))
        ok &= pre < 1 << 24 and X < 1 << 24 and 0x0D800000 <= nb < 0x7F000000 and (nb & 0x7F800000) == int(ef[L, J + 1])
        Ef = int(ef[L, J + 1])
        S = (nb & 0x7FFFFF) | 0x800000
        bstart = before
    if not ok:
        return False, s
    pre = (total - bstart) & 0xFFFFFFFF
    if pre > 1 << 24 or S + pre > 1 << 24:
        return False, s
    return True, F32(F32(S + pre) * f32(Ef - (23 << 23)))


def chain_nonneg(a, s, stats=None):
    """wg_chain_nonneg<4>: 16 plain terms, then passes of up to 4096 terms (4 or
    8 per lane when that covers them, else 16) while at least 512 remain, then
    the plain chain."""
    a = np.asarray(a, F32)
    n = len(a)
    if n < 16 + 512:
        return serial(a, s)
    s = serial(a[:16], s)
    i = 16
    while n - i >= 512:
        m = min(64 * NW * 16, n - i)
        rl = next(r for r in (4, 8, 16) if m <= 64 * NW * r)
        ok, out = chain_pass(a[i:i + m], s, rl)
        if stats is not None:
            stats.append(ok)
        s = out if ok else serial(a[i:i + m], s)
        i += m
    return serial(a[i:], s) if n > i else s


def family(kind, n, rng):
    g = rng.standard_normal(n).astype(F32)
    if kind == "squares":
        return (g * g).astype(F32)
    if kind == "small_squares":
        x = (g * F32(0.02)).astype(F32)
        return (x * x).astype(F32)
    if kind == "softmax":
        return np.exp(-rng.uniform(0, 20, n)).astype(F32)
    if kind == "ones_past_2p24":  # every term a tie once the sum passes 2^24
        return np.ones(n, F32)
    if kind == "quarters":
        return (rng.integers(0, 4, n) * 0.25).astype(F32)
    if kind == "powers_of_two":
        return np.ldexp(F32(1), rng.integers(-30, 30, n)).astype(F32)
    if kind == "huge_jumps":
        return np.where(rng.integers(0, 50, n) == 0, F32(1e30), rng.random(n)).astype(F32)
    if kind == "negatives":
        return np.where(rng.integers(0, 200, n) == 0, -rng.random(n), rng.random(n)).astype(F32)
    if kind == "nan_inf":
        x = rng.random(n).astype(F32)
        x[rng.integers(0, n, 2)] = [np.inf, np.nan]
        return x
    if kind == "subnormal":
        return np.ldexp(rng.random(n), -140).astype(F32)
    if kind == "near_overflow":
        return (rng.random(n) * 3e37).astype(F32)
    if kind == "halves":
        return (rng.integers(0, 3, n) + 0.5).astype(F32)
    if kind == "near_powers":  # sums that sit just below powers of two: mispredictions
        x = (rng.random(n) * 1e-6).astype(F32)
        x[::64] = (np.ldexp(F32(1), rng.integers(0, 8, len(x[::64]))) * (1 - 1e-7 * rng.integers(0, 40, len(x[::64]))))
        return x.astype(F32)
    raise ValueError(kind)


KINDS = ["squares", "small_squares", "softmax", "ones_past_2p24", "quarters", "powers_of_two", "huge_jumps",
         "negatives", "nan_inf", "subnormal", "near_overflow", "halves", "near_powers"]


def same(x, y):
    x, y = F32(x), F32(y)
    return (np.isnan(x) and np.isnan(y)) or int(bits(x)) == int(bits(y))


@pytest.mark.parametrize("kind", KINDS)
def test_chain_matches_sequential_sum(kind):
    rng = np.random.default_rng(KINDS.index(kind))
    for t in range(8):
        n = int(rng.choice([640, 1100, 2048, 2176, 2560, 4096, 5000, 8192]))
        a = family(kind, n, rng)
        s0 = F32(1 << 24) if kind == "ones_past_2p24" else (F32(rng.random() * 10) if t % 3 == 0 else F32(0))
        want = F32(np.add.accumulate(np.concatenate([[s0], a]).astype(F32), dtype=F32)[-1])
        assert same(want, serial(a, s0))
        got = chain_nonneg(a, s0)
        assert same(got, want), f"{kind} n={n}: {got!r} vs {want!r}"


def test_ordinary_rows_take_the_fast_path():
    rng = np.random.default_rng(7)
    stats = []
    for n in (2048, 2560, 4096):
        for _ in range(6):
            x = rng.standard_normal(n).astype(F32)
            chain_nonneg((x * x).astype(F32), F32(0), stats)
    assert len(stats) == 18 and all(stats), f"{stats.count(False)} of {len(stats)} passes fell back"  # one pass per row


def test_a_planted_rounding_slip_is_caught():
    """The bit-exact comparison has teeth: rounding every term down instead
    of to nearest changes the sum of ordinary squares."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal(2048).astype(F32)
    a = (x * x).astype(F32)
    want = serial(a, F32(0))
    s = serial(a[:128], F32(0))
    sb = int(bits(s))
    S = (sb & 0x7FFFFF) | 0x800000
    inv_u = f32(0x8A800000 - (sb & 0x7F800000))
    slip = S + int(np.floor(a[128:512] * inv_u).astype(np.int64).sum())
    assert not same(F32(F32(slip) * f32((sb & 0x7F800000) - (23 << 23))), serial(a[:512], F32(0)))
    assert same(chain_nonneg(a, F32(0)), want)
