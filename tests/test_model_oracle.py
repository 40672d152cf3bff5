"""Pins of the oracle's forward-pass pieces (crates/nr-tensor/src/vec.rs,
rope.rs; crates/nr-model/src/infer.rs). The reference's libm crate is not
present, so expf/sincosf are pinned to the correctly rounded values within
1 ulp, and the f32 vector ops against their closed forms in float64."""
import math

import numpy as np
import pytest

TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=1000, norm_eps=1e-5,
            rope_theta=500000.0)


def ulps(got, want64):
    want = np.float32(want64)
    if np.isnan(want):
        return 0 if np.isnan(got) else 1 << 30
    return abs(int(np.float32(got).view(np.int32)) - int(want.view(np.int32)))


def test_expf_within_one_ulp(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-103, 88.7, 20000), rng.uniform(-1, 1, 5000),
                        rng.uniform(-2e-4, 2e-4, 2000)]).astype(np.float32)
    y = oracle.expf_array(x)
    assert max(ulps(g, math.exp(float(v))) for v, g in zip(x, y)) <= 1


def test_expf_special_values(oracle):
    assert oracle.expf(0.0) == 1.0 and oracle.expf(-0.0) == 1.0
    assert oracle.expf(float("-inf")) == 0.0 and oracle.expf(float("inf")) == float("inf")
    assert math.isnan(oracle.expf(float("nan")))
    assert oracle.expf(89.0) == float("inf") and oracle.expf(-104.0) == 0.0
    assert 0.0 < oracle.expf(-100.0) < 1e-43  # subnormal result


def test_sincosf_within_one_ulp(oracle):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-1200, 1200, 20000), rng.uniform(-8, 8, 5000),
                        rng.uniform(-1e-3, 1e-3, 1000)]).astype(np.float32)
    s, c = oracle.sincosf_array(x)
    worst = max(max(ulps(a, math.sin(float(v))), ulps(b, math.cos(float(v)))) for v, a, b in zip(x, s, c))
    assert worst <= 1


def test_rmsnorm_closed_form(oracle):
    x = oracle.Rng(3).normal(2048)
    w = oracle.Rng(4).vec(2048)
    got = oracle.rmsnorm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
    assert np.allclose(got, want, rtol=1e-5, atol=1e-7)


def test_softmax_and_swiglu_closed_form(oracle):
    x = oracle.Rng(5).normal(1100) * np.float32(4)
    p = oracle.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)
    g, u = oracle.Rng(6).normal(512) * np.float32(3), oracle.Rng(7).normal(512)
    g64 = g.astype(np.float64)
    assert np.allclose(oracle.swiglu(g, u), g64 / (1 + np.exp(-g64)) * u, rtol=1e-5, atol=1e-7)


def test_argmax_first_index_nan_never_wins(oracle):
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle.argmax(np.array([np.nan, 2, np.nan, 5, 5], np.float32)) == 3
    assert oracle.argmax(np.array([np.nan, np.nan], np.float32)) == 0
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


def test_rope_is_a_rotation(oracle):
    hd = 64
    f = oracle.rope_freqs(hd, 500000.0)
    assert f[0] == 1.0 and np.all(np.diff(f) < 0)
    assert np.allclose(f, 500000.0 ** (-2 * np.arange(32) / 64), rtol=1e-6)
    x = oracle.Rng(8).normal(4 * hd)
    assert np.array_equal(oracle.rope_apply(x, hd, f, 0), x)  # angle 0: exact identity
    y = oracle.rope_apply(x, hd, f, 777)
    n0 = np.hypot(x[0::2].astype(np.float64), x[1::2])
    n1 = np.hypot(y[0::2].astype(np.float64), y[1::2])
    assert np.allclose(n0, n1, rtol=1e-6)


def test_prefill_equals_sequential_decode(oracle):
    """crates/nr-model/tests/prefill.rs: batched prefill gives the logits AND
    the KV cache of token-by-token decode, bit for bit, across a chunk
    boundary (70 = 64 + 6)."""
    w = oracle.gen_model(TINY, 1234)
    toks = np.random.default_rng(1).integers(0, TINY["vocab"], 70).astype(np.uint32)
    a = oracle.Model(TINY, w, ctx=128, threads=4)
    la = a.prefill(toks)
    b = oracle.Model(TINY, w, ctx=128, threads=4)
    for t in toks:
        lb = b.forward(int(t))
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    assert a.pos == b.pos == 70


def test_forward_is_deterministic_and_uses_history(oracle):
    """Token 5 after token 3 differs from token 5 first (cache + rope); the
    same history replayed gives identical logits."""
    w = oracle.gen_model(TINY, 7)
    a = oracle.Model(TINY, w, ctx=16, threads=1)
    a.forward(3)
    l1 = a.forward(5)
    b = oracle.Model(TINY, w, ctx=16, threads=2)
    assert not np.array_equal(b.forward(5), l1)
    c = oracle.Model(TINY, w, ctx=16, threads=3)
    c.forward(3)
    assert np.array_equal(c.forward(5), l1)
