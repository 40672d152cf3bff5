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


# ---- the Qwen3 / Granite recipe (infer.rs:383-461, 515-595, 608-750) ----------------

QWEN = dict(TINY, rope_theta=10000.0,
            recipe=dict(rope="neox", embed_scale=1.6, attn_scale=0.3, residual_scale=0.6, logit_scale=2.5))
LAYER_MATS = ["wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"]


def f64_logits(oracle, cfg, w, tokens, mistake=None):
    """InferCtx::forward in float64 over the dequantized weights (no
    activation quantization, no f16 cache rounding): logits after each token.
    `mistake` plants one plausible error in this float64 reference."""
    r = cfg.get("recipe", {})
    d, hd, nh, nkv = cfg["dim"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv_heads"]
    eps, V = cfg["norm_eps"], cfg["vocab"]
    neox = r.get("rope") == "neox" and mistake != "adjacent"
    es = 1.0 if mistake == "no_embed_scale" else r.get("embed_scale", 1.0)
    rs = 1.0 if mistake == "no_residual_scale" else r.get("residual_scale", 1.0)
    att = r.get("attn_scale", 0.0) or 1.0 / np.sqrt(hd)
    if mistake == "default_attn_scale":
        att = 1.0 / np.sqrt(hd)
    ls = 1.0 if mistake == "no_logit_scale" else r.get("logit_scale", 1.0)
    deq = lambda b, rows, cols: oracle.dequantize_q8_0(b).astype(np.float64).reshape(rows, cols)
    E = deq(w["embed"], V, d)
    shapes = oracle.layer_shapes(cfg)
    Ls = [{n: deq(lw[n], *shapes[n]) for n in LAYER_MATS} for lw in w["layers"]]
    rms = lambda x, g: x / np.sqrt(np.mean(x * x) + eps) * g
    freqs = cfg["rope_theta"] ** (-2.0 * np.arange(hd // 2) / hd)

    def rope(v, pos):
        v = v.reshape(-1, hd).copy()
        half = hd // 2
        ia = np.arange(half) if neox else 2 * np.arange(half)
        ib = ia + half if neox else ia + 1
        c, s = np.cos(pos * freqs), np.sin(pos * freqs)
        a, b = v[:, ia].copy(), v[:, ib].copy()
        v[:, ia] = a * c - b * s
        v[:, ib] = a * s + b * c
        return v.reshape(-1)

    K, Vc, out = [[] for _ in Ls], [[] for _ in Ls], []
    for pos, t in enumerate(tokens):
        x = E[t] * es
        for l, (lw, W) in enumerate(zip(w["layers"], Ls)):
            xb = rms(x, lw["attn_norm"].astype(np.float64))
            q, k, v = W["wq"] @ xb, W["wk"] @ xb, W["wv"] @ xb
            if "q_norm" in lw and mistake != "no_qk_norm":
                q = np.concatenate([rms(h, lw["q_norm"].astype(np.float64)) for h in q.reshape(nh, hd)])
                k = np.concatenate([rms(h, lw["k_norm"].astype(np.float64)) for h in k.reshape(nkv, hd)])
            q, k = rope(q, pos), rope(k, pos)
            K[l].append(k)
            Vc[l].append(v)
            Km, Vm = np.array(K[l]), np.array(Vc[l])
            o = []
            for h in range(nh):
                g = h // (nh // nkv)
                sc = Km[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd] * att
                p = np.exp(sc - sc.max())
                o.append(p / p.sum() @ Vm[:, g * hd:(g + 1) * hd])
            x = x + rs * (W["wo"] @ np.concatenate(o))
            xb = rms(x, lw["ffn_norm"].astype(np.float64))
            g_, u = W["w_gate"] @ xb, W["w_up"] @ xb
            x = x + rs * (W["w_down"] @ (g_ / (1 + np.exp(-g_)) * u))
        out.append(E @ rms(x, w["out_norm"].astype(np.float64)) / ls)
    return np.array(out)


def test_rmsnorm_inplace_closed_form(oracle):
    """vec.rs:17-28 against float64; with unit weights it is x * scale, the
    same bits as rmsnorm (vec.rs:4-14) with unit weights."""
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, 128).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    got = oracle.rmsnorm_inplace(x, w, 1e-6).astype(np.float64)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    assert np.max(np.abs(got - want) / np.abs(want)) < 1e-6
    ones = np.ones(128, np.float32)
    assert np.array_equal(oracle.rmsnorm_inplace(x, ones, 1e-6), oracle.rmsnorm(x, ones, 1e-6))


def test_neox_rope_is_adjacent_rope_on_interleaved_halves(oracle):
    """rope.rs:55-58: Neox rotates (x_i, x_{i+half}) exactly as Adjacent
    rotates (x_2i, x_2i+1), so interleaving each head's halves maps one onto
    the other bit for bit; and it is a rotation (norm kept)."""
    hd, half = 64, 32
    freqs = oracle.rope_freqs(hd, 10000.0)
    x = np.random.default_rng(12).normal(0, 1, 3 * hd).astype(np.float32)
    perm = np.concatenate([[h * hd + i, h * hd + i + half] for h in range(3) for i in range(half)])
    for pos in (0, 1, 17, 1000):
        nx = oracle.rope_apply(x, hd, freqs, pos, neox=True)
        ax = oracle.rope_apply(x[perm], hd, freqs, pos)
        assert np.array_equal(nx[perm].view(np.uint32), ax.view(np.uint32))
        assert abs(np.linalg.norm(nx) - np.linalg.norm(x)) < 1e-5 * np.linalg.norm(x)
    assert not np.array_equal(oracle.rope_apply(x, hd, freqs, 5, neox=True), oracle.rope_apply(x, hd, freqs, 5))


def test_neutral_recipe_is_the_llama_recipe(oracle):
    """Adjacent rope, unit scales and attn_scale = 1/sqrtf(head_dim) give the
    Llama logits bit for bit (the Granite code path with neutral scalars)."""
    w = oracle.gen_model(TINY, 21)
    neutral = dict(TINY, recipe=dict(rope="adjacent", embed_scale=1.0, attn_scale=float(np.float32(1 / np.sqrt(64))),
                                     residual_scale=1.0, logit_scale=1.0))
    a, b = oracle.Model(TINY, w, ctx=16), oracle.Model(neutral, w, ctx=16)
    for t in (3, 9, 400):
        assert np.array_equal(a.forward(t).view(np.uint32), b.forward(t).view(np.uint32))


def test_logit_scale_is_one_multiply(oracle):
    """infer.rs:589-591: logits *= 1/logit_scale after the head, exactly."""
    w = oracle.gen_model(TINY, 22)
    a = oracle.Model(TINY, w, ctx=16)
    b = oracle.Model(dict(TINY, recipe=dict(logit_scale=2.5)), w, ctx=16)
    for t in (1, 2):
        la, lb = a.forward(t), b.forward(t)
        assert np.array_equal(lb.view(np.uint32), (la * np.float32(1 / np.float32(2.5))).view(np.uint32))


def test_recipe_forward_against_float64(oracle):
    """Qwen3 qk-norm + Neox rope with muP scalars, eight positions: the
    oracle is within 4% (activation quantization, f16 cache) of a float64
    forward, while each planted mistake moves the float64 logits by more than
    10% at every position past the first."""
    w = oracle.gen_model(QWEN, 77, qk_norm=True)
    toks = np.random.default_rng(5).integers(0, QWEN["vocab"], 8)
    m = oracle.Model(QWEN, w, ctx=16)
    got = np.array([m.forward(int(t)).copy() for t in toks])
    ref = f64_logits(oracle, QWEN, w, toks)
    rel = lambda a, b: np.linalg.norm(a - b) / np.linalg.norm(b)
    for i in range(len(toks)):
        assert rel(got[i], ref[i]) < 0.04, i
    for mistake in ("no_embed_scale", "no_residual_scale", "default_attn_scale", "no_logit_scale", "adjacent",
                    "no_qk_norm"):
        bad = f64_logits(oracle, QWEN, w, toks, mistake)
        assert min(rel(bad[i], ref[i]) for i in range(1, len(toks))) > 0.10, mistake


def test_recipe_prefill_equals_sequential_decode(oracle):
    """The recipe in prefill_chunk (infer.rs:608-750) gives decode's logits
    and KV cache bit for bit, across a chunk boundary."""
    w = oracle.gen_model(QWEN, 1235, qk_norm=True)
    toks = np.random.default_rng(2).integers(0, QWEN["vocab"], 70).astype(np.uint32)
    a = oracle.Model(QWEN, w, ctx=128, threads=4)
    la = a.prefill(toks)
    b = oracle.Model(QWEN, w, ctx=128, threads=4)
    for t in toks:
        lb = b.forward(int(t))
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    ka, va = a.kv_cache()
    kb, vb = b.kv_cache()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
