"""GPU parity of the device-resident Llama-family decode (nrq_model_*) and of
its math functions against the CPU oracle's restatement of
crates/nr-model/src/infer.rs, bit for bit.

The full-size case is the Llama-3.2-1B architecture, all Q8_0, random init
(16 layers, hidden 2048, 32 query / 8 KV heads of 64, SwiGLU 8192, tied
128256-token head, RMSNorm eps 1e-5, adjacent RoPE theta 500000, norms 1.0):
the KV cache is filled with 1024 seeded random token ids, then 128 tokens are
generated greedily; the tokens, the last logits and the f16 KV cache must be
identical to the oracle's.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=1000, norm_eps=1e-5,
            rope_theta=500000.0)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitwise(got, want, what=""):
    g, w = bits(got), bits(want)
    if not np.array_equal(g, w):
        bad = np.nonzero(g != w)[0]
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ; first at {i}: "
                             f"{g[i:i + 1].view(np.float32)} vs {w[i:i + 1].view(np.float32)}")


def math_inputs():
    rng = np.random.default_rng(11)
    xs = [rng.uniform(-110, 95, 400000), rng.uniform(-3, 3, 200000), rng.uniform(-1e-3, 1e-3, 50000),
          rng.uniform(-1200, 1200, 300000),
          np.array([0.0, -0.0, 1e-45, -1e-45, 1e-38, 88.72283, 88.7229, -87.33655, -103.97208, -104.0, 1e30, -1e30,
                    np.inf, -np.inf, np.nan, 0.5 * np.log(2), 1.5 * np.log(2), np.pi / 4, 3 * np.pi / 4,
                    5 * np.pi / 4, 7 * np.pi / 4, 9 * np.pi / 4])]
    return np.concatenate(xs).astype(np.float32)


def test_device_expf_sincosf_bitexact(gpu, oracle):
    """The device restatements of expf and sincosf return the oracle's bits
    on ~1M inputs: the range softmax/swiglu/rope use, extremes, the branch
    boundaries, zeros, subnormals, inf and NaN."""
    import torch

    from nightrun_amd import model

    x = math_inputs()
    xd = torch.from_numpy(x).cuda()
    e = model.mathf(0, xd).cpu().numpy()
    s = model.mathf(1, xd).cpu().numpy()
    c = model.mathf(2, xd).cpu().numpy()
    we = oracle.expf_array(x)
    ws, wc = oracle.sincosf_array(x)
    for got, want, name in ((e, we, "expf"), (s, ws, "sin"), (c, wc, "cos")):
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), name
        assert_bitwise(got[~nan], want[~nan], name)


def top2_gap(logits):
    """Largest minus second-largest logit: the distance a numeric difference
    would have to move a logit to change the greedy token."""
    t = np.sort(np.asarray(logits, np.float64))[-2:]
    return float(t[1] - t[0])


def run_pair(oracle, cfg, weights, ctx, prompt, n_gen, check_kv=True, prefill=False):
    """Feeds `prompt` then generates n_gen tokens greedily on both sides.
    The oracle takes the prompt in 64-token prefill chunks; the GPU one
    forward step at a time, or with `prefill` in its own 64-token batched
    chunks (bitwise equal by the reference's prefill invariant,
    crates/nr-model/tests/prefill.rs)."""
    from nightrun_amd.model import Model

    ref = oracle.Model(cfg, weights, ctx=ctx, threads=THREADS)
    want_logits = ref.prefill(prompt)
    ref_prompt_logits = want_logits.copy()
    tok = oracle.argmax(want_logits)
    want_tokens = []
    gaps = []  # top-2 logit margin of each greedy choice
    for _ in range(n_gen):
        want_tokens.append(tok)
        gaps.append(top2_gap(want_logits))
        want_logits = ref.forward(tok)
        tok = oracle.argmax(want_logits)
    want_tokens.append(tok)
    gaps.append(top2_gap(want_logits))
    print(f"top-2 logit gap over {len(gaps)} greedy choices: min {min(gaps):.6g}, median {np.median(gaps):.6g}")

    m = Model(cfg, ctx)
    try:
        m.set_weights(weights)
        if prefill:
            lg = m.prefill(prompt)
            assert m.pos == len(prompt)
            assert_bitwise(lg, ref_prompt_logits, "prompt logits")
        else:
            for i, t in enumerate(prompt):
                lg = m.forward(int(t), logits=(i == len(prompt) - 1))
        first = oracle.argmax(lg) if lg is not None else None  # vec.rs:80-90: NaN never wins
        # the first generated token comes from the prompt's last logits
        assert first == want_tokens[0], (first, want_tokens[0])
        got_tokens, last = m.generate(first, n_gen, logits=True)
        assert m.pos == len(prompt) + n_gen
        assert [first] + list(got_tokens) == want_tokens, f"greedy tokens differ (min top-2 gap {min(gaps):.6g})"
        assert_bitwise(last, want_logits, "last logits")
        if check_kv:
            k, v = m.kv_cache()
            rk, rv = ref.kv_cache()
            assert np.array_equal(k, rk) and np.array_equal(v, rv), "KV cache differs"
    finally:
        m.close()


def test_tiny_model_forward_and_generate(gpu, oracle):
    """2 layers, GQA 4:2, 70 prompt tokens across a 64-token chunk boundary,
    20 greedy steps, all Q8_0."""
    w = oracle.gen_model(TINY, 1234)
    prompt = np.random.default_rng(1).integers(0, TINY["vocab"], 70).astype(np.uint32)
    run_pair(oracle, TINY, w, 128, prompt, 20)


@pytest.mark.parametrize("case", ["all_equal", "two_best_and_nan"])
def test_greedy_pick_ties_and_nan(gpu, oracle, case):
    """The greedy pick (vec.rs:80-90: the first index of the largest logit,
    NaN never chosen) over the head launch's workgroups, which each leave the
    pick of their own rows: every row of the tied head equal (every logit
    ties, token 0), or all rows zero but two equal ones in different
    workgroups and one whose scale is NaN."""
    w = oracle.gen_model(TINY, 4321)
    e = w["embed"].reshape(TINY["vocab"], -1, 34).copy()
    if case == "all_equal":
        e[:] = e[7]
        prompt = [3, 9, 27]
    else:
        keep = e[123].copy()
        e[:] = 0
        e[300] = keep
        e[700] = keep
        e[5, :, 0:2] = np.array([0x7E00], dtype=np.uint16).view(np.uint8)  # f16 NaN scales
        prompt = [300, 700, 300, 1]
    w["embed"] = e.reshape(w["embed"].shape)
    run_pair(oracle, TINY, w, 64, np.array(prompt, dtype=np.uint32), 6)


def test_step_profile_is_a_forward_step(gpu, oracle):
    """nrq_model_step_profile runs the same step as nrq_model_forward (the
    next step's logits are bitwise the same either way) and reports a positive
    time for every stage but the unused ones."""
    from nightrun_amd.model import Model

    w = oracle.gen_model(TINY, 77)
    prompt = np.random.default_rng(3).integers(0, TINY["vocab"], 9).astype(np.uint32)
    out = []
    for profiled in (False, True):
        m = Model(TINY, 64)
        try:
            m.set_weights(w)
            m.prefill(prompt, logits=False)
            if profiled:
                st = m.step_profile(5)
                assert set(st) == set(Model.STEP_STAGES)
                for k in ("embed", "norm_qkv", "attention", "o", "norm_gate_up_swiglu", "down", "head",
                          "argmax_or_sampler"):
                    assert st[k] > 0.0, (k, st)
            else:
                m.forward(5, logits=False)
            assert m.pos == 10
            out.append(m.forward(7))
        finally:
            m.close()
    assert_bitwise(out[1], out[0], "logits after a profiled step")


def test_tiny_model_logits_every_step(gpu, oracle):
    """Logits of every forward step equal the oracle's (not only the argmax)."""
    from nightrun_amd.model import Model

    w = oracle.gen_model(TINY, 99)
    ref = oracle.Model(TINY, w, ctx=64, threads=THREADS)
    m = Model(TINY, 64)
    try:
        m.set_weights(w)
        for i, t in enumerate(np.random.default_rng(3).integers(0, TINY["vocab"], 40)):
            assert_bitwise(m.forward(int(t)), ref.forward(int(t)), f"step {i}")
    finally:
        m.close()


def test_tiny_model_kquant_weights(gpu, oracle):
    """Q4_K attention/gate/up and Q6_K down weights (Q8_K activations), Q8_0
    embedding and head: the Qwen3 / Granite Q4_K_M weight mix on the Llama
    recipe."""
    w = oracle.gen_model(TINY, 4321)
    shapes = oracle.layer_shapes(TINY)
    for l, lw in enumerate(w["layers"]):
        for i, name in enumerate(oracle.LAYER_MATS):
            dt = 3 if name == "w_down" else 2
            rows, cols = shapes[name]
            lw[name] = oracle.gen_weights(dt, 777 + 16 * l + i, rows, cols)
            lw["dtypes"][name] = dt
    prompt = np.random.default_rng(2).integers(0, TINY["vocab"], 9).astype(np.uint32)
    run_pair(oracle, TINY, w, 64, prompt, 12)


MIXES = {
    # a Q4_K_M file: q, k, o, gate, up Q4_K; v and down Q6_K (q|k and gate|up
    # go out as grouped launches, v alone on the other activation format)
    "q4k_m": {"wq": 2, "wk": 2, "wv": 3, "wo": 2, "w_gate": 2, "w_up": 2, "w_down": 3},
    # Q6_K gate|up (the Q6_K grouped launch), Q8_0 q/k/v with a Q4_K o and down
    "q6k_ffn": {"wq": 1, "wk": 1, "wv": 1, "wo": 2, "w_gate": 3, "w_up": 3, "w_down": 2},
    # Q8_0 gate|up into a Q4_K down (swiglu without the fused Q8_0 epilogue)
    "q8_into_q4k": {"wq": 2, "wk": 3, "wv": 2, "wo": 1, "w_gate": 1, "w_up": 1, "w_down": 2},
}


@pytest.mark.parametrize("prefill", [False, True])
@pytest.mark.parametrize("mix", sorted(MIXES))
def test_tiny_model_format_mixes(gpu, oracle, mix, prefill):
    """Per-matrix format mixes the grouping logic must split correctly:
    logits, tokens and KV cache bit-identical to the oracle in decode and in
    the batched prefill."""
    w = oracle.gen_model(TINY, 5151)
    shapes = oracle.layer_shapes(TINY)
    for l, lw in enumerate(w["layers"]):
        for i, name in enumerate(oracle.LAYER_MATS):
            dt = MIXES[mix][name]
            rows, cols = shapes[name]
            lw[name] = oracle.gen_weights(dt, 901 + 16 * l + i, rows, cols)
            lw["dtypes"][name] = dt
    prompt = np.random.default_rng(7).integers(0, TINY["vocab"], 70).astype(np.uint32)
    run_pair(oracle, TINY, w, 96, prompt, 10, prefill=prefill)


def test_context_exhausted_panics(gpu, oracle):
    """infer.rs:513: forward past the context asserts."""
    from nightrun_amd import NrPanic
    from nightrun_amd.model import Model

    w = oracle.gen_model(TINY, 5)
    m = Model(TINY, 3)
    try:
        m.set_weights(w)
        for t in (1, 2, 3):
            m.forward(t, logits=False)
        with pytest.raises(NrPanic, match="context window exhausted"):
            m.forward(4, logits=False)
    finally:
        m.close()


def test_llama_1b_greedy_token_identical(gpu, oracle):
    """The full-model benchmark: Llama-3.2-1B architecture, all Q8_0, KV
    filled to 1024 positions, 128 greedy tokens identical to the oracle's,
    with the same last logits and KV cache."""
    cfg = oracle.LLAMA_1B
    w = oracle.gen_model(cfg, 0x5EED0005)
    prompt = np.random.default_rng(0x5EED0005).integers(0, cfg["vocab"], 1024).astype(np.uint32)
    run_pair(oracle, cfg, w, 1152, prompt, 128, prefill=True)


WIDE = dict(dim=2048, n_layers=1, n_heads=32, n_kv_heads=8, head_dim=64, ffn_dim=256, vocab=300, norm_eps=1e-5,
            rope_theta=500000.0)


def q8_0_row(q, d_bits):
    """One embedding row of Q8_0 blocks: q (int8 values, len a multiple of 32)
    with the f16 scale bits d_bits per block."""
    q = np.asarray(q, np.int64).reshape(-1, 32)
    d = np.broadcast_to(np.asarray(d_bits, np.uint16), (q.shape[0],))
    out = np.zeros((q.shape[0], 34), np.uint8)
    out[:, 0] = d & 0xFF
    out[:, 1] = d >> 8
    out[:, 2:] = (q & 0xFF).astype(np.uint8)
    return out


@pytest.mark.parametrize("fmt", ["q8_0", "q4k_m"])
@pytest.mark.parametrize("prefill", [False, True])
def test_wide_norm_sums_on_crafted_rows(gpu, oracle, fmt, prefill):
    """Hidden width 2048, so the fused norms' sum of squares takes the
    wave-parallel exact path. The prompt's embedding rows are crafted for
    it: after a large first value every square is an exact tie (the pass gives
    up past 48 special terms and falls back), squares mixing ties and exact
    multiples of the unit, a ramp crossing binades late, and an ordinary row.
    Logits and KV bit-identical to the oracle."""
    w = oracle.gen_model(WIDE, 6161)
    if fmt == "q4k_m":
        shapes = oracle.layer_shapes(WIDE)
        for l, lw in enumerate(w["layers"]):
            for i, name in enumerate(oracle.LAYER_MATS):
                dt = MIXES["q4k_m"][name]
                rows, cols = shapes[name]
                lw[name] = oracle.gen_weights(dt, 611 + 16 * l + i, rows, cols)
                lw["dtypes"][name] = dt
    dim, nb = WIDE["dim"], WIDE["dim"] // 32
    emb = w["embed"].reshape(WIDE["vocab"], nb, 34)
    rng = np.random.default_rng(61)
    # f16 0x3000 = 0.125, 0x1800 = 2^-9
    big_then_ties = np.ones(dim, np.int64)
    big_then_ties[0] = 80  # x = 10 (d 0.125): the sum sits at 100, unit 2^-17
    emb[1] = np.concatenate([q8_0_row(big_then_ties[:32], 0x3000), q8_0_row(big_then_ties[32:], 0x1800)])
    mixed = rng.integers(1, 4, dim)  # squares (q * 2^-9)^2: q = 1, 3 ties, q = 2 exact
    mixed[0] = 80
    emb[2] = np.concatenate([q8_0_row(mixed[:32], 0x3000), q8_0_row(mixed[32:], 0x1800)])
    ramp = np.clip(np.round(np.sqrt(np.linspace(1, 16000, dim))), 1, 127).astype(np.int64) * rng.choice([-1, 1], dim)
    emb[3] = q8_0_row(ramp, 0x2000)  # d = 2^-7
    prompt = np.array([1, 2, 3, 4, 1, 3], np.uint32)  # token 4: an ordinary generated row
    run_pair(oracle, WIDE, w, 32, prompt, 4, prefill=prefill)


@pytest.mark.parametrize("ctx", [1024, 4096])
def test_tiny_model_long_context(gpu, oracle, ctx):
    """700 prompt positions (six 128-position chunks of the decode attention's
    value loop), in a 1024- and a 4096-position cache (the attention's LDS
    holds ctx scores): prefill and 12 greedy steps bit-exact with the oracle."""
    w = oracle.gen_model(TINY, 3100 + ctx)
    prompt = np.random.default_rng(ctx).integers(0, TINY["vocab"], 700).astype(np.uint32)
    run_pair(oracle, TINY, w, ctx, prompt, 12, prefill=True)


TINY8 = dict(TINY, dim=512, n_heads=8, n_kv_heads=2)
QWEN8_HD128 = dict(dim=1024, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=512, vocab=1000,
                   norm_eps=1e-6, rope_theta=1000000.0, recipe=dict(rope="neox"))


@pytest.mark.parametrize("split", ["default", "1"])
@pytest.mark.parametrize("cfg", [TINY8, QWEN8_HD128], ids=["hd64", "qwen-hd128"])
def test_decode_attention_dimension_split(gpu, oracle, monkeypatch, cfg, split):
    """Eight heads: the decode attention runs 32 value dimensions per
    workgroup (two per 64-wide head, four per 128-wide Qwen3 head with its
    q/k norms, 256-position value chunks) by default, one workgroup per head
    with NRQ_ATT_SPLIT=1. 1100 prompt positions, so the split kernel's value
    loop runs five chunks and reuses every ring slot; then 12 greedy steps,
    each bit-exact against the oracle."""
    if split == "1":
        monkeypatch.setenv("NRQ_ATT_SPLIT", split)
    qk = "recipe" in cfg
    w = oracle.gen_model(cfg, 5150, qk_norm=qk)
    prompt = np.random.default_rng(5150).integers(0, cfg["vocab"], 1100).astype(np.uint32)
    run_pair(oracle, cfg, w, 2048, prompt, 12, prefill=True)


# Q4_K_M's layer formats: q, k, o, gate, up Q4_K; v, down Q6_K
Q4K_M = {"wq": 2, "wk": 2, "wv": 3, "wo": 2, "w_gate": 2, "w_up": 2, "w_down": 3}


@pytest.mark.parametrize("prefill", [False, True], ids=["decode", "prefill"])
def test_qwen3_q4k_m_layer_formats(gpu, oracle, prefill):
    """Qwen3 (q/k norms, Neox rope, 128-wide heads) with the Q4_K_M layer
    formats: in the decode step the fused norm + q|k launch (Q4_K) also stores
    the Q8_K activation that v's Q6_K matvec reads, and the Q6_K down
    projection takes swiglu from the Q8_K quantizer. Logits, tokens and the KV
    cache bit-exact against the oracle."""
    cfg = QWEN8_HD128
    w = oracle.gen_model(cfg, 4242, qk_norm=True)
    shapes = oracle.layer_shapes(cfg)
    for l, lw in enumerate(w["layers"]):
        for i, name in enumerate(oracle.LAYER_MATS):
            rows, cols = shapes[name]
            lw[name] = oracle.gen_weights(Q4K_M[name], 4300 + 16 * l + i, rows, cols)
            lw["dtypes"][name] = Q4K_M[name]
    prompt = np.random.default_rng(4242).integers(0, cfg["vocab"], 70).astype(np.uint32)
    run_pair(oracle, cfg, w, 128, prompt, 8, prefill=prefill)


@pytest.mark.parametrize("n", [1, 5, 63, 64, 65, 70, 130])
def test_tiny_model_prefill(gpu, oracle, n):
    """Device prefill (64-token batched chunks) == the oracle's prefill: the
    prompt's last logits, the KV cache, and the greedy continuation."""
    w = oracle.gen_model(TINY, 2000 + n)
    prompt = np.random.default_rng(n).integers(0, TINY["vocab"], n).astype(np.uint32)
    run_pair(oracle, TINY, w, 160, prompt, 6, prefill=True)


TINY_GQA4 = dict(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=1000, norm_eps=1e-5,
                 rope_theta=500000.0)


@pytest.mark.parametrize("group", ["1", "0"])
def test_prefill_attention_paths(gpu, oracle, monkeypatch, group):
    """Prefill attention with one workgroup per KV group (all its query heads,
    the default for head_dim 64) and with one workgroup per query head
    (NRQ_ATT_GROUP=0): GQA 4:1 and 2:1, prompts across a chunk boundary."""
    monkeypatch.setenv("NRQ_ATT_GROUP", group)
    for cfg, seed in ((TINY_GQA4, 41), (TINY, 42)):
        w = oracle.gen_model(cfg, seed)
        prompt = np.random.default_rng(seed).integers(0, cfg["vocab"], 100).astype(np.uint32)
        run_pair(oracle, cfg, w, 128, prompt, 4, prefill=True)


def test_tiny_model_prefill_kquant(gpu, oracle):
    """Q4_K q/k/v/o/gate/up and Q6_K down (Q8_K activations through the 32x32
    MFMA kernels), an untied Q6_K head."""
    w = oracle.gen_model(TINY, 4322)
    shapes = oracle.layer_shapes(TINY)
    for l, lw in enumerate(w["layers"]):
        for i, name in enumerate(oracle.LAYER_MATS):
            dt = 3 if name == "w_down" else 2
            rows, cols = shapes[name]
            lw[name] = oracle.gen_weights(dt, 1777 + 16 * l + i, rows, cols)
            lw["dtypes"][name] = dt
    w["output"] = oracle.gen_weights(3, 4444, TINY["vocab"], TINY["dim"])
    w["output_dtype"] = 3
    prompt = np.random.default_rng(9).integers(0, TINY["vocab"], 100).astype(np.uint32)
    run_pair(oracle, TINY, w, 128, prompt, 5, prefill=True)


def test_prefill_after_decode_steps(gpu, oracle):
    """Prefill at a non-zero position: forward steps, then a 67-token prefill
    (chunks of 64 and 3 starting at position 3), then decode."""
    from nightrun_amd.model import Model

    w = oracle.gen_model(TINY, 77)
    toks = np.random.default_rng(77).integers(0, TINY["vocab"], 70).astype(np.uint32)
    ref = oracle.Model(TINY, w, ctx=96, threads=THREADS)
    m = Model(TINY, 96)
    try:
        m.set_weights(w)
        for t in toks[:3]:
            assert_bitwise(m.forward(int(t)), ref.forward(int(t)), "forward")
        assert_bitwise(m.prefill(toks[3:]), ref.prefill(toks[3:]), "prefill at position 3")
        assert m.pos == 70
        k, v = m.kv_cache()
        rk, rv = ref.kv_cache()
        assert np.array_equal(k, rk) and np.array_equal(v, rv), "KV cache differs"
        assert_bitwise(m.forward(5), ref.forward(5), "decode after prefill")
    finally:
        m.close()


def test_prefill_context_exhausted_panics(gpu, oracle):
    """infer.rs:605: a chunk past the context asserts; an empty prompt asserts (infer.rs:754)."""
    from nightrun_amd import NrPanic
    from nightrun_amd.model import Model

    w = oracle.gen_model(TINY, 6)
    m = Model(TINY, 40)
    try:
        m.set_weights(w)
        m.prefill(np.arange(30, dtype=np.uint32), logits=False)
        with pytest.raises(NrPanic, match="context window exhausted"):
            m.prefill(np.arange(11, dtype=np.uint32), logits=False)
        with pytest.raises(NrPanic, match="is_empty"):
            m.prefill(np.arange(0, dtype=np.uint32), logits=False)
        assert m.pos == 30
    finally:
        m.close()


# ---- the Qwen3 / Granite recipe (infer.rs:383-461): qk-norm, Neox rope, muP ----------

MUP = dict(embed_scale=1.6, attn_scale=0.3, residual_scale=0.6, logit_scale=2.5)
QWEN_HD64 = dict(TINY, rope_theta=10000.0, recipe=dict(rope="neox", **MUP))
QWEN_HD128 = dict(dim=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128, ffn_dim=512, vocab=1000,
                  norm_eps=1e-6, rope_theta=1000000.0, recipe=dict(rope="neox"))
GRANITE = dict(TINY, recipe=dict(rope="adjacent", embed_scale=12.0, attn_scale=0.0, residual_scale=0.22,
                                 logit_scale=8.0))


@pytest.mark.parametrize("cfg", [QWEN_HD64, QWEN_HD128], ids=["hd64-mup", "hd128"])
@pytest.mark.parametrize("prefill", [False, True], ids=["decode", "prefill"])
def test_qwen3_recipe_matches_oracle(gpu, oracle, cfg, prefill):
    """Per-head q/k RMSNorm before Neox rope, in the decode attention kernel
    and in the prefill rope kernel; with muP scalars on the head_dim 64 model.
    70 prompt tokens cross a prefill chunk boundary."""
    w = oracle.gen_model(cfg, 606, qk_norm=True)
    prompt = np.random.default_rng(606).integers(0, cfg["vocab"], 70).astype(np.uint32)
    run_pair(oracle, cfg, w, 128, prompt, 10, prefill=prefill)


LLAMA_HD96 = dict(dim=768, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=96, ffn_dim=512, vocab=1000,
                  norm_eps=1e-5, rope_theta=500000.0)
QWEN_HD96 = dict(LLAMA_HD96, norm_eps=1e-6, rope_theta=1000000.0, recipe=dict(rope="neox"))


@pytest.mark.parametrize("cfg", [LLAMA_HD96, QWEN_HD96, QWEN_HD128], ids=["llama-hd96", "qwen-hd96", "qwen-hd128"])
@pytest.mark.parametrize("prefill", [False, True], ids=["decode", "prefill"])
def test_wide_heads_long_context(gpu, oracle, cfg, prefill):
    """96- and 128-wide heads (768-thread attention, 64-position value chunks
    in a three-slot ring) over 330 prompt positions, six chunks, so every ring
    slot is reused; the Qwen3 models take the early LDS staging of the step's
    own rows in decode. Then 8 greedy steps; logits, tokens and the KV cache
    bit-exact against the oracle."""
    qk = "recipe" in cfg
    w = oracle.gen_model(cfg, 808 + cfg["head_dim"] + 2 * qk, qk_norm=qk)
    prompt = np.random.default_rng(cfg["head_dim"]).integers(0, cfg["vocab"], 330).astype(np.uint32)
    run_pair(oracle, cfg, w, 512, prompt, 8, prefill=prefill)


def test_granite_recipe_kquant_matches_oracle(gpu, oracle):
    """Adjacent rope and muP scalars with Q4_K/Q6_K layers: the residual scale
    is applied by the fused K-quant norm + matvec launches in decode and by
    norm_kernel in prefill."""
    w = oracle.gen_model(GRANITE, 707)
    shapes = oracle.layer_shapes(GRANITE)
    for l, lw in enumerate(w["layers"]):
        for i, name in enumerate(oracle.LAYER_MATS):
            dt = 3 if name == "w_down" else 2
            rows, cols = shapes[name]
            lw[name] = oracle.gen_weights(dt, 2777 + 16 * l + i, rows, cols)
            lw["dtypes"][name] = dt
    prompt = np.random.default_rng(707).integers(0, GRANITE["vocab"], 40).astype(np.uint32)
    run_pair(oracle, GRANITE, w, 96, prompt, 8)
    run_pair(oracle, GRANITE, w, 96, prompt, 8, prefill=True)


def test_recipe_rejects_bad_scales_and_unpaired_norms(gpu, oracle):
    """nrq_model_set_recipe takes the ranges Model::parse accepts; a layer with
    attn_q_norm but no attn_k_norm is refused at the first step."""
    from nightrun_amd import NrqError
    from nightrun_amd.model import ATTN_Q_NORM, F32, ROPE_NEOX, Model

    m = Model(TINY, 32)
    try:
        for bad in ((7, 1.0, 0.0, 1.0, 1.0), (ROPE_NEOX, 1.0, -0.5, 1.0, 1.0), (ROPE_NEOX, 1.0, 0.0, 0.0, 1.0),
                    (ROPE_NEOX, float("nan"), 0.0, 1.0, 1.0), (ROPE_NEOX, 1.0, 0.0, 1.0, 0.0)):
            with pytest.raises(NrqError, match="rope style|out of range"):
                m.set_recipe(*bad)
        m.set_weights(oracle.gen_model(TINY, 808))
        m._bind(ATTN_Q_NORM, 0, F32, np.ones(TINY["head_dim"], np.float32))
        with pytest.raises(NrqError, match="pair"):
            m.forward(1)
    finally:
        m.close()


@pytest.mark.parametrize("edt", [2, 3], ids=["q4k", "q6k"])
def test_kquant_embedding_matches_oracle(gpu, oracle, edt):
    """A Q4_K or Q6_K token embedding (QMat::dequant_row, infer.rs:36-56,
    kquant.rs:95-142), tied to the head: every element of the dequantized row
    feeds the first norm, so decode and prefill logits pin the element maps."""
    w = oracle.gen_model(TINY, 909 + edt)
    w["embed"] = oracle.gen_weights(edt, 9090 + edt, TINY["vocab"], TINY["dim"])
    w["embed_dtype"] = edt
    prompt = np.random.default_rng(edt).integers(0, TINY["vocab"], 30).astype(np.uint32)
    run_pair(oracle, TINY, w, 64, prompt, 6)
    run_pair(oracle, TINY, w, 64, prompt, 6, prefill=True)
