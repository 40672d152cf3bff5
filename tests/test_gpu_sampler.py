"""Device sampler (nrq_dev_sample, and nrq_model_generate with a sampler set)
against the oracle's Sampler (crates/nr-model/src/sample.rs:32-96): the same
drawn ids and the same xorshift state after every draw, over 128256-token
vocabularies, small ones with NaN and -inf logits (fewer than 64 candidates),
tied logits inside the candidate set, temperatures from 0.05 to 3, top_p from
1e-6 to 1; and greedy (temperature 0). The logit vectors are checked to have
no tie between the 64th and 65th largest logit, where the reference's heap
and unstable sort leave the candidate order open.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=1000, norm_eps=1e-5,
            rope_theta=500000.0)


def boundary_untied(logits):
    v = np.sort(logits[logits > -np.inf])[::-1]
    return v.size <= 64 or v[63] != v[64]


def logit_cases():
    rng = np.random.default_rng(123)
    out = []
    for i in range(6):
        out.append(rng.normal(0, 2.0, 128256).astype(np.float32))
    x = rng.normal(0, 1, 1000).astype(np.float32)
    x[rng.choice(1000, 30, replace=False)] = 3.25  # 30 exact ties inside the top 64
    out.append(x)
    small = rng.normal(0, 1, 40).astype(np.float32)
    small[[3, 9]] = np.nan
    small[[5, 6, 7]] = -np.inf
    out.append(small)  # 35 valid logits: (-inf, 0) slots fill the rest
    out.append(rng.normal(0, 1, 70).astype(np.float32))
    allnan = np.full(100, np.nan, np.float32)
    out.append(allnan)  # no candidate at all
    return [c for c in out if boundary_untied(c)]


def test_device_sampler_matches_oracle(gpu, oracle):
    import torch

    from nightrun_amd.model import sample

    cases = logit_cases()
    assert len(cases) == 10
    params = [(0.7, 0.9), (1.0, 1.0), (2.5, 0.5), (0.05, 0.9), (3.0, 1e-6), (0.0, 0.9)]
    for ci, logits in enumerate(cases):
        dev = torch.from_numpy(logits).cuda()
        for T, top_p in params:
            seed = 1000 * ci + int(T * 100) + 7
            ref = oracle.Sampler(T, top_p, seed)
            rng = torch.tensor([np.uint64(seed | 1).view(np.int64)], dtype=torch.int64, device="cuda")
            for d in range(12):
                want = ref.sample(logits)
                got = sample(dev, T, top_p, rng)
                state = int(rng.cpu().numpy().view(np.uint64)[0])
                assert got == want, (ci, T, top_p, d, got, want)
                assert state == ref.rng.value, (ci, T, top_p, d)


def test_generate_with_sampler_matches_oracle(gpu, oracle):
    """Prefill, then 24 sampled steps inside the captured decode graph; then
    greedy again after set_sampler(0, ...)."""
    from nightrun_amd.model import Model

    w = oracle.gen_model(TINY, 505)
    prompt = np.random.default_rng(505).integers(0, TINY["vocab"], 20).astype(np.uint32)
    T, top_p, seed = 0.8, 0.9, 0xDEADBEEF12345
    ref = oracle.Model(TINY, w, ctx=96, threads=THREADS)
    ref.prefill(prompt[:-1])
    s = oracle.Sampler(T, top_p, seed)
    tok, want = int(prompt[-1]), []
    for _ in range(24):
        tok = s.sample(ref.forward(tok))
        want.append(tok)
    greedy_want = []
    for _ in range(5):
        tok = oracle.argmax(ref.forward(tok))
        greedy_want.append(tok)

    m = Model(TINY, 96)
    try:
        m.set_weights(w)
        m.prefill(prompt[:-1], logits=False)
        m.set_sampler(T, top_p, seed)
        got = m.generate(int(prompt[-1]), 24)
        assert list(got) == want
        assert m.sampler_state() == s.rng.value
        m.set_sampler(0.0, 1.0, 1)
        assert list(m.generate(int(got[-1]), 5)) == greedy_want
    finally:
        m.close()


def test_device_sampler_ties_at_the_top(gpu, oracle):
    """More than 64 logits tied at the maximum: the reference's heap admits them
    in index order and never evicts one (strict >), so its candidates are the 64
    lowest ids of the tie, as the device's id bisection picks them (in each
    wave's slice, each workgroup's, and the final list)."""
    import torch

    from nightrun_amd.model import sample

    rng = np.random.default_rng(77)
    cases = [np.full(1000, 0.5, np.float32), np.zeros(128256, np.float32)]
    x = rng.normal(0, 1, 128256).astype(np.float32)
    x[rng.choice(128256, 300, replace=False)] = 9.0  # 300 ties above every other logit
    cases.append(x)
    y = rng.normal(0, 1, 151936).astype(np.float32)
    y[rng.choice(151936, 70, replace=False)] = -0.0
    y[y > 0] = -1.0 - y[y > 0]
    y[rng.choice(151936, 20, replace=False)] = 0.0  # 90 ties of -0 and +0 at the top
    cases.append(y)
    for ci, logits in enumerate(cases):
        dev = torch.from_numpy(logits).cuda()
        for T, top_p in [(1.0, 1.0), (0.7, 0.9)]:
            seed = 31 * ci + 5
            ref = oracle.Sampler(T, top_p, seed)
            st = torch.tensor([np.uint64(seed | 1).view(np.int64)], dtype=torch.int64, device="cuda")
            for d in range(8):
                want = ref.sample(logits)
                got = sample(dev, T, top_p, st)
                assert got == want, (ci, T, top_p, d, got, want)
                assert int(st.cpu().numpy().view(np.uint64)[0]) == ref.rng.value


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 2047, 2048, 2049, 4097])
def test_device_sampler_slice_boundaries(gpu, oracle, n):
    """Vocabulary sizes around the selection kernels' units: one logit, fewer
    or more than the 64 candidates, a first-kernel slice of 2048 logits plus
    or minus one (partial workgroups, empty waves, one-list merges)."""
    import torch

    from nightrun_amd.model import sample

    logits = np.random.default_rng(n).normal(0, 1.5, n).astype(np.float32)
    if not boundary_untied(logits):
        pytest.skip("64th and 65th largest tie")
    dev = torch.from_numpy(logits).cuda()
    for T, top_p in [(0.7, 0.9), (1.5, 1.0)]:
        seed = 7 * n + 1
        ref = oracle.Sampler(T, top_p, seed)
        st = torch.tensor([np.uint64(seed | 1).view(np.int64)], dtype=torch.int64, device="cuda")
        for d in range(6):
            want = ref.sample(logits)
            got = sample(dev, T, top_p, st)
            assert got == want, (n, T, top_p, d, got, want)
            assert int(st.cpu().numpy().view(np.uint64)[0]) == ref.rng.value
