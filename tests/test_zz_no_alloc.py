"""nrq_dev_sample_noalloc (the sampler with its partial lists in a fixed
per-device array) against nrq_dev_sample (stream-ordered scratch), both
through the C ABI: the same drawn id and the same xorshift state after every
draw, on two calls in a row with the second on fewer logits, at several
temperatures and cut-offs; greedy; and the size limit, rejected before any
launch. Also checked against the oracle's Sampler (sample.rs:32-96).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _untied_at_64(x):
    v = np.sort(x[x > -np.inf])[::-1]
    return v.size <= 64 or v[63] != v[64]


def _draw(L, fn, logits, n, temperature, top_p, rng, tok, stream):
    rc = getattr(L, fn)(logits.data_ptr(), n, temperature, top_p, rng.data_ptr(), tok.data_ptr(), stream)
    assert rc == 0, (fn, rc, L.nrq_last_error())


def test_sample_noalloc_matches_sample(gpu, oracle):
    import torch

    from nightrun_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(77)
    # two calls in a row: a 151936-token vocabulary, then a smaller one
    for n, T, top_p in ((151936, 0.7, 0.9), (4097, 1.3, 0.5), (151936, 0.05, 1.0), (70, 2.0, 0.95)):
        x = rng.normal(0, 2.0, n).astype(np.float32)
        assert _untied_at_64(x)
        d = torch.from_numpy(x).cuda()
        seed = int(rng.integers(1, 2 ** 62)) | 1
        ra = torch.tensor([seed], dtype=torch.int64, device="cuda")
        rb = ra.clone()
        ta = torch.zeros(1, dtype=torch.int32, device="cuda")
        tb = torch.zeros(1, dtype=torch.int32, device="cuda")
        ref = oracle.Sampler(T, top_p, seed)
        for k in range(6):
            _draw(L, "nrq_dev_sample", d, n, T, top_p, ra, ta, stream)
            _draw(L, "nrq_dev_sample_noalloc", d, n, T, top_p, rb, tb, stream)
            torch.cuda.synchronize()
            want = ref.sample(x)
            assert int(ta.item()) == int(tb.item()) == want, (n, k)
            assert int(ra.item()) == int(rb.item()), (n, k)
            assert int(rb.item()) & (2 ** 64 - 1) == ref.rng.value, (n, k)


def test_sample_noalloc_greedy_and_limits(gpu):
    import torch

    from nightrun_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    x = np.random.default_rng(5).normal(0, 1, 1000).astype(np.float32)
    d = torch.from_numpy(x).cuda()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    r = torch.tensor([3], dtype=torch.int64, device="cuda")
    _draw(L, "nrq_dev_sample_noalloc", d, 1000, 0.0, 0.9, r, tok, stream)
    torch.cuda.synchronize()
    assert int(tok.item()) == int(np.argmax(x)) and int(r.item()) == 3
    # beyond the fixed scratch: a clear error, nothing launched (n is checked
    # before any pointer is read)
    rc = L.nrq_dev_sample_noalloc(d.data_ptr(), (1 << 19) + 1, 0.7, 0.9, r.data_ptr(), tok.data_ptr(), stream)
    assert rc == _lib.NRQ_ERR_UNSUPPORTED
    assert "524288" in L.nrq_last_error().decode()
    assert L.nrq_dev_sample_noalloc(d.data_ptr(), 0, 0.7, 0.9, r.data_ptr(), tok.data_ptr(), stream) != 0
    assert L.nrq_dev_sample_noalloc(None, 10, 0.7, 0.9, r.data_ptr(), tok.data_ptr(), stream) != 0
    # the largest accepted size still runs
    big = torch.from_numpy(np.random.default_rng(6).normal(0, 1, 1 << 19).astype(np.float32)).cuda()
    ra = torch.tensor([11], dtype=torch.int64, device="cuda")
    rb = ra.clone()
    ta = torch.zeros(1, dtype=torch.int32, device="cuda")
    tb = torch.zeros(1, dtype=torch.int32, device="cuda")
    _draw(L, "nrq_dev_sample", big, 1 << 19, 0.8, 0.9, ra, ta, stream)
    _draw(L, "nrq_dev_sample_noalloc", big, 1 << 19, 0.8, 0.9, rb, tb, stream)
    torch.cuda.synchronize()
    assert int(ta.item()) == int(tb.item()) and int(ra.item()) == int(rb.item())
