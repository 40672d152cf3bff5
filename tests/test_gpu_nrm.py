"""GPU side of .nrm files: the device CRC-32 (nrq_dev_crc32) against the oracle
over every length and alignment class its decomposition has (head bytes before
16-byte alignment, whole 2 KiB stripes, spans of 16 or more stripes, a front-
padded first span, a tail under 16 bytes, running values), and the loader
(nrq_model_load_nrm) against the oracle's InferCtx: a file written from the
oracle's weights, loaded and verified on the device, must decode the same
greedy tokens, logits and f16 KV cache bit for bit as the oracle model (tied
and untied heads, K-quant layers, Llama-3 rope scaling, a RopeFreqs tensor),
and must fail the way InferCtx::new does on a missing or misshapen tensor and
the way verify_data does on a corrupted byte.
"""
import os
import zlib

import numpy as np
import pytest

from oracle import nrm as ON

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
TINY = dict(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=1000, norm_eps=1e-5,
            rope_theta=500000.0)


def dev_bytes(arr):
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr, np.uint8)).cuda()


def test_dev_crc32_reference_vectors(gpu):
    from nightrun_amd import nrm

    for data, want in ((b"123456789", 0xCBF43926), (b"a", 0xE8B7BE43), (b"\0" * 16, zlib.crc32(b"\0" * 16))):
        assert nrm.dev_crc32(dev_bytes(np.frombuffer(data, np.uint8))) == want
    t = dev_bytes(np.zeros(64, np.uint8))
    assert nrm.dev_crc32(t, nbytes=0) == 0
    assert nrm.dev_crc32(t, crc=0x1234ABCD, nbytes=0) == 0x1234ABCD


def test_dev_crc32_lengths_and_alignments(gpu, oracle):
    from nightrun_amd import nrm

    data = np.random.default_rng(21).integers(0, 256, 600_000, dtype=np.uint8)
    t = dev_bytes(data)
    lengths = (1, 2, 15, 16, 17, 31, 32, 33, 1023, 1024, 2047, 2048, 2049, 4096, 32767, 32768, 32769, 65536 + 5,
               100_003, 262_144, 400_000, 599_000)
    for off in (0, 1, 3, 8, 15, 16, 17, 255):
        for n in lengths:
            got = nrm.dev_crc32(t, nbytes=n, offset=off)
            want = oracle.crc32(data[off:off + n])
            assert got == want, (off, n, hex(got), hex(want))
    # running values: the CRC of a prefix continued on the device
    seed = oracle.crc32(data[:12345])
    assert nrm.dev_crc32(t, crc=seed, offset=12345, nbytes=300_000) == oracle.crc32(data[:312_345])


def test_dev_crc32_reference_stream(gpu, oracle):
    """The xorshift64 stream of crates/nr-model/tests/verify.rs:31-39."""
    from nightrun_amd import nrm

    x, m, out = 0x12345678, (1 << 64) - 1, bytearray(100_003)
    for i in range(len(out)):
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        out[i] = x & 0xFF
    arr = np.frombuffer(bytes(out), np.uint8)
    t = dev_bytes(arr)
    for n in (0, 1, 7, 8, 9, 63, 100_003):
        assert nrm.dev_crc32(t, nbytes=n) == oracle.crc32_bitwise(arr[:n]), n


def test_dev_crc32_large_buffer(gpu, oracle):
    """300 MB: 36 stripes per span, 4096 spans, a front-padded first span, four
    spans per thread in the combine; plus a flipped bit changes the value."""
    import torch

    from nightrun_amd import nrm

    n = 300_000_011
    data = np.random.default_rng(22).integers(0, 256, n, dtype=np.uint8)
    t = dev_bytes(data)
    want = oracle.crc32(data)
    assert nrm.dev_crc32(t) == want
    assert nrm.dev_crc32(t, offset=5, nbytes=n - 5) == oracle.crc32(data[5:])
    t[123_456_789] ^= 4
    torch.cuda.synchronize()
    assert nrm.dev_crc32(t) != want


# ---- loader ----------------------------------------------------------------------------

def kquant_layers(oracle, cfg, w, seed):
    shapes = oracle.layer_shapes(cfg)
    for l, lw in enumerate(w["layers"]):
        for i, name in enumerate(oracle.LAYER_MATS):
            dt = 3 if name == "w_down" else 2
            rows, cols = shapes[name]
            lw[name] = oracle.gen_weights(dt, seed + 16 * l + i, rows, cols)
            lw["dtypes"][name] = dt
    return w


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def decode_pair(oracle, cfg, w, blob, ctx, prompt, n_gen, freqs=None):
    """Loads `blob` on the device; feeds the prompt and generates greedily on
    both sides; tokens, last logits and the KV cache must be identical."""
    from nightrun_amd import nrm

    ref = oracle.Model(cfg, w, ctx=ctx, threads=THREADS)
    if freqs is not None:
        ref.set_freqs(freqs)
    want = ref.prefill(prompt)
    tok = oracle.argmax(want)
    want_tokens = [tok]
    for _ in range(n_gen):
        want = ref.forward(tok)
        tok = oracle.argmax(want)
        want_tokens.append(tok)

    m = nrm.NrmFile(blob).load(ctx, verify=True)
    try:
        for i, t in enumerate(prompt):
            lg = m.forward(int(t), logits=(i == len(prompt) - 1))
        first = int(np.argmax(lg))
        got, last = m.generate(first, n_gen, logits=True)
        assert [first] + list(got) == want_tokens, "greedy tokens differ"
        assert np.array_equal(bits(last), bits(want)), "last logits differ"
        k, v = m.kv_cache()
        rk, rv = ref.kv_cache()
        assert np.array_equal(k, rk) and np.array_equal(v, rv), "KV cache differs"
    finally:
        m.close()


def test_load_tied_q8_model(gpu, oracle):
    w = oracle.gen_model(TINY, 31)
    blob = ON.write(ON.default_meta(**TINY, flags=ON.FLAG_TIED_EMBEDDINGS), ON.model_tensors(TINY, w, tied=True))
    prompt = np.random.default_rng(31).integers(0, TINY["vocab"], 13).astype(np.uint32)
    decode_pair(oracle, TINY, w, bytes(blob), 64, prompt, 10)


def test_load_untied_kquant_model_with_rope_scaling(gpu, oracle):
    """Q4_K/Q6_K layers, a separate Q6_K head, Llama-3.2 rope scaling."""
    w = kquant_layers(oracle, TINY, oracle.gen_model(TINY, 32), 900)
    w["output"] = oracle.gen_weights(3, 555, TINY["vocab"], TINY["dim"])
    w["output_dtype"] = 3
    scal = dict(rope_factor=32.0, rope_low=1.0, rope_high=4.0, rope_orig_ctx=8192.0)
    blob = ON.write(ON.default_meta(**TINY, **scal), ON.model_tensors(TINY, w, tied=False))
    freqs = oracle.infer_freqs(TINY["head_dim"], TINY["rope_theta"], 32.0, 1.0, 4.0, 8192.0)
    assert not np.array_equal(freqs, oracle.rope_freqs(TINY["head_dim"], TINY["rope_theta"]))
    prompt = np.random.default_rng(32).integers(0, TINY["vocab"], 70).astype(np.uint32)
    decode_pair(oracle, TINY, w, bytes(blob), 96, prompt, 8, freqs=freqs)


def test_load_rope_freqs_tensor(gpu, oracle):
    """A RopeFreqs tensor divides the base spectrum and overrides header scaling."""
    w = oracle.gen_model(TINY, 33)
    fac = np.linspace(1.0, 32.0, TINY["head_dim"] // 2).astype(np.float32)
    meta = ON.default_meta(**TINY, flags=ON.FLAG_TIED_EMBEDDINGS, rope_factor=8.0, rope_low=1.0, rope_high=4.0,
                           rope_orig_ctx=8192.0)
    blob = ON.write(meta, ON.model_tensors(TINY, w, tied=True, rope_factors=fac))
    freqs = oracle.infer_freqs(TINY["head_dim"], TINY["rope_theta"], factors=fac)
    prompt = np.random.default_rng(33).integers(0, TINY["vocab"], 21).astype(np.uint32)
    decode_pair(oracle, TINY, w, bytes(blob), 64, prompt, 6, freqs=freqs)


def test_load_qwen3_model_with_mup_scales(gpu, oracle):
    """Qwen3 (per-head q/k RMSNorm tensors, Neox rope) with non-neutral muP
    scalars in the header: the loader sets the recipe InferCtx::new derives
    (infer.rs:383-461)."""
    mup = dict(embed_scale=1.6, attn_scale=0.3, residual_scale=0.6, logit_scale=2.5)
    cfg = dict(TINY, rope_theta=10000.0, recipe=dict(rope="neox", **mup))
    w = oracle.gen_model(cfg, 36, qk_norm=True)
    meta = ON.default_meta(**TINY, **mup, flags=ON.FLAG_TIED_EMBEDDINGS, arch=ON.ARCH_QWEN3)
    meta["rope_theta"] = 10000.0
    blob = ON.write(meta, ON.model_tensors(cfg, w, tied=True))
    prompt = np.random.default_rng(36).integers(0, TINY["vocab"], 17).astype(np.uint32)
    decode_pair(oracle, cfg, w, bytes(blob), 64, prompt, 8)


def test_load_granite_model_with_mup_scales(gpu, oracle):
    """Granite: adjacent rope, no qk-norm, muP scalars (attn_scale 0 = 1/sqrt(head_dim))."""
    mup = dict(embed_scale=12.0, attn_scale=0.0, residual_scale=0.22, logit_scale=8.0)
    cfg = dict(TINY, recipe=dict(rope="adjacent", **mup))
    w = oracle.gen_model(cfg, 37)
    meta = ON.default_meta(**TINY, **mup, flags=ON.FLAG_TIED_EMBEDDINGS, arch=ON.ARCH_GRANITE)
    blob = ON.write(meta, ON.model_tensors(cfg, w, tied=True))
    prompt = np.random.default_rng(37).integers(0, TINY["vocab"], 11).astype(np.uint32)
    decode_pair(oracle, cfg, w, bytes(blob), 64, prompt, 8)


def test_load_rejects_corrupt_data(gpu, oracle):
    from nightrun_amd import nrm

    w = oracle.gen_model(TINY, 34)
    blob = ON.write(ON.default_meta(**TINY, flags=ON.FLAG_TIED_EMBEDDINGS), ON.model_tensors(TINY, w, tied=True))
    meta, _ = ON.parse(bytes(blob))
    assert nrm.NrmFile(bytes(blob)).verify_data()
    bad = bytearray(blob)
    bad[meta["data_off"] + 12345] ^= 0x01  # verify.rs:78-80
    f = nrm.NrmFile(bytes(bad))  # the meta CRC does not cover the data
    assert not f.verify_data()
    with pytest.raises(nrm.ParseError) as e:
        f.load(64, verify=True)
    assert e.value.variant == "DataCrc"
    f.load(64, verify=False).close()


def test_load_reports_missing_and_misshapen_tensors(gpu, oracle):
    from nightrun_amd import NrqError, nrm

    w = oracle.gen_model(TINY, 35)
    meta = ON.default_meta(**TINY, flags=ON.FLAG_TIED_EMBEDDINGS)
    full = ON.model_tensors(TINY, w, tied=True)
    no_k1 = [t for t in full if not (t[0] == ON.ATTN_K and t[1] == 1)]
    with pytest.raises(nrm.ParseError, match="attn_k") as e:
        nrm.NrmFile(bytes(ON.write(meta, no_k1))).load(64)
    assert e.value.variant == "MissingTensor"
    untied = ON.default_meta(**TINY)
    with pytest.raises(nrm.ParseError, match="output"):
        nrm.NrmFile(bytes(ON.write(untied, full))).load(64)
    wrong = [(k, l, dt, r, c, p) if not (k == ON.ATTN_K and l == 0) else (k, l, dt, c, r, p)
             for (k, l, dt, r, c, p) in full]  # 128x256 stored as 256x128: same bytes, wrong shape
    with pytest.raises(nrm.ParseError, match="bad matrix shape"):
        nrm.NrmFile(bytes(ON.write(meta, wrong))).load(64)
    qn = full + [(ON.ATTN_Q_NORM, 0, ON.F32, 1, TINY["head_dim"], bytes(4 * TINY["head_dim"]))]
    with pytest.raises(nrm.ParseError, match="unexpected attn_q_norm"):
        nrm.NrmFile(bytes(ON.write(meta, qn))).load(64)
    with pytest.raises(nrm.ParseError, match="attn_q_norm") as e:  # Qwen3 needs its qk-norm tensors
        nrm.NrmFile(bytes(ON.write({**meta, "arch": ON.ARCH_QWEN3}, full))).load(64)
    assert e.value.variant == "MissingTensor"
