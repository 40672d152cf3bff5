"""Benchmark of NightRun's quantized matrix path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config cfg2] [--order scalar|avx2]
                    [--no-decode] [--no-prefill] [--no-cpu-baseline]

Headline (`value`): the decode matvec of the Q4_K 8192 x 3072 matrix
(Llama-3.2-3B FFN shape) against a runtime-quantized Q8_K activation. A step
is one matvec launch over weights already resident in HBM; the K timed steps
run back to back as one captured HIP graph. Weights come from distinct copies
(as many as the K steps, up to 2 x the 256 MiB MALL), and a 1 GiB read runs
before every replay, so no timed read can hit the MALL. `value` is
algorithmic bytes x K / the graph's wall time (HIP events on the launch
stream); `roofline.achieved` is algorithmic bytes / the mean time per launch
inside that graph.

Beside it, in the same JSON line:
  other_configs  the Q8_0 8192x2048 and Q6_K 128256x3072 matvecs, same method
  prefill        one Qwen3-4B layer's seven matmuls at M = 64 tokens (int8 MFMA)
  decode         greedy tokens/s of a Llama-3.2-1B-shape Q8_0 model (random
                 init) with the KV cache filled to 1024 positions, each step one
                 HIP graph replay (nrq_model_generate); the model is loaded from
                 an in-memory .nrm file (load time beside it) and its data
                 section's CRC-32 is timed on the device (verify_crc); the
                 1024-token prompt goes through the batched prefill
                 (prefill tok/s beside it)
  cpu_baseline   the CPU oracle's AVX2 and scalar restatements of the matvec,
                 each on 1 thread and on the box's host-core share (median of
                 >= 21 full matvecs), and its scalar-order restatement of the
                 full decode step at the GPU leg's KV positions
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q-matvec HBM GB/s (% of peak); decode tok/s, Llama-3.2-1B-shape Q8_0"
HBM_PEAK_GBS = 8000.0     # MI355X HBM3E, vendor peak
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, vendor peak
MALL_BYTES = 256 << 20
# HBM bytes per launch of the headline kernel: rocprofv3 FETCH_SIZE and WRITE_SIZE passes over this
# script, each scaled by the same counter's reading for a 256 MiB device copy
# (profiles/wstream_matvec_q4k_8192x3072.md). Workloads not counted report None.
MEASURED_TRAFFIC = {("cfg2", "scalar"): 14306076}

# name -> (dtype, rows, cols, seed, description)
CONFIGS = {
    "cfg1": (1, 8192, 2048, 0x5EED0001, "Q8_0 matvec 8192x2048 (Llama-3.2-1B ffn_gate), Q8_0 activation"),
    "cfg2": (2, 8192, 3072, 0x5EED0002, "Q4_K matvec 8192x3072 (Llama-3.2-3B FFN), Q8_K activation"),
    "cfg3": (3, 128256, 3072, 0x5EED0003, "Q6_K matvec 128256x3072 (tied output head), Q8_K activation"),
}
WBYTES = {1: 34, 2: 144, 3: 210}
XBYTES = {1: 34, 2: 292, 3: 292}
QK = {1: 32, 2: 256, 3: 256}
# Qwen3-4B layer: hidden 2560, attention 4096, ffn 9728, KV width 1024 (8 heads x 128)
QWEN3_4B_LAYER = [("wq", 2, 4096, 2560), ("wk", 2, 1024, 2560), ("wv", 2, 1024, 2560), ("wo", 2, 2560, 4096),
                  ("w_gate", 2, 9728, 2560), ("w_up", 2, 9728, 2560), ("w_down", 3, 2560, 9728)]
LLAMA_1B = dict(dim=2048, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64, ffn_dim=8192, vocab=128256,
                norm_eps=1e-5, rope_theta=500000.0)
# Qwen3-4B (36 layers, hidden 2560, 32 query / 8 KV heads of 128, ffn 9728, tied
# 151936 head), with the formats of a Q4_K_M file: Q4_K q/k/o/gate/up, Q6_K v,
# down and embedding
QWEN3_4B = dict(dim=2560, n_layers=36, n_heads=32, n_kv_heads=8, head_dim=128, ffn_dim=9728, vocab=151936,
                norm_eps=1e-6, rope_theta=1000000.0)
QWEN3_DTYPES = {"wq": 2, "wk": 2, "wv": 3, "wo": 2, "w_gate": 2, "w_up": 2, "w_down": 3}


def synth_weights(dtype, rows, cols, seed):
    """Random blocks as the benchmark configs specify (numpy generator):
    Q8_0: d = f16(|N(0,0.02)|/127), qs uniform in [-127,127];
    Q4_K: d, dmin = f16(|N(0,0.01)|), random scales/qs bytes;
    Q6_K: random ql/qh/scales bytes, d = f16(|N(0,0.01)|)."""
    rng = np.random.default_rng(seed)
    nb = rows * (cols // QK[dtype])
    if dtype == 1:
        w = np.empty((nb, 34), dtype=np.uint8)
        d = (np.abs(rng.normal(0, 0.02, nb)) / 127).astype(np.float16)
        w[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        w[:, 2:] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    elif dtype == 2:
        w = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
        d = np.abs(rng.normal(0, 0.01, (nb, 2))).astype(np.float16)
        w[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    else:
        w = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
        d = np.abs(rng.normal(0, 0.01, nb)).astype(np.float16)
        w[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return w


def algorithmic_bytes(dtype, rows, cols, batch=1):
    """Weights + quantized activations + f32 outputs, each touched once."""
    bpr = cols // QK[dtype]
    return rows * bpr * WBYTES[dtype] + batch * bpr * XBYTES[dtype] + batch * rows * 4


class MallFlush:
    """A read of 1 GiB (four times the 256 MiB MALL), run untimed before a
    measured region so that none of the weights it reads can still be cached
    there. It only reads (a sum), so it leaves no dirty lines whose write-back
    the measured kernels would pay for."""

    BYTES = 1 << 30

    def __init__(self):
        import torch

        self.buf = torch.ones(self.BYTES // 4, dtype=torch.float32, device="cuda")

    def __call__(self, stream):
        import torch

        with torch.cuda.stream(stream):
            self.out = self.buf.sum()


def graph_time(stream, launch, k, flush=None):
    """Captures k launches (launch(i)) into one HIP graph, replays it once
    untimed, then times one replay with HIP events on `stream`; `flush(stream)`
    runs before each replay, outside the timed region. Returns (seconds per
    replay, seconds per launch)."""
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        g.capture_begin()
        for i in range(k):
            launch(i)
        g.capture_end()
    if flush:
        flush(stream)
    with torch.cuda.stream(stream):  # replay() launches on the current stream
        g.replay()
    if flush:
        flush(stream)
    stream.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        g.replay()
        b.record(stream)
    b.synchronize()
    s = a.elapsed_time(b) / 1e3
    del g
    return s, s / k


def measure_read(nbytes, steps):
    """The plain streaming-read rate at `nbytes` per launch (nrq_dev_stream_read),
    timed like the matvecs: K launches in one graph over rotating copies after a
    MALL flush. The ceiling a bandwidth-bound matvec of that size can reach."""
    import torch

    import nightrun_amd
    from nightrun_amd import _lib

    nightrun_amd.init(0)
    n16 = -(-nbytes // 16)
    copies = max(2, min(steps, -(-(2 * MALL_BYTES) // (16 * n16))))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        bufs = [torch.ones(n16 * 4, dtype=torch.int32, device="cuda") for _ in range(copies)]
        out = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream.synchronize()
    flush = MallFlush()

    def step(i):
        _lib.check(_lib.lib().nrq_dev_stream_read(bufs[i % copies].data_ptr(), 16 * n16, out.data_ptr(),
                                                  stream.cuda_stream))

    for i in range(3):
        step(i)
    wall, per = graph_time(stream, step, steps, flush)
    del bufs
    torch.cuda.empty_cache()
    return {"bytes": 16 * n16, "us": round(per * 1e6, 3), "gbs": round(16 * n16 / per / 1e9, 1),
            "frac_of_peak": round(16 * n16 / per / 1e9 / HBM_PEAK_GBS, 4), "copies": copies}


def measure_matvec(name, steps, warmup, order):
    import torch

    import nightrun_amd
    from nightrun_amd import device

    dtype, rows, cols, seed, _ = CONFIGS[name]
    nightrun_amd.init(0)
    w = synth_weights(dtype, rows, cols, seed)
    xf = np.random.default_rng(seed + 1).normal(0, 1, cols).astype(np.float32)
    # distinct copies for the K steps, up to 2 x MALL of them: within a replay a
    # copy is read again only after 2 x MALL of other weights
    copies = max(2, min(steps, -(-(2 * MALL_BYTES) // w.nbytes)))
    flush = MallFlush()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        w0 = torch.from_numpy(w).cuda()
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        xd = torch.from_numpy(xf).cuda()
        bpr = cols // QK[dtype]
        xq = torch.empty(bpr * XBYTES[dtype], dtype=torch.uint8, device="cuda")
        (device.quantize_q8_0 if dtype == 1 else device.quantize_q8k)(xd, xq, stream=stream)
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
    stream.synchronize()

    def step(i):
        device.matvec(dtype, order, y, ws[i % copies], xq, rows, cols, stream=stream)

    flush(stream)
    for i in range(warmup):
        step(i)
    stream.synchronize()
    wall, per = graph_time(stream, step, steps, flush)
    nbytes = algorithmic_bytes(dtype, rows, cols)
    # the activation quantizer, reported beside
    q0, q1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    q0.record(stream)
    for _ in range(20):
        (device.quantize_q8_0 if dtype == 1 else device.quantize_q8k)(xd, xq, stream=stream)
    q1.record(stream)
    stream.synchronize()
    out = {"bytes": nbytes, "copies": copies, "rotated_weight_bytes": copies * int(w.nbytes),
           "timed_distinct_weight_bytes": min(steps, copies) * int(w.nbytes), "wall_s": wall,
           "ms_per_step": wall / steps * 1e3,
           "value_gbs": nbytes * steps / wall / 1e9, "kernel_us": per * 1e6, "kernel_gbs": nbytes / per / 1e9,
           "quant_us": q0.elapsed_time(q1) / 20 * 1e3}
    del ws, w0, flush
    torch.cuda.empty_cache()
    return out


def measure_prefill(reps=3, order=0):
    """One Qwen3-4B layer's seven matmuls at M = 64 (Q8_K activations) in its
    four groups (q|k|v and gate|up share an activation and one launch), as one
    graph of `reps` layers over rotating weight copies. order 1: the AVX2 f32
    order (the x86 host's 4-token tiles), one launch per matrix."""
    import torch

    import nightrun_amd
    from nightrun_amd import device

    nightrun_amd.init(0)
    stream = torch.cuda.Stream()
    mats, tot_bytes, tot_ops = [], 0, 0.0
    copies = 4  # the layers of one replay read distinct weight copies
    with torch.cuda.stream(stream):
        for j, (name, dt, rows, cols) in enumerate(QWEN3_4B_LAYER):
            w = torch.from_numpy(synth_weights(dt, rows, cols, 0x5EED0004 + j)).cuda()
            ws = [w] + [w.clone() for _ in range(copies - 1)]
            if j in (1, 2, 5):  # k, v, up take the activation of q and gate
                xq = mats[-1][4]
            else:
                xf = torch.from_numpy(np.random.default_rng(40 + j).normal(0, 1, 64 * cols).astype(np.float32)).cuda()
                xq = torch.empty(64 * cols // 256 * 292, dtype=torch.uint8, device="cuda")
                device.quantize_q8k(xf, xq, stream=stream)
            y = torch.empty(64 * rows, dtype=torch.float32, device="cuda")
            mats.append((dt, rows, cols, ws, xq, y))
            tot_bytes += algorithmic_bytes(dt, rows, cols, 64) - (64 * (cols // 256) * 292 if j in (1, 2, 5) else 0)
            tot_ops += 2.0 * 64 * rows * cols
    stream.synchronize()

    # the layer's matmul groups (q|k|v, gate|up share their input, as Acts::matmul_group runs them)
    groups = [[0, 1, 2], [3], [4, 5], [6]]

    def layer(i):
        for g in groups:
            dt, cols, xq = mats[g[0]][0], mats[g[0]][2], mats[g[0]][4]
            if order == 0:
                device.matmul_group(dt, [mats[j][5] for j in g], [mats[j][3][i % copies] for j in g],
                                    [mats[j][1] for j in g], xq, cols, 64, stream=stream)
            else:
                for j in g:
                    device.matmul(dt, order, mats[j][5], mats[j][3][i % copies], xq, mats[j][1], cols, 64,
                                  stream=stream)

    flush = MallFlush()
    flush(stream)
    layer(0)
    stream.synchronize()
    wall, per = graph_time(stream, layer, reps, flush)
    del mats, flush
    torch.cuda.empty_cache()
    return {"workload": "Qwen3-4B layer at M=64: Q/K/V/O/gate/up Q4_K, down Q6_K (hidden 2560, attention 4096, "
                        "KV 1024, ffn 9728), per-row Q8_K activations",
            "order": "scalar" if order == 0 else "avx2",
            "us_per_layer": round(per * 1e6, 2), "tok_s_36_layers": round(64 / (36 * per), 1),
            "gbs": round(tot_bytes / per / 1e9, 1), "int8_tops": round(tot_ops / per / 1e12, 2),
            "mfma_frac_of_int8_peak": round(tot_ops / per / 1e12 / INT8_PEAK_TOPS, 4),
            "algorithmic_bytes_per_layer": tot_bytes}


def synth_model(cfg, seed, dtypes=None, embed_dtype=1, qk_norm=False):
    """Llama-family random-init weights with the numpy generator: all Q8_0
    unless `dtypes` names a format per matrix, norms 1.0 (Qwen3's per-head q/k
    norms too, with qk_norm), head tied to the embedding."""
    d, hd = cfg["dim"], cfg["head_dim"]
    att, kv, ffn = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["ffn_dim"]
    shapes = {"wq": (att, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, att), "w_gate": (ffn, d), "w_up": (ffn, d),
              "w_down": (d, ffn)}
    w = {"embed": synth_weights(embed_dtype, cfg["vocab"], d, seed), "embed_dtype": embed_dtype,
         "out_norm": np.ones(d, np.float32), "layers": []}
    for l in range(cfg["n_layers"]):
        lw = {"attn_norm": np.ones(d, np.float32), "ffn_norm": np.ones(d, np.float32), "dtypes": {}}
        for i, (name, (rows, cols)) in enumerate(shapes.items()):
            dt = dtypes[name] if dtypes else 1
            lw[name] = synth_weights(dt, rows, cols, seed + 1 + 16 * l + i)
            lw["dtypes"][name] = dt
        if qk_norm:
            lw["q_norm"] = np.ones(hd, np.float32)
            lw["k_norm"] = np.ones(hd, np.float32)
        w["layers"].append(lw)
    return w


def model_bytes_per_token(cfg, kv_pos):
    d, hd = cfg["dim"], cfg["head_dim"]
    att, kv, ffn = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["ffn_dim"]
    per_layer = (att * d + 2 * kv * d + d * att + 3 * ffn * d) // 32 * 34
    head = cfg["vocab"] * d // 32 * 34
    kv_bytes = cfg["n_layers"] * kv_pos * kv * 2 * 2
    return cfg["n_layers"] * per_layer + head + kv_bytes


def nrm_blob(cfg, w, arch=1, name=b"llama-1b"):
    """The weights `w` as a .nrm v3 file in memory (crates/nr-model/src/format.rs:1-10:
    192-byte header | tokenizer blob | 32-byte table entries | data, every tensor
    64-byte aligned, meta and data CRCs), head tied to the embedding."""
    import struct

    from nightrun_amd import nrm

    d, hd = cfg["dim"], cfg["head_dim"]
    att, kv, ffn = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["ffn_dim"]
    shapes = {"wq": (11, att, d), "wk": (12, kv, d), "wv": (13, kv, d), "wo": (14, d, att), "w_gate": (16, ffn, d),
              "w_up": (17, ffn, d), "w_down": (18, d, ffn)}
    ts = [(1, 0, w["embed_dtype"], cfg["vocab"], d, w["embed"]), (2, 0, 0, 1, d, w["out_norm"])]
    for l, lw in enumerate(w["layers"]):
        ts += [(10, l, 0, 1, d, lw["attn_norm"]), (15, l, 0, 1, d, lw["ffn_norm"])]
        if "q_norm" in lw:  # Qwen3 (TensorKind AttnQNorm / AttnKNorm)
            ts += [(19, l, 0, 1, hd, lw["q_norm"]), (20, l, 0, 1, hd, lw["k_norm"])]
        ts += [(k, l, lw["dtypes"][n], r, c, lw[n]) for n, (k, r, c) in shapes.items()]
    tok = b"\0" * 64
    table_off = 192 + len(tok)
    data_off = -(-(table_off + 32 * len(ts)) // 64) * 64
    offs, pos = [], 0
    for t in ts:
        offs.append(pos)
        pos = -(-(pos + t[5].nbytes) // 64) * 64
    data_size = offs[-1] + ts[-1][5].nbytes
    b = np.zeros(data_off + data_size, np.uint8)
    hdr = bytearray(192)
    hdr[0:4] = b"NRUN"
    struct.pack_into("<II8I", hdr, 4, 3, arch, d, cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"], hd, ffn,
                     cfg["vocab"], 131072)
    struct.pack_into("<6fI4f", hdr, 44, cfg["rope_theta"], cfg["norm_eps"], 0.0, 0.0, 0.0, 0.0, 1, 1.0, 0.0, 1.0, 1.0)
    hdr[88:88 + len(name)] = name
    struct.pack_into("<QQQIIQQ", hdr, 136, 192, len(tok), table_off, len(ts), 0, data_off, data_size)
    table = bytearray(32 * len(ts))
    for i, (t, off) in enumerate(zip(ts, offs)):
        struct.pack_into("<HHHHQQII", table, 32 * i, t[0], t[1], t[2], 0, off, t[5].nbytes, t[3], t[4])
        b[data_off + off:data_off + off + t[5].nbytes] = np.ascontiguousarray(t[5]).view(np.uint8).ravel()
    struct.pack_into("<I", hdr, 184, nrm.crc32(b[data_off:]))
    b[table_off:table_off + len(table)] = np.frombuffer(bytes(table), np.uint8)
    b[192:192 + len(tok)] = np.frombuffer(tok, np.uint8)
    c = nrm.crc32(bytes(hdr[:184]) + bytes(8))
    c = nrm.crc32(tok, c)
    struct.pack_into("<I", hdr, 188, nrm.crc32(bytes(table), c))
    b[:192] = np.frombuffer(bytes(hdr), np.uint8)
    return b


def measure_crc(data, want=None, reps=20):
    """nrq_dev_crc32 over the uint8 device tensor `data`, `reps` calls back to
    back on one stream, HIP events around them."""
    import torch

    from nightrun_amd import _lib

    n = data.numel()
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    L = _lib.lib()
    torch.cuda.synchronize()
    _lib.check(L.nrq_dev_crc32(data.data_ptr(), n, 0, out.data_ptr(), stream.cuda_stream))
    stream.synchronize()
    got = int(out.cpu().item()) & 0xFFFFFFFF
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        _lib.check(L.nrq_dev_crc32(data.data_ptr(), n, 0, out.data_ptr(), stream.cuda_stream))
    b.record(stream)
    b.synchronize()
    per = a.elapsed_time(b) / 1e3 / reps
    r = {"bytes": n, "us": round(per * 1e6, 2), "gbs": round(n / per / 1e9, 1),
         "frac_of_hbm_peak": round(n / per / 1e9 / HBM_PEAK_GBS, 4)}
    if want is not None:
        r["matches_header"] = got == want
    return r


def measure_decode(fill=1024, n=128):
    """The model comes in through the .nrm path (parse, one upload of the data
    section, CRC on the device, binding), then greedy decode."""
    import torch

    import nightrun_amd
    from nightrun_amd import nrm

    nightrun_amd.init(0)
    cfg = LLAMA_1B
    w = synth_model(cfg, 0x5EED0005)
    blob = nrm_blob(cfg, w)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    f = nrm.NrmFile(blob)
    m = f.load(fill + n + 8, verify=True)
    load_s = time.perf_counter() - t0
    data = f.upload()
    crc = {"workload": "CRC-32 (IEEE) of the Llama-3.2-1B-shape Q8_0 data section in HBM",
           **measure_crc(data, f.meta["data_crc"])}
    del data
    # the prompt: `fill` random tokens through the batched prefill (512-token
    # chunks), once untimed for warm-up, then timed from position 0
    prompt = np.random.default_rng(5).integers(0, cfg["vocab"], fill).astype(np.uint32)
    m.prefill(prompt[:64], logits=False)
    m.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lg = m.prefill(prompt)
    pf_dt = time.perf_counter() - t0
    t0 = time.perf_counter()
    out = m.generate(int(np.argmax(lg)), n)
    dt = time.perf_counter() - t0
    # the same steps drawing from the top 64 at temperature 0.7, top-p 0.9 (the
    # reference's chat defaults, crates/nr-boot/src/app.rs:290): the sampler
    # kernel in place of argmax inside the step graph
    m.reset()
    m.prefill(prompt, logits=False)
    m.set_sampler(0.7, 0.9, 0x5EED0006)
    m.generate(int(np.argmax(lg)), 8)  # captures the sampling step
    m.reset()
    m.prefill(prompt, logits=False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.generate(int(np.argmax(lg)), n)
    sdt = time.perf_counter() - t0
    # untimed: the first steps again one forward at a time, for the margin
    # between the two largest logits (how far a numeric difference would have
    # to move a logit to change the greedy token) and the token check
    m.reset()
    m.set_sampler(0.0, 1.0, 0)
    m.prefill(prompt, logits=False)
    gaps, same, tok = [], True, int(np.argmax(lg))
    for i in range(min(n, 16)):
        step_lg = m.forward(tok)
        top2 = np.sort(step_lg)[-2:]
        gaps.append(float(top2[1] - top2[0]))
        tok = int(np.argmax(step_lg))
        same = same and tok == int(out[i])
    stages = step_stages(m, tok)
    m.close()
    torch.cuda.empty_cache()
    mid = fill + n // 2
    load = {"file_bytes": int(blob.size), "data_bytes": int(f.meta["data_size"]), "seconds": round(load_s, 4),
            "gbs_pcie_inclusive": round(blob.size / load_s / 1e9, 2),
            "what": "nrq_nrm_open + nrq_model_load_nrm(verify): parse and meta CRC on the host, one hipMemcpy of "
                    "the data section from pageable memory, data CRC on the device, tensor binding"}
    return {"workload": "Llama-3.2-1B architecture, all Q8_0, random init (16 layers, hidden 2048, 32/8 heads x 64, "
                        f"ffn 8192, tied 128256 head), f16 KV cache at positions {fill}..{fill + n - 1}, greedy",
            "tok_s": round(n / dt, 1), "ms_per_token": round(dt / n * 1e3, 4),
            "bytes_per_token": model_bytes_per_token(cfg, mid),
            "gbs": round(model_bytes_per_token(cfg, mid) * n / dt / 1e9, 1), "tokens": int(n),
            "first_tokens": [int(t) for t in out[:4]], "load": load, "verify_crc": crc,
            "sampled_tok_s": round(n / sdt, 1),
            "step_stages_us": {"what": f"eager steps at KV {fill + min(n, 16)}.., HIP events after each stage, "
                                       "medians of 8 (the graph replay above runs the same kernels)", **stages},
            "stage_gbs": stage_gbs(cfg, stages, fill + min(n, 16)),
            "top2_logit_gap": {"steps": len(gaps), "min": round(min(gaps), 6), "median": round(float(np.median(gaps)), 6),
                               "per_step": [round(g, 6) for g in gaps], "forward_tokens_match_generate": bool(same)},
            "prefill": {"tokens": int(fill), "chunks_of": 64, "seconds": round(pf_dt, 4),
                        "tok_s": round(fill / pf_dt, 1),
                        "what": "nrq_model_prefill of the random prompt from position 0 (KV 0..1023), host sync "
                                "per chunk, logits of the last token copied back"},
            # for the host-side comparison, removed before the line is printed
            "_weights": w, "_prompt": prompt,
            "_tokens": [int(np.argmax(lg))] + [int(t) for t in out]}


def step_stages(m, token, steps=8):
    """Median microseconds per stage of `steps` eagerly launched decode steps,
    each stage bracketed by HIP events on the model's stream."""
    rows = [m.step_profile(token) for _ in range(steps)]
    out = {k: round(float(np.median([r[k] for r in rows])), 2) for k in rows[0]}
    out["sum"] = round(sum(v for k, v in out.items()), 2)
    return out


def kquant_bytes(dt, rows, cols):
    return rows * cols // 256 * (144 if dt == 2 else 210) if dt in (2, 3) else rows * cols // 32 * 34


def stage_gbs(cfg, stages, kv_pos, dtypes=None, head_dtype=1):
    """GB/s of each decode stage: the bytes it reads per token (weights of all
    layers; attention: the K and V rows of kv_pos positions, f16) over its
    eager microseconds (events between stages included, so a lower bound)."""
    d, hd, L = cfg["dim"], cfg["head_dim"], cfg["n_layers"]
    att, kv, ffn = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["ffn_dim"]
    dt = dtypes or {k: 1 for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")}
    b = {"norm_qkv": L * (kquant_bytes(dt["wq"], att, d) + kquant_bytes(dt["wk"], kv, d) + kquant_bytes(dt["wv"], kv, d)),
         "attention": L * kv_pos * kv * 2 * 2,
         "o": L * kquant_bytes(dt["wo"], d, att),
         "norm_gate_up_swiglu": L * (kquant_bytes(dt["w_gate"], ffn, d) + kquant_bytes(dt["w_up"], ffn, d)),
         "down": L * kquant_bytes(dt["w_down"], d, ffn),
         "head": kquant_bytes(head_dtype, cfg["vocab"], d)}
    out = {k: round(v / (stages[k] * 1e-6) / 1e9, 1) for k, v in b.items() if stages.get(k)}
    out["weights_and_kv"] = round(sum(b.values()) / (stages["sum"] * 1e-6) / 1e9, 1)
    return out


def measure_qwen3(fill=512, n=64):
    """Qwen3-4B shape with Q4_K_M formats through a Qwen3 .nrm file (the loader
    sets the recipe: per-head q/k RMSNorm, Neox rope): a `fill`-token prefill,
    then n greedy steps. The reference publishes 10.6-11.9 tok/s decode and
    20.7 tok/s batch-64 prefill for Qwen3-4B Q4_K_M on its 8-thread x86 host."""
    import torch

    from nightrun_amd import nrm

    cfg = QWEN3_4B
    w = synth_model(cfg, 0x5EED0044, dtypes=QWEN3_DTYPES, embed_dtype=3, qk_norm=True)
    blob = nrm_blob(cfg, w, arch=2, name=b"qwen3-4b")
    del w
    t0 = time.perf_counter()
    f = nrm.NrmFile(blob)
    m = f.load(fill + n + 8, verify=False)
    load_s = time.perf_counter() - t0
    del blob
    prompt = np.random.default_rng(44).integers(0, cfg["vocab"], fill).astype(np.uint32)
    m.prefill(prompt[:64], logits=False)  # warm-up
    m.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lg = m.prefill(prompt)
    pf_dt = time.perf_counter() - t0
    m.generate(int(np.argmax(lg)), 4)  # captures the step graph
    m.reset()
    m.prefill(prompt, logits=False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = m.generate(int(np.argmax(lg)), n)
    dt = time.perf_counter() - t0
    stages = step_stages(m, int(out[-1]))
    m.close()
    torch.cuda.empty_cache()
    d, hd = cfg["dim"], cfg["head_dim"]
    att, kv, ffn = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["ffn_dim"]
    shapes = {"wq": (att, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, att), "w_gate": (ffn, d), "w_up": (ffn, d),
              "w_down": (d, ffn)}
    per_tok = cfg["n_layers"] * sum(kquant_bytes(QWEN3_DTYPES[k], r, c) for k, (r, c) in shapes.items())
    per_tok += kquant_bytes(3, cfg["vocab"], d) + cfg["n_layers"] * (fill + n // 2) * kv * 2 * 2
    return {"workload": "Qwen3-4B architecture, Q4_K_M formats (Q4_K q/k/o/gate/up, Q6_K v/down/embedding, tied "
                        "151936 head), random init, Qwen3 recipe (qk-norm, Neox rope) from the .nrm header; "
                        f"prefill of {fill} tokens, then greedy at positions {fill}..{fill + n - 1}",
            "tok_s": round(n / dt, 1), "ms_per_token": round(dt / n * 1e3, 4), "bytes_per_token": int(per_tok),
            "gbs": round(per_tok * n / dt / 1e9, 1), "prefill_tok_s": round(fill / pf_dt, 1),
            "load_seconds": round(load_s, 3),
            "step_stages_us": {"what": f"eager steps at KV {fill + n}.., HIP events after each stage, medians of 8",
                               **stages},
            "stage_gbs": stage_gbs(cfg, stages, fill + n, dtypes=QWEN3_DTYPES, head_dtype=3),
            "reference_host": {"decode_tok_s": "10.6-11.9", "prefill_batch64_tok_s": 20.7,
                               "source": "docs/benchmarks.md:63-64, docs/baseline-x86.md:144"}}


def measure_qwen3_prefill(tokens):
    """The Qwen3 leg's model (Q4_K_M formats through a Qwen3 .nrm file), then
    nrq_model_prefill of a random `tokens`-token prompt in 512-token chunks
    (eager launches, no graph): the prefill alone, for kernel traces."""
    import torch

    from nightrun_amd import nrm

    cfg = QWEN3_4B
    w = synth_model(cfg, 0x5EED0044, dtypes=QWEN3_DTYPES, embed_dtype=3, qk_norm=True)
    blob = nrm_blob(cfg, w, arch=2, name=b"qwen3-4b")
    del w
    f = nrm.NrmFile(blob)
    m = f.load(tokens + 8, verify=False)
    del blob
    prompt = np.random.default_rng(44).integers(0, cfg["vocab"], tokens).astype(np.uint32)
    m.prefill(prompt[:64], logits=False)  # warm-up
    m.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    m.prefill(prompt, logits=False)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    m.close()
    return {"workload": f"Qwen3-4B architecture, Q4_K_M formats, random init: prefill of {tokens} tokens in "
                        "512-token chunks, eager launches", "tokens": tokens, "seconds": round(dt, 4),
            "tok_s": round(tokens / dt, 1)}


def measure_qwen3_eager(steps, fill=512):
    """The Qwen3-4B leg's model and prompt, then `steps` greedy decode steps
    launched eagerly (nrq_model_forward, no graph): a kernel trace of the
    K-quant step without the captured-graph path."""
    import torch

    from nightrun_amd import nrm

    cfg = QWEN3_4B
    w = synth_model(cfg, 0x5EED0044, dtypes=QWEN3_DTYPES, embed_dtype=3, qk_norm=True)
    blob = nrm_blob(cfg, w, arch=2, name=b"qwen3-4b")
    del w
    f = nrm.NrmFile(blob)
    m = f.load(fill + steps + 8, verify=False)
    del blob
    prompt = np.random.default_rng(44).integers(0, cfg["vocab"], fill).astype(np.uint32)
    lg = m.prefill(prompt)
    tok = int(np.argmax(lg))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = int(np.argmax(m.forward(tok)))
    dt = time.perf_counter() - t0
    m.close()
    return {"workload": "Qwen3-4B architecture, Q4_K_M formats, eager greedy steps (nrq_model_forward, logits "
                        f"copied back each step) at positions {fill}..{fill + steps - 1}",
            "steps": steps, "ms_per_step": round(dt / steps * 1e3, 4)}


def host_cores():
    """Threads for the CPU baselines: every CPU this process may run on, up to
    the 16-core host share a one-GPU box gives a job (the pool is not sized past
    what the job owns, whatever the machine reports)."""
    return min(16, len(os.sched_getaffinity(0)))


def cpu_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "machine_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "pool_threads": host_cores()}


def _median_rate(fn, nbytes, reps, seconds):
    """Median GB/s of fn() over at least `reps` calls (more while under `seconds`)."""
    fn()  # warm-up (pool threads, page faults)
    ts = []
    t_end = time.perf_counter() + seconds
    while len(ts) < reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    med = ts[len(ts) // 2]
    return nbytes / med / 1e9, len(ts), med


def cpu_baseline_matvec(name, seconds):
    """The oracle's AVX2 and scalar restatements (the reference's x86 fast path
    and its scalar kernels, kernels.rs / kquant.rs) on full matvecs of the same
    workload, each on 1 thread and on the host-core share with a
    parallel.rs-style row pool (chunk rule parallel.rs:97, calling thread
    included), weights rotated over copies beyond the LLC; median of >= 21
    calls. `value` is the AVX2 order on all pool threads (the reference's own
    timed host path)."""
    import oracle as O

    dtype, rows, cols, seed, _ = CONFIGS[name]
    threads = host_cores()
    w = O.gen_weights(dtype, seed, rows, cols)
    copies = max(1, min(8, -(-(256 << 20) // w.nbytes)))
    ws = [w] + [w.copy() for _ in range(copies - 1)]
    x = O.quantize_act(dtype, O.Rng(seed ^ 0xABCDEF).normal(cols))
    nbytes = algorithmic_bytes(dtype, rows, cols)
    runs = {}
    per = max(1.0, seconds / 4)
    for order, oname in ((O.ORDER_AVX2, "avx2"), (O.ORDER_SCALAR, "scalar")):
        for nt in (1, threads):
            k = [0]

            def call():
                O.matvec(dtype, order, ws[k[0] % copies], x, rows, cols, nt)
                k[0] += 1

            gbs, n, med = _median_rate(call, nbytes, 21, per)
            runs[f"{oname}_{nt}t"] = {"gbs": round(gbs, 3), "median_ms": round(med * 1e3, 3), "calls": n,
                                      "threads": nt}
    top = runs[f"avx2_{threads}t"]
    return {"value": top["gbs"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"median of {top['calls']} full {name} matvecs (AVX2 order, {threads} threads, {copies} "
                      f"rotating weight copies); every order x thread count in `runs`",
            "runs": runs, **cpu_info()}


def cpu_baseline_decode(seconds, fill=1024, device=None):
    """The reference's decode on this host's cores, restated by the oracle:
    the x86 path nrhost runs (AVX2 matvec dots, F16C attention dot and axpy,
    the parallel.rs pool on every core: tools/nrhost/src/main.rs:41-51,
    108-153) and the scalar-order path, greedy at the GPU leg's KV positions.
    For the rates the model is moved to position `fill` without computing the
    cache rows before it (their cost does not depend on their values).
    With the GPU leg's weights, prompt and tokens (`device`), the x86 path also
    prefills the same prompt and decodes greedily, and its tokens are compared
    with the device's, which follow the scalar order."""
    import oracle as O

    threads = host_cores()
    cfg = dict(O.LLAMA_1B)
    w = device["_weights"] if device else O.gen_model(cfg, 0x5EED0005)

    def rate(order, secs):
        m = O.Model(cfg, w, ctx=fill + 136, threads=threads, order=order)
        m.seek(fill)
        tok = O.argmax(m.forward(1))  # warm-up step at position fill
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < secs and n < 128:
            tok = O.argmax(m.forward(tok))
            n += 1
        return n, time.perf_counter() - t0

    n1, dt1 = rate(O.ORDER_AVX2, seconds)
    n0, dt0 = rate(O.ORDER_SCALAR, seconds / 2)
    out = {"value": round(n1 / dt1, 3), "unit": "tok/s", "cores": threads, "kind": "port",
           "sample": f"{n1} greedy decode steps at KV positions {fill + 1}..{fill + n1} of the Llama-3.2-1B-shape Q8_0 "
                     f"model in {dt1:.1f} s, x86 path (AVX2 dots, F16C attention) on {threads} threads; cache rows "
                     f"before {fill} not computed (same cost per step)",
           "scalar_order": {"value": round(n0 / dt0, 3), "unit": "tok/s", "cores": threads,
                            "sample": f"{n0} steps the same way with the scalar-order kernels"}}
    if device:
        dev = device["_tokens"]
        m = O.Model(cfg, w, ctx=fill + 136, threads=threads, order=O.ORDER_AVX2)
        t0 = time.perf_counter()
        lg = m.prefill(device["_prompt"])
        pf = time.perf_counter() - t0
        toks, gaps = [], []
        t0 = time.perf_counter()
        while len(toks) < len(dev) and (len(toks) < 8 or time.perf_counter() - t0 < seconds):
            top2 = np.sort(lg)[-2:]
            gaps.append(float(top2[1] - top2[0]))
            toks.append(O.argmax(lg))
            # after a divergence the x86 run keeps its own tokens
            lg = m.forward(toks[-1])
        same = [a == b for a, b in zip(toks, dev)]
        first_diff = same.index(False) if not all(same) else None
        out["x86_vs_device_tokens"] = {
            "compared": len(toks), "identical": int(sum(same)), "first_difference": first_diff,
            "top2_gap_min": round(min(gaps), 6), "top2_gap_median": round(float(np.median(gaps)), 6),
            "top2_gap_at_first_difference": None if first_diff is None else round(gaps[first_diff], 6),
            "prefill_tok_s": round(fill / pf, 3),
            "what": f"the same {fill}-token prompt through the x86 path's prefill (4-token AVX2 tiles), then greedy "
                    "decode; compared position by position with the device's scalar-order tokens (the first is "
                    "the prompt's argmax); the top-2 logit gap of each x86 step"}
    return out


def cpu_baseline_crc(seconds):
    """The oracle's slicing-by-8 CRC-32 (crc32.rs) on one host core over 64 MiB
    chunks for about `seconds`."""
    import oracle as O

    chunk = np.random.default_rng(9).integers(0, 256, 64 << 20, dtype=np.uint8)
    n, c = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        c = O.crc32(chunk, c)
        n += chunk.size
    dt = time.perf_counter() - t0
    return {"value": round(n / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n >> 20} MiB of random bytes in 64 MiB calls, {dt:.1f} s"}


def progress(msg):
    """One line per finished leg on stderr (the JSON line stays alone on stdout)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def copy_calibration(nbytes):
    """Five device-to-device copies of `nbytes` (reads nbytes, writes nbytes):
    the reference kernel for scaling FETCH_SIZE / WRITE_SIZE counter readings."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "copies": 5}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2", choices=list(CONFIGS))
    ap.add_argument("--order", default="scalar", choices=["scalar", "avx2"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--decode-tokens", type=int, default=128, help="greedy tokens timed by the decode leg")
    ap.add_argument("--also", default="cfg1,cfg3", help="other matvec configs reported beside (comma list)")
    ap.add_argument("--qwen3-only", action="store_true", help="only the Qwen3-4B decode/prefill leg")
    ap.add_argument("--no-qwen3", action="store_true", help="skip the Qwen3-4B decode/prefill leg")
    ap.add_argument("--qwen3-eager", type=int, default=0, metavar="STEPS",
                    help="only: the Qwen3-4B model, then STEPS eagerly launched greedy steps (no graph)")
    ap.add_argument("--qwen3-prefill", type=int, default=0, metavar="TOKENS",
                    help="only: the Qwen3-4B model, then nrq_model_prefill of TOKENS tokens (eager, no graph)")
    ap.add_argument("--prefill-only", type=int, default=0, metavar="TOKENS",
                    help="only time nrq_model_prefill of TOKENS tokens on the Llama-3.2-1B-shape model")
    ap.add_argument("--crc-only", type=int, default=0, metavar="BYTES",
                    help="only time nrq_dev_crc32 over BYTES random device bytes (profiling the CRC kernels)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (a known-size kernel for HBM counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration << 20)
        return
    if args.qwen3_eager:
        import nightrun_amd

        nightrun_amd.init(0)
        print(json.dumps({"decode_qwen3_eager": measure_qwen3_eager(args.qwen3_eager)}))
        return
    if args.qwen3_prefill:
        import nightrun_amd

        nightrun_amd.init(0)
        print(json.dumps({"prefill_qwen3": measure_qwen3_prefill(args.qwen3_prefill)}))
        return
    if args.qwen3_only:
        import nightrun_amd

        nightrun_amd.init(0)
        print(json.dumps({"decode_qwen3": measure_qwen3()}))
        return
    if args.prefill_only:
        import torch

        import nightrun_amd
        from nightrun_amd.model import Model

        nightrun_amd.init(0)
        cfg = LLAMA_1B
        m = Model(cfg, ctx=args.prefill_only + 8)
        m.set_weights(synth_model(cfg, 0x5EED0005))
        prompt = np.random.default_rng(5).integers(0, cfg["vocab"], args.prefill_only).astype(np.uint32)
        m.prefill(prompt[:64], logits=False)
        m.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m.prefill(prompt)
        dt = time.perf_counter() - t0
        m.close()
        print(json.dumps({"prefill_only": {"tokens": args.prefill_only, "seconds": round(dt, 4),
                                           "tok_s": round(args.prefill_only / dt, 1)}}))
        return
    if args.crc_only:
        import torch

        import nightrun_amd

        nightrun_amd.init(0)
        data = torch.randint(0, 256, (args.crc_only,), dtype=torch.uint8, device="cuda")
        print(json.dumps({"crc_only": measure_crc(data, reps=args.steps)}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding of the path is design-only"}))
        sys.exit(2)
    order = 0 if args.order == "scalar" else 1
    r = measure_matvec(args.config, args.steps, args.warmup, order)
    progress(f"{args.config} matvec {r['kernel_us']:.3f} us")
    others = {}
    for name in [s for s in args.also.split(",") if s and s != args.config]:
        o = measure_matvec(name, args.steps, args.warmup, order)
        others[name] = {k: round(v, 3) if isinstance(v, float) else v for k, v in o.items()}
        progress(f"{name} matvec {o['kernel_us']:.3f} us")
    ceil = {name: measure_read(algorithmic_bytes(CONFIGS[name][0], CONFIGS[name][1], CONFIGS[name][2]), args.steps)
            for name in [args.config] + [s for s in args.also.split(",") if s and s != args.config]}
    progress("read ceiling")
    prefill = None if args.no_prefill else measure_prefill()
    if prefill is not None:
        progress("prefill layer")
        prefill["avx2_order"] = measure_prefill(order=1)
        progress("prefill layer, AVX2 order")
    decode = None if args.no_decode else measure_decode(n=args.decode_tokens)
    if decode is not None:
        progress(f"decode {decode['tok_s']} tok/s")
    qwen3 = None
    if not args.no_decode and not args.no_qwen3:
        try:
            qwen3 = measure_qwen3()
        except Exception as e:  # reported, never fatal to the bench line
            qwen3 = {"error": f"{type(e).__name__}: {e}"}
        progress("qwen3")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_matvec(args.config, args.cpu_seconds)
        progress("cpu matvec")
        if decode is not None:
            cpu["decode"] = cpu_baseline_decode(args.cpu_seconds, device=decode)
            cpu["verify_crc"] = cpu_baseline_crc(min(args.cpu_seconds, 5.0))
            progress("cpu decode")
    if decode is not None:
        for k in ("_weights", "_prompt", "_tokens"):
            decode.pop(k, None)
    dtype, rows, cols, _, desc = CONFIGS[args.config]
    out = {
        "metric": METRIC,
        "value": round(r["value_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random weights, N(0,1) activation)",
        "config": {
            "workload": desc,
            "order": args.order,
            "rotating_weight_copies": r["copies"],
            "algorithmic_bytes_per_step": r["bytes"],
            "activation_quantize_us": round(r["quant_us"], 3),
            "timing": "K launches captured in one HIP graph, HIP events on the launch stream",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(r["kernel_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": MEASURED_TRAFFIC.get((args.config, args.order)),
            "kernel_us": round(r["kernel_us"], 3),
            "read_ceiling": {**ceil[args.config], "kernel_frac_of_read": round(r["kernel_gbs"] / ceil[args.config]["gbs"], 4),
                             "what": "a plain streaming read of the same bytes per launch, timed the same way"},
        },
        "cpu_baseline": cpu,
        "other_configs": {k: {**v, "read_ceiling": ceil.get(k)} for k, v in others.items()},
        "prefill": prefill,
        "decode": decode,
        "decode_qwen3": qwen3,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
