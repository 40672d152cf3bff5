"""CPU oracle for the quantized matrix path -- TEST INFRASTRUCTURE ONLY.

ctypes view of ``liboracle.so`` (built from ``nrq_oracle.c`` by the Makefile
beside this file). Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this module, and only as the
checker; the product library (``nightrun_amd``) never imports it.

Each wrapped function restates a function of the reference's Rust crate
``crates/nr-tensor`` (citations in ``nrq_oracle.h``). Blocks travel as numpy
``uint8`` arrays of shape ``(nblocks, block_bytes)``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0, Q4K, Q6K = 1, 2, 3
ORDER_SCALAR, ORDER_AVX2 = 0, 1
QK = {Q8_0: 32, Q4K: 256, Q6K: 256}
WBYTES = {Q8_0: 34, Q4K: 144, Q6K: 210}
XBYTES = {Q8_0: 34, Q4K: 292, Q6K: 292}
Q8K_BYTES = 292

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, sz, f32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_float)
        L.nro_f16_to_f32.argtypes, L.nro_f16_to_f32.restype = [C.c_uint16], C.c_float
        L.nro_f32_to_f16.argtypes, L.nro_f32_to_f16.restype = [C.c_float], C.c_uint16
        for name in ("nro_quantize_q8_0", "nro_quantize_q8k"):
            getattr(L, name).argtypes = [vp, sz, vp]
        L.nro_dequantize_q8_0.argtypes = [vp, sz, vp]
        L.nro_q4k_scale_min.argtypes = [vp, C.c_int, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        for name in ("nro_dequant_q4k", "nro_dequant_q6k", "nro_quantize_q4k_ref", "nro_quantize_q6k_ref"):
            getattr(L, name).argtypes = [vp, vp]
        for q in ("q8", "q4k", "q6k"):
            for kind in ("scalar", "avx2"):
                fn = getattr(L, f"nro_dot_{q}_{kind}")
                fn.argtypes, fn.restype = [vp, vp, sz], C.c_float
            getattr(L, f"nro_dot_{q}_avx2_x4").argtypes = [vp, C.POINTER(vp), sz, f32p]
        L.nro_matvec.argtypes = [C.c_int, C.c_int, vp, vp, vp, sz, sz, C.c_int]
        L.nro_matmul.argtypes = [C.c_int, C.c_int, vp, vp, vp, sz, sz, sz, C.c_int]
        L.nro_block_sums.argtypes, L.nro_block_sums.restype = [C.c_int, vp, vp, sz, vp], sz
        L.nro_rng_vec.argtypes = [C.POINTER(C.c_uint64), vp, sz]
        L.nro_rng_adversarial.argtypes = [C.POINTER(C.c_uint64), vp, sz]
        L.nro_rng_normal.argtypes = [C.POINTER(C.c_uint64), vp, sz, C.c_float]
        L.nro_rng_bytes.argtypes = [C.POINTER(C.c_uint64), vp, sz]
        L.nro_gen_weights.argtypes = [C.c_int, C.c_uint64, vp, sz]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---- f16.rs -----------------------------------------------------------------

def f16_to_f32(bits: int) -> float:
    return lib().nro_f16_to_f32(bits)


def f32_to_f16(v: float) -> int:
    return lib().nro_f32_to_f16(v)


def f16_to_f32_array(bits: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.nro_f16_to_f32(int(b)) for b in bits.ravel()], dtype=np.float32).reshape(bits.shape)


# ---- quantizers ---------------------------------------------------------------

def quantize_q8_0(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32).ravel()
    out = np.zeros((src.size // 32, 34), dtype=np.uint8)
    lib().nro_quantize_q8_0(_p(src), src.size, _p(out))
    return out


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.zeros(blocks.shape[0] * 32, dtype=np.float32)
    lib().nro_dequantize_q8_0(_p(blocks), blocks.shape[0], _p(out))
    return out


def quantize_q8k(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32).ravel()
    out = np.zeros((src.size // 256, Q8K_BYTES), dtype=np.uint8)
    lib().nro_quantize_q8k(_p(src), src.size, _p(out))
    return out


def quantize_act(dtype: int, src: np.ndarray) -> np.ndarray:
    """The activation format each weight dtype consumes (Q8_0 or Q8_K)."""
    return quantize_q8_0(src) if dtype == Q8_0 else quantize_q8k(src)


def q8k_fields(blocks: np.ndarray):
    """(d f32[n], qs i8[n,256], bsums i16[n,16]) views of Q8_K blocks."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    d = b[:, 0:4].copy().view(np.float32).ravel()
    qs = b[:, 4:260].view(np.int8)
    bsums = b[:, 260:292].copy().view(np.int16)
    return d, qs, bsums


def q4k_scale_min(scales12: np.ndarray, j: int):
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc, m = C.c_uint8(), C.c_uint8()
    lib().nro_q4k_scale_min(_p(s), j, C.byref(sc), C.byref(m))
    return sc.value, m.value


def dequant_q4k(block: np.ndarray) -> np.ndarray:
    block = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(256, dtype=np.float32)
    lib().nro_dequant_q4k(_p(block), _p(out))
    return out


def dequant_q6k(block: np.ndarray) -> np.ndarray:
    block = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.zeros(256, dtype=np.float32)
    lib().nro_dequant_q6k(_p(block), _p(out))
    return out


def quantize_q4k_ref(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32).ravel()
    n = src.size // 256
    out = np.zeros((n, 144), dtype=np.uint8)
    for i in range(n):
        lib().nro_quantize_q4k_ref(_p(src[i * 256:(i + 1) * 256]), _p(out[i]))
    return out


def quantize_q6k_ref(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32).ravel()
    n = src.size // 256
    out = np.zeros((n, 210), dtype=np.uint8)
    for i in range(n):
        lib().nro_quantize_q6k_ref(_p(src[i * 256:(i + 1) * 256]), _p(out[i]))
    return out


def quantize_weights_ref(dtype: int, src: np.ndarray) -> np.ndarray:
    if dtype == Q8_0:
        return quantize_q8_0(src)
    return quantize_q4k_ref(src) if dtype == Q4K else quantize_q6k_ref(src)


# ---- dots ---------------------------------------------------------------------

_DOT = {Q8_0: "q8", Q4K: "q4k", Q6K: "q6k"}


def dot(dtype: int, order: int, w: np.ndarray, x: np.ndarray) -> float:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.uint8)
    kind = "avx2" if order == ORDER_AVX2 else "scalar"
    fn = getattr(lib(), f"nro_dot_{_DOT[dtype]}_{kind}")
    return fn(_p(w), _p(x), min(w.shape[0], x.shape[0]))


def dot_x4(dtype: int, w: np.ndarray, xs) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xs = [np.ascontiguousarray(x, dtype=np.uint8) for x in xs]
    arr = (C.c_void_p * 4)(*[x.ctypes.data for x in xs])
    out = np.zeros(4, dtype=np.float32)
    getattr(lib(), f"nro_dot_{_DOT[dtype]}_avx2_x4")(_p(w), arr, w.shape[0], out.ctypes.data_as(C.POINTER(C.c_float)))
    return out


def matvec(dtype: int, order: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.uint8)
    y = np.zeros(rows, dtype=np.float32)
    lib().nro_matvec(dtype, order, _p(y), _p(w), _p(x), rows, cols, threads)
    return y


def matmul(dtype: int, order: int, w: np.ndarray, xs: np.ndarray, rows: int, cols: int, batch: int,
           threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.uint8)
    y = np.zeros(batch * rows, dtype=np.float32)
    lib().nro_matmul(dtype, order, _p(y), _p(w), _p(xs), rows, cols, batch, threads)
    return y


def block_sums(dtype: int, w_row: np.ndarray, x: np.ndarray) -> np.ndarray:
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.uint8)
    nb = min(w_row.shape[0], x.shape[0])
    per = {Q8_0: 1, Q4K: 9, Q6K: 16}[dtype]
    out = np.zeros(nb * per, dtype=np.int32)
    lib().nro_block_sums(dtype, _p(w_row), _p(x), nb, _p(out))
    return out


# ---- generators ----------------------------------------------------------------

class Rng:
    """xorshift64 13/7/17 (tests/kernels.rs:9-29, tests/kquant.rs:7-39)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def vec(self, n: int) -> np.ndarray:
        out = np.zeros(n, dtype=np.float32)
        lib().nro_rng_vec(C.byref(self.state), _p(out), n)
        return out

    def adversarial(self, n: int) -> np.ndarray:
        out = np.zeros(n, dtype=np.float32)
        lib().nro_rng_adversarial(C.byref(self.state), _p(out), n)
        return out

    def normal(self, n: int, sigma: float = 1.0) -> np.ndarray:
        out = np.zeros(n, dtype=np.float32)
        lib().nro_rng_normal(C.byref(self.state), _p(out), n, sigma)
        return out

    def bytes(self, n: int) -> np.ndarray:
        out = np.zeros(n, dtype=np.uint8)
        lib().nro_rng_bytes(C.byref(self.state), _p(out), n)
        return out


def gen_weights(dtype: int, seed: int, rows: int, cols: int) -> np.ndarray:
    nb = rows * (cols // QK[dtype])
    out = np.zeros((nb, WBYTES[dtype]), dtype=np.uint8)
    lib().nro_gen_weights(dtype, seed, _p(out), nb)
    return out


# ---- forward pass (nrq_model_oracle.c) -------------------------------------------

_model_sigs_done = False


def _model_lib():
    global _model_sigs_done
    L = lib()
    if not _model_sigs_done:
        vp, sz, f32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_float)
        L.nro_expf.argtypes, L.nro_expf.restype = [C.c_float], C.c_float
        L.nro_sincosf.argtypes = [C.c_float, f32p, f32p]
        L.nro_expf_n.argtypes = [vp, vp, sz]
        L.nro_sincosf_n.argtypes = [vp, vp, vp, sz]
        L.nro_rmsnorm.argtypes = [vp, vp, vp, sz, C.c_float]
        L.nro_softmax.argtypes = [vp, sz]
        L.nro_swiglu.argtypes = [vp, vp, sz]
        L.nro_argmax.argtypes, L.nro_argmax.restype = [vp, sz], C.c_uint32
        L.nro_rope_freqs.argtypes = [vp, sz, C.c_float]
        L.nro_rope_apply.argtypes = [vp, sz, sz, vp, sz]
        L.nro_rope_apply_style.argtypes = [vp, sz, sz, vp, sz, C.c_int]
        L.nro_rmsnorm_inplace.argtypes = [vp, vp, sz, C.c_float]
        L.nro_model_set_recipe.argtypes = [vp, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float]
        L.nro_model_set_qk_norm.argtypes = [vp, C.c_int, vp, vp]
        L.nro_model_new.argtypes, L.nro_model_new.restype = [C.POINTER(C.c_int), C.c_float, C.c_float, C.c_int], vp
        L.nro_model_free.argtypes = [vp]
        L.nro_model_set_globals.argtypes = [vp, vp, C.c_int, vp, C.c_int, vp]
        L.nro_model_set_layer.argtypes = [vp, C.c_int, C.POINTER(vp), C.POINTER(C.c_int), vp, vp]
        L.nro_model_forward.argtypes, L.nro_model_forward.restype = [vp, C.c_uint32], f32p
        L.nro_model_prefill_chunk.argtypes, L.nro_model_prefill_chunk.restype = [vp, C.POINTER(C.c_uint32), C.c_int], f32p
        L.nro_model_pos.argtypes, L.nro_model_pos.restype = [vp], C.c_int
        L.nro_model_reset.argtypes = [vp]
        L.nro_model_set_order.argtypes = [vp, C.c_int]
        L.nro_dot_f16.argtypes, L.nro_dot_f16.restype = [C.c_int, vp, vp, sz], C.c_float
        L.nro_axpy_f16.argtypes = [C.c_int, vp, C.c_float, vp, sz]
        L.nro_model_seek.argtypes = [vp, C.c_int]
        L.nro_model_kcache.argtypes, L.nro_model_kcache.restype = [vp], C.POINTER(C.c_uint16)
        L.nro_model_vcache.argtypes, L.nro_model_vcache.restype = [vp], C.POINTER(C.c_uint16)
        L.nro_model_set_freqs.argtypes = [vp, vp]
        L.nro_sampler_next_f32.argtypes, L.nro_sampler_next_f32.restype = [C.POINTER(C.c_uint64)], C.c_float
        L.nro_sample.argtypes = [C.c_float, C.c_float, C.POINTER(C.c_uint64), vp, sz]
        L.nro_sample.restype = C.c_uint32
        for name in ("nro_crc32", "nro_crc32_bitwise"):
            getattr(L, name).argtypes, getattr(L, name).restype = [C.c_uint32, vp, sz], C.c_uint32
        L.nro_infer_freqs.argtypes = [vp, sz, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float, vp]
        _model_sigs_done = True
    return L


def expf(x: float) -> float:
    return _model_lib().nro_expf(x)


def expf_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.empty_like(x)
    _model_lib().nro_expf_n(_p(x), _p(y), x.size)
    return y


def sincosf_array(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32).ravel()
    s, c = np.empty_like(x), np.empty_like(x)
    _model_lib().nro_sincosf_n(_p(x), _p(s), _p(c), x.size)
    return s, c


def sincosf(x: float):
    s, c = C.c_float(), C.c_float()
    _model_lib().nro_sincosf(x, C.byref(s), C.byref(c))
    return s.value, c.value


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    _model_lib().nro_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def rmsnorm_inplace(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """vec.rs:17-28: x * (scale * w), scale = 1/sqrtf(mean(x^2) + eps)."""
    x = np.array(x, dtype=np.float32)
    w = np.ascontiguousarray(w, np.float32)
    _model_lib().nro_rmsnorm_inplace(_p(x), _p(w), x.size, eps)
    return x


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    _model_lib().nro_softmax(_p(x), x.size)
    return x


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.array(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, np.float32)
    _model_lib().nro_swiglu(_p(g), _p(u), g.size)
    return g


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return _model_lib().nro_argmax(_p(x), x.size)


def rope_freqs(head_dim: int, theta: float) -> np.ndarray:
    out = np.zeros(head_dim // 2, np.float32)
    _model_lib().nro_rope_freqs(_p(out), head_dim, theta)
    return out


def infer_freqs(head_dim: int, theta: float, factor: float = 0.0, low: float = 0.0, high: float = 0.0,
                orig_ctx: float = 0.0, factors=None) -> np.ndarray:
    """InferCtx::new's rope table (infer.rs:433-447 over rope.rs:14-34)."""
    out = np.zeros(head_dim // 2, np.float32)
    f = None if factors is None else np.ascontiguousarray(factors, np.float32)
    _model_lib().nro_infer_freqs(_p(out), head_dim, theta, factor, low, high, orig_ctx,
                                 None if f is None else _p(f))
    return out


class Sampler:
    """sample.rs:5-96 restated: Sampler::new(temperature, top_p, seed) keeps seed | 1."""

    def __init__(self, temperature: float, top_p: float, seed: int):
        self.temperature, self.top_p = temperature, top_p
        self.rng = C.c_uint64((seed | 1) & 0xFFFFFFFFFFFFFFFF)

    def next_f32(self) -> float:
        return _model_lib().nro_sampler_next_f32(C.byref(self.rng))

    def sample(self, logits: np.ndarray) -> int:
        x = np.ascontiguousarray(logits, np.float32)
        return _model_lib().nro_sample(self.temperature, self.top_p, C.byref(self.rng), _p(x), x.size)


def crc32(data, crc: int = 0) -> int:
    """CRC-32 of crates/nr-model/src/crc32.rs (slicing by 8), zlib running-value convention."""
    b = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data)
    return _model_lib().nro_crc32(crc, b.ctypes.data if b.size else None, b.nbytes)


def crc32_bitwise(data, crc: int = 0) -> int:
    """The classic bit-at-a-time CRC-32 (crates/nr-model/tests/verify.rs:16-30)."""
    b = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data)
    return _model_lib().nro_crc32_bitwise(crc, b.ctypes.data if b.size else None, b.nbytes)


def rope_apply(x: np.ndarray, head_dim: int, freqs: np.ndarray, pos: int, neox: bool = False) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    f = np.ascontiguousarray(freqs, np.float32)
    _model_lib().nro_rope_apply_style(_p(x), x.size, head_dim, _p(f), pos, int(neox))
    return x


# Llama-3.2-1B architecture (the full-model benchmark shape)
LLAMA_1B = dict(dim=2048, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64, ffn_dim=8192, vocab=128256,
                norm_eps=1e-5, rope_theta=500000.0)
# tensor order of a layer's matrices
LAYER_MATS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


def layer_shapes(cfg: dict):
    d, hd = cfg["dim"], cfg["head_dim"]
    att, kv, ffn = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["ffn_dim"]
    return {"wq": (att, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, att), "w_gate": (ffn, d), "w_up": (ffn, d),
            "w_down": (d, ffn)}


def gen_model(cfg: dict, seed: int, dtype: int = Q8_0, qk_norm: bool = False) -> dict:
    """Random-init weights of the given architecture: every matrix with the
    synthetic generator of its dtype (distinct seed per tensor), RMSNorm
    weights 1.0, output head tied to the embedding. With qk_norm, each layer
    also gets Qwen3's per-head q/k RMSNorm weights, drawn from [0.5, 1.5) so
    that a norm left out changes the result."""
    w = {"embed": gen_weights(dtype, seed, cfg["vocab"], cfg["dim"]), "embed_dtype": dtype,
         "out_norm": np.ones(cfg["dim"], np.float32), "layers": []}
    shapes = layer_shapes(cfg)
    for l in range(cfg["n_layers"]):
        lw = {"attn_norm": np.ones(cfg["dim"], np.float32), "ffn_norm": np.ones(cfg["dim"], np.float32),
              "dtypes": {}}
        for i, name in enumerate(LAYER_MATS):
            rows, cols = shapes[name]
            lw[name] = gen_weights(dtype, seed + 1 + 16 * l + i, rows, cols)
            lw["dtypes"][name] = dtype
        if qk_norm:
            r = np.random.default_rng(seed + 9000 + l)
            lw["q_norm"] = r.uniform(0.5, 1.5, cfg["head_dim"]).astype(np.float32)
            lw["k_norm"] = r.uniform(0.5, 1.5, cfg["head_dim"]).astype(np.float32)
        w["layers"].append(lw)
    return w


def dot_f16(order: int, k_bits: np.ndarray, q: np.ndarray) -> float:
    """kernels::dot_f16 (kernels.rs:146-160): scalar, or dot_f16_f16c (:174-201) with ORDER_AVX2."""
    k = np.ascontiguousarray(k_bits, dtype=np.uint16)
    q = np.ascontiguousarray(q, dtype=np.float32)
    return _model_lib().nro_dot_f16(order, _p(k), _p(q), min(k.size, q.size))


def axpy_f16(order: int, out: np.ndarray, a: float, v_bits: np.ndarray) -> np.ndarray:
    """kernels::axpy_f16 (kernels.rs:163-173): scalar, or axpy_f16_f16c (:203-220) with ORDER_AVX2."""
    o = np.ascontiguousarray(out, dtype=np.float32).copy()
    v = np.ascontiguousarray(v_bits, dtype=np.uint16)
    _model_lib().nro_axpy_f16(order, _p(o), a, _p(v), min(o.size, v.size))
    return o


class Model:
    """InferCtx restated on the CPU: scalar f32 order throughout by default;
    order=ORDER_AVX2 runs the x86 host's kernels instead (AVX2 matvec dots
    and 4-token prefill tiles, F16C attention dot and axpy)."""

    def __init__(self, cfg: dict, weights: dict, ctx: int, threads: int = 1, order: int = ORDER_SCALAR):
        L = _model_lib()
        dims = (C.c_int * 8)(cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                             cfg["ffn_dim"], cfg["vocab"], ctx)
        self.cfg, self.w, self.ctx = cfg, weights, ctx
        self.h = L.nro_model_new(dims, cfg["norm_eps"], cfg["rope_theta"], threads)
        L.nro_model_set_order(self.h, order)
        out = weights.get("output", weights["embed"])  # infer.rs:415-419: tied unless a head is given
        out_dt = weights.get("output_dtype", weights["embed_dtype"])
        L.nro_model_set_globals(self.h, _p(weights["embed"]), weights["embed_dtype"], _p(out), out_dt,
                                _p(weights["out_norm"]))
        for l, lw in enumerate(weights["layers"]):
            ptrs = (C.c_void_p * 7)(*[lw[n].ctypes.data for n in LAYER_MATS])
            dts = (C.c_int * 7)(*[lw["dtypes"][n] for n in LAYER_MATS])
            L.nro_model_set_layer(self.h, l, ptrs, dts, _p(lw["attn_norm"]), _p(lw["ffn_norm"]))
            if "q_norm" in lw:
                L.nro_model_set_qk_norm(self.h, l, _p(lw["q_norm"]), _p(lw["k_norm"]))
        r = cfg.get("recipe")
        if r:
            L.nro_model_set_recipe(self.h, int(r.get("rope") == "neox"), r.get("embed_scale", 1.0),
                                   r.get("attn_scale", 0.0), r.get("residual_scale", 1.0), r.get("logit_scale", 1.0))

    def __del__(self):
        if getattr(self, "h", None):
            _model_lib().nro_model_free(self.h)
            self.h = None

    @property
    def pos(self) -> int:
        return _model_lib().nro_model_pos(self.h)

    def seek(self, pos: int) -> None:
        """Timing aid: moves to `pos` without computing the cache rows before it."""
        _model_lib().nro_model_seek(self.h, pos)

    def set_freqs(self, freqs: np.ndarray) -> None:
        """Replaces the rope table (head_dim/2 floats), e.g. with infer_freqs' scaled one."""
        f = np.ascontiguousarray(freqs, np.float32)
        assert f.size == self.cfg["head_dim"] // 2
        _model_lib().nro_model_set_freqs(self.h, _p(f))

    def forward(self, token: int) -> np.ndarray:
        p = _model_lib().nro_model_forward(self.h, token)
        return np.ctypeslib.as_array(p, shape=(self.cfg["vocab"],)).copy()

    def prefill_chunk(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.uint32)
        assert 1 <= t.size <= 64
        p = _model_lib().nro_model_prefill_chunk(self.h, t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size)
        return np.ctypeslib.as_array(p, shape=(self.cfg["vocab"],)).copy()

    def prefill(self, tokens) -> np.ndarray:
        """InferCtx::prefill (infer.rs:753-759): chunks of MAX_BATCH = 64."""
        t = np.ascontiguousarray(tokens, np.uint32)
        out = None
        for i in range(0, t.size, 64):
            out = self.prefill_chunk(t[i:i + 64])
        return out

    def kv_cache(self):
        L = _model_lib()
        n = self.cfg["n_layers"] * self.ctx * self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        k = np.ctypeslib.as_array(L.nro_model_kcache(self.h), shape=(n,)).copy()
        v = np.ctypeslib.as_array(L.nro_model_vcache(self.h), shape=(n,)).copy()
        return k, v
