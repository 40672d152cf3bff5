"""Host side of the device-resident Llama-family decode (the C ABI's
nrq_model_*): the role of crates/nr-model's InferCtx (infer.rs:352-760) over
tensors that live in HBM.

    m = Model(cfg, ctx=1152)
    m.set_weights(weights)            # numpy block arrays -> HBM, bound once
    logits = m.forward(token)          # InferCtx::forward
    logits = m.prefill(prompt)         # InferCtx::prefill, batched chunks of up to 512 tokens
    toks = m.generate(token, n)        # greedy (sample.rs:33-35), one HIP graph per step

torch provides the device memory; every computation is a libnrq kernel.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

# TensorKind ids (crates/nr-model/src/format.rs:53-69)
TOK_EMBED, OUTPUT_NORM, OUTPUT = 1, 2, 3
ATTN_NORM, ATTN_Q, ATTN_K, ATTN_V, ATTN_O, FFN_NORM, FFN_GATE, FFN_UP, FFN_DOWN = 10, 11, 12, 13, 14, 15, 16, 17, 18
ATTN_Q_NORM, ATTN_K_NORM = 19, 20  # TensorKind (format.rs:53-69)
ROPE_ADJACENT, ROPE_NEOX = 0, 1
F32 = 0
LAYER_KINDS = {"wq": ATTN_Q, "wk": ATTN_K, "wv": ATTN_V, "wo": ATTN_O, "w_gate": FFN_GATE, "w_up": FFN_UP,
               "w_down": FFN_DOWN}


class ModelConfig(C.Structure):
    _fields_ = [("dim", C.c_int), ("n_layers", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("ffn_dim", C.c_int), ("vocab", C.c_int), ("ctx", C.c_int),
                ("norm_eps", C.c_float), ("rope_theta", C.c_float)]


class Model:
    def __init__(self, cfg: dict, ctx: int):
        import torch

        _lib.init(torch.cuda.current_device())
        self.cfg, self.ctx = dict(cfg), ctx
        c = ModelConfig(cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                        cfg["ffn_dim"], cfg["vocab"], ctx, cfg["norm_eps"], cfg["rope_theta"])
        h = C.c_void_p()
        _lib.check(_lib.lib().nrq_model_create(C.byref(c), C.byref(h)))
        self.h = h
        r = cfg.get("recipe")
        if r:  # Qwen3 / Granite (infer.rs:447-461)
            self.set_recipe(ROPE_NEOX if r.get("rope") == "neox" else ROPE_ADJACENT, r.get("embed_scale", 1.0),
                            r.get("attn_scale", 0.0), r.get("residual_scale", 1.0), r.get("logit_scale", 1.0))
        self._keep = []  # device tensors the model points at

    @classmethod
    def from_handle(cls, h, cfg: dict, ctx: int) -> "Model":
        """Wraps a model the C ABI already created (nrq_model_load_nrm)."""
        m = cls.__new__(cls)
        m.cfg, m.ctx, m.h, m._keep = dict(cfg), ctx, h, []
        return m

    def set_rope_freqs(self, freqs) -> None:
        """Replaces the rope table (head_dim/2 floats; InferCtx::new, infer.rs:433-447)."""
        f = np.ascontiguousarray(freqs, np.float32)
        _lib.check(_lib.lib().nrq_model_set_rope_freqs(self.h, f.ctypes.data, f.size))

    def close(self):
        if getattr(self, "h", None):
            _lib.lib().nrq_model_destroy(self.h)
            self.h = None
        self._keep = []

    def __del__(self):
        self.close()

    def _bind(self, kind: int, layer: int, dtype: int, arr: np.ndarray):
        import torch

        t = torch.from_numpy(np.ascontiguousarray(arr)).cuda()
        self._keep.append(t)
        _lib.check(_lib.lib().nrq_model_set_tensor(self.h, kind, layer, dtype, t.data_ptr()))

    def set_weights(self, w: dict) -> None:
        """w: {"embed", "embed_dtype", "out_norm", "layers": [{name: blocks, "dtypes": {...},
        "attn_norm", "ffn_norm"}], optional "output", "output_dtype"}, numpy arrays
        of blocks (matrices) and f32 (norms). Uploads every tensor once."""
        self._bind(TOK_EMBED, 0, w["embed_dtype"], w["embed"])
        if "output" in w:
            self._bind(OUTPUT, 0, w["output_dtype"], w["output"])
        self._bind(OUTPUT_NORM, 0, F32, w["out_norm"])
        for l, lw in enumerate(w["layers"]):
            self._bind(ATTN_NORM, l, F32, lw["attn_norm"])
            self._bind(FFN_NORM, l, F32, lw["ffn_norm"])
            for name, kind in LAYER_KINDS.items():
                self._bind(kind, l, lw["dtypes"][name], lw[name])
            if "q_norm" in lw:  # Qwen3 (infer.rs:393-404)
                self._bind(ATTN_Q_NORM, l, F32, lw["q_norm"])
                self._bind(ATTN_K_NORM, l, F32, lw["k_norm"])

    def set_recipe(self, rope_style: int, embed_scale: float = 1.0, attn_scale: float = 0.0,
                   residual_scale: float = 1.0, logit_scale: float = 1.0) -> None:
        """The recipe InferCtx::new takes from the file (infer.rs:447-461): rope
        pairs, muP embedding / attention-score / residual / logit scales."""
        _lib.check(_lib.lib().nrq_model_set_recipe(self.h, rope_style, embed_scale, attn_scale, residual_scale,
                                                   logit_scale))

    @property
    def pos(self) -> int:
        return _lib.lib().nrq_model_pos(self.h)

    def reset(self) -> None:
        _lib.check(_lib.lib().nrq_model_reset(self.h))

    def forward(self, token: int, logits: bool = True):
        out = np.empty(self.cfg["vocab"], np.float32) if logits else None
        _lib.check(_lib.lib().nrq_model_forward(self.h, int(token), out.ctypes.data if logits else None))
        return out

    def prefill(self, tokens, logits: bool = True):
        """InferCtx::prefill (infer.rs:753-759): the prompt in chunks of up to 512 tokens
        (the reference takes 64; the results are the same at any chunk size), each one
        batched pass; returns the last token's logits."""
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32) if logits else None
        _lib.check(_lib.lib().nrq_model_prefill(self.h, t.ctypes.data, t.size, out.ctypes.data if logits else None))
        return out

    def set_sampler(self, temperature: float, top_p: float, seed: int) -> None:
        """Sampler::new (sample.rs:15-21) for generate(): temperature <= 0 is greedy."""
        _lib.check(_lib.lib().nrq_model_set_sampler(self.h, temperature, top_p, seed & 0xFFFFFFFFFFFFFFFF))

    def sampler_state(self) -> int:
        st = C.c_uint64()
        _lib.check(_lib.lib().nrq_model_sampler_state(self.h, C.byref(st)))
        return st.value

    def generate(self, token: int, n: int, logits: bool = False):
        toks = np.empty(n, np.uint32)
        last = np.empty(self.cfg["vocab"], np.float32) if logits else None
        _lib.check(_lib.lib().nrq_model_generate(self.h, int(token), n, toks.ctypes.data,
                                                 last.ctypes.data if logits else None))
        return (toks, last) if logits else toks

    STEP_STAGES = ("embed", "norm_qkv", "attention", "o", "norm_gate_up_swiglu", "down", "final_norm", "head",
                   "argmax_or_sampler")

    def step_profile(self, token: int) -> dict:
        """One eager decode step of `token` with a HIP event after each stage
        (nrq_model_step_profile): microseconds per stage, summed over layers.
        Advances the position like forward()."""
        us = np.zeros(len(self.STEP_STAGES), np.float32)
        _lib.check(_lib.lib().nrq_model_step_profile(self.h, int(token), us.ctypes.data, us.size))
        return dict(zip(self.STEP_STAGES, (float(v) for v in us)))

    def kv_cache(self):
        n = self.cfg["n_layers"] * self.ctx * self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        k = np.empty(n, np.uint16)
        v = np.empty(n, np.uint16)
        _lib.check(_lib.lib().nrq_model_kv_cache(self.h, k.ctypes.data, v.ctypes.data, n * 2))
        return k, v


def sample(logits, temperature: float, top_p: float, rng):
    """Sampler::sample (sample.rs:32-96) on the device over a torch f32 tensor;
    rng: a one-element torch int64 tensor on the device holding the state
    (advanced in place). Returns the drawn id."""
    import torch

    _lib.init(torch.cuda.current_device())
    tok = torch.zeros(1, dtype=torch.int32, device=logits.device)
    _lib.check(_lib.lib().nrq_dev_sample(logits.data_ptr(), logits.numel(), temperature, top_p, rng.data_ptr(),
                                         tok.data_ptr(), torch.cuda.current_stream().cuda_stream))
    return int(tok.cpu().item())


def mathf(fn: int, x):
    """Device expf (fn 0) / sin (1) / cos (2) of sincosf over a torch tensor."""
    import torch

    y = torch.empty_like(x)
    _lib.init(torch.cuda.current_device())
    _lib.check(_lib.lib().nrq_dev_mathf(fn, x.data_ptr(), y.data_ptr(), x.numel(),
                                        torch.cuda.current_stream().cuda_stream))
    return y
