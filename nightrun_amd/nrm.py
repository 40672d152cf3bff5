""".nrm v3 model files over libnrq (include/nrq.h ``nrq_nrm_*``): the role of
crates/nr-model/src/format.rs's ``Model`` (parse, tensor, has_tensor,
verify_data) and crc32.rs, with the data check and the upload on the GPU.

    f = NrmFile(blob)                      # Model::parse; raises ParseError(variant)
    f.meta["dim"], f.tensor(ATTN_Q, 0)["rows"]
    m = f.load(ctx=2048, verify=True)      # InferCtx::new -> nightrun_amd.model.Model
    toks = m.generate(first_token, 32)

``blob`` is any buffer (bytes, bytearray, mmap, numpy uint8); it is kept
alive by the handle, as the reference's ``Model<'a>`` borrows its blob.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

# TensorKind (format.rs:53-69)
TOK_EMBED, OUTPUT_NORM, OUTPUT, ROPE_FREQS = 1, 2, 3, 4
ATTN_NORM, ATTN_Q, ATTN_K, ATTN_V, ATTN_O = 10, 11, 12, 13, 14
FFN_NORM, FFN_GATE, FFN_UP, FFN_DOWN, ATTN_Q_NORM, ATTN_K_NORM = 15, 16, 17, 18, 19, 20
F32, Q8_0, Q4K, Q6K = 0, 1, 2, 3
ARCH_LLAMA3, ARCH_QWEN3, ARCH_GRANITE = 1, 2, 3
FLAG_TIED_EMBEDDINGS = 1
VERIFY_DATA = 1

VARIANTS = {
    _lib.NRQ_ERR_NRM_TOO_SHORT: "TooShort",
    _lib.NRQ_ERR_NRM_BAD_MAGIC: "BadMagic",
    _lib.NRQ_ERR_NRM_BAD_VERSION: "BadVersion",
    _lib.NRQ_ERR_NRM_META_CRC: "MetaCrc",
    _lib.NRQ_ERR_NRM_BAD_TABLE: "BadTable",
    _lib.NRQ_ERR_NRM_MISSING_TENSOR: "MissingTensor",
    _lib.NRQ_ERR_NRM_DATA_CRC: "DataCrc",
}


class ParseError(Exception):
    """format.rs:217-224 ParseError (plus verify.rs's DataCrc); ``variant`` names it."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code
        self.variant = VARIANTS.get(code, "Other")
        self.msg = msg


def _check(rc: int) -> None:
    if rc in VARIANTS:
        raise ParseError(rc, _lib.lib().nrq_last_error().decode(errors="replace"))
    _lib.check(rc)


class Meta(C.Structure):
    """nrq_nrm_meta: Meta (format.rs:126-156) + the header's section fields."""
    _fields_ = [(n, C.c_uint32) for n in ("arch", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                          "vocab", "ctx_train")] + \
               [(n, C.c_float) for n in ("rope_theta", "norm_eps", "rope_factor", "rope_low", "rope_high",
                                         "rope_orig_ctx")] + \
               [("flags", C.c_uint32)] + \
               [(n, C.c_float) for n in ("embed_scale", "attn_scale", "residual_scale", "logit_scale")] + \
               [("name", C.c_ubyte * 48), ("tok_off", C.c_uint64), ("tok_size", C.c_uint64), ("table_off", C.c_uint64),
                ("tensor_count", C.c_uint32), ("data_crc", C.c_uint32), ("meta_crc", C.c_uint32),
                ("reserved", C.c_uint32), ("data_off", C.c_uint64), ("data_size", C.c_uint64)]


class TensorInfo(C.Structure):
    """nrq_nrm_tensor_info: TensorEntry (format.rs:159-169)."""
    _fields_ = [(n, C.c_uint32) for n in ("kind", "layer", "dtype", "rows", "cols", "reserved")] + \
               [("offset", C.c_uint64), ("size", C.c_uint64)]


def _as_dict(s: C.Structure) -> dict:
    d = {n: getattr(s, n) for n, _ in s._fields_ if n != "reserved"}
    if "name" in d:
        d["name"] = bytes(d["name"])  # all 48 bytes, NUL padding included
    return d


def _buffer(blob):
    a = np.frombuffer(blob, np.uint8) if not isinstance(blob, np.ndarray) else np.ascontiguousarray(blob, np.uint8)
    return a, (a.ctypes.data if a.size else None), a.size


class NrmFile:
    """Model::parse over the C ABI; the parser runs on the host, no GPU needed."""

    def __init__(self, blob):
        self._arr, ptr, n = _buffer(blob)
        h = C.c_void_p()
        _check(_lib.lib().nrq_nrm_open(ptr, n, C.byref(h)))
        self.h = h
        m = Meta()
        _check(_lib.lib().nrq_nrm_get_meta(self.h, C.byref(m)))
        self.meta = _as_dict(m)

    def close(self):
        if getattr(self, "h", None):
            _lib.lib().nrq_nrm_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def entries(self):
        out = []
        for i in range(self.meta["tensor_count"]):
            t = TensorInfo()
            _check(_lib.lib().nrq_nrm_entry(self.h, i, C.byref(t)))
            out.append(_as_dict(t))
        return out

    def tensor(self, kind: int, layer: int) -> dict:
        """Model::tensor (format.rs:424-435); ParseError('MissingTensor') if absent."""
        t = TensorInfo()
        _check(_lib.lib().nrq_nrm_tensor(self.h, kind, layer, C.byref(t)))
        return _as_dict(t)

    def has_tensor(self, kind: int) -> bool:
        return bool(_lib.lib().nrq_nrm_has_tensor(self.h, kind))

    def data(self) -> np.ndarray:
        """The data section as a view of the blob."""
        o, n = self.meta["data_off"], self.meta["data_size"]
        return self._arr[o:o + n]

    def upload(self):
        """The data section in HBM (one copy), as a torch uint8 tensor."""
        import torch

        _lib.init(torch.cuda.current_device())
        return torch.from_numpy(np.ascontiguousarray(self.data())).cuda()

    def verify_data(self, dev_data=None) -> bool:
        """Model::verify_data (format.rs:409-422), the CRC computed on the GPU over a
        device copy of the data section (uploaded here unless given)."""
        import torch

        d = self.upload() if dev_data is None else dev_data
        rc = _lib.lib().nrq_nrm_verify_data(self.h, d.data_ptr(), torch.cuda.current_stream().cuda_stream)
        if rc == _lib.NRQ_ERR_NRM_DATA_CRC:
            return False
        _check(rc)
        return True

    def load(self, ctx: int, verify: bool = True):
        """InferCtx::new (infer.rs:352-447) on the device: a nightrun_amd.model.Model
        whose tensors live in one HBM copy of the data section."""
        import torch

        from .model import Model

        _lib.init(torch.cuda.current_device())
        h = C.c_void_p()
        _check(_lib.lib().nrq_model_load_nrm(self.h, ctx, VERIFY_DATA if verify else 0, C.byref(h)))
        M = self.meta
        cfg = dict(dim=M["dim"], n_layers=M["n_layers"], n_heads=M["n_heads"], n_kv_heads=M["n_kv_heads"],
                   head_dim=M["head_dim"], ffn_dim=M["ffn_dim"], vocab=M["vocab"], norm_eps=M["norm_eps"],
                   rope_theta=M["rope_theta"])
        return Model.from_handle(h, cfg, ctx)


def crc32(data, crc: int = 0) -> int:
    """crc32::checksum / Crc32::update (crc32.rs:38-79) on host bytes; zlib's running-value convention."""
    _, ptr, n = _buffer(data)
    return _lib.lib().nrq_crc32(crc, ptr, n)


def dev_crc32(t, crc: int = 0, nbytes: int | None = None, offset: int = 0) -> int:
    """The same CRC computed on the GPU over a torch tensor's bytes [offset, offset + nbytes)."""
    import torch

    _lib.init(torch.cuda.current_device())
    n = t.numel() * t.element_size() - offset if nbytes is None else nbytes
    out = torch.zeros(1, dtype=torch.int32, device=t.device)
    _lib.check(_lib.lib().nrq_dev_crc32(t.data_ptr() + offset, n, crc, out.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream))
    return int(out.cpu().item()) & 0xFFFFFFFF
