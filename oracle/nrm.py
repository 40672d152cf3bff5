"""The .nrm v3 container restated in Python -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py`` import this, as
the checker and to write test files; the product (``libnrq``'s C++ parser and
loader) never does.

* ``parse(blob)`` restates ``Model::parse`` (crates/nr-model/src/format.rs:260-406):
  it returns ``(meta, entries)`` or raises ``ParseError`` with the variant name
  (``TooShort``, ``BadMagic``, ``BadVersion``, ``MetaCrc``, ``BadTable``).
* ``tensor(entries, kind, layer)`` restates ``Model::tensor`` (format.rs:424-435).
* ``write(meta, tensors, tok_blob)`` lays out a file the way the converter does
  (header | tokenizer blob | tensor table | 64-byte-aligned data, both section
  CRCs), which is the layout crates/nr-model/tests/format_malformed.rs:9-71
  builds by hand; ``reseal`` restates that test's meta-CRC re-seal (:75-94).

Header field offsets (little-endian): magic 0, version 4, arch 8, dims 12..44
(dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, ctx_train),
f32 rope_theta 44, norm_eps 48, rope_factor 52, rope_low 56, rope_high 60,
rope_orig_ctx 64, u32 flags 68, f32 embed/attn/residual/logit scales 72..88,
name 88..136, u64 tok_off 136, tok_size 144, table_off 152, u32 count 160,
pad 164, u64 data_off 168, data_size 176, u32 data_crc 184, meta_crc 188.
Table entry (32 B): u16 kind, layer, dtype, pad; u64 offset, size; u32 rows, cols.
"""
from __future__ import annotations

import math
import struct

from . import crc32

MAGIC = b"NRUN"
VERSION = 3
HEADER_SIZE = 192
NAME_LEN = 48
ENTRY_SIZE = 32
DATA_ALIGN = 64
FLAG_TIED_EMBEDDINGS = 1
U64 = (1 << 64) - 1

ARCH_LLAMA3, ARCH_QWEN3, ARCH_GRANITE = 1, 2, 3
F32, Q8_0, Q4K, Q6K = 0, 1, 2, 3
# TensorKind (format.rs:53-69)
TOK_EMBED, OUTPUT_NORM, OUTPUT, ROPE_FREQS = 1, 2, 3, 4
ATTN_NORM, ATTN_Q, ATTN_K, ATTN_V, ATTN_O = 10, 11, 12, 13, 14
FFN_NORM, FFN_GATE, FFN_UP, FFN_DOWN, ATTN_Q_NORM, ATTN_K_NORM = 15, 16, 17, 18, 19, 20

META_U32 = ("dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "ctx_train")
META_F32A = ("rope_theta", "norm_eps", "rope_factor", "rope_low", "rope_high", "rope_orig_ctx")
META_F32B = ("embed_scale", "attn_scale", "residual_scale", "logit_scale")


class ParseError(Exception):
    def __init__(self, variant: str, detail=None):
        super().__init__(variant if detail is None else f"{variant}({detail})")
        self.variant = variant
        self.detail = detail


def byte_size(dtype: int, n: int):
    """TensorDtype::byte_size (format.rs:107-123); None where the Rust returns None."""
    if dtype == F32:
        v = n * 4
    elif dtype == Q8_0:
        v = n // 32 * 34 if n % 32 == 0 else None
    elif dtype == Q4K:
        v = n // 256 * 144 if n % 256 == 0 else None
    else:
        v = n // 256 * 210 if n % 256 == 0 else None
    return v if v is not None and v <= U64 else None


def _f32(b: bytes, off: int) -> float:
    return struct.unpack_from("<f", b, off)[0]


def parse(blob: bytes):
    """Model::parse (format.rs:260-406)."""
    b = bytes(blob)
    if len(b) < HEADER_SIZE:
        raise ParseError("TooShort")
    if b[0:4] != MAGIC:
        raise ParseError("BadMagic")
    version = struct.unpack_from("<I", b, 4)[0]
    if version != VERSION:
        raise ParseError("BadVersion", version)
    arch = struct.unpack_from("<I", b, 8)[0]
    if arch not in (ARCH_LLAMA3, ARCH_QWEN3, ARCH_GRANITE):
        raise ParseError("BadTable")
    meta = {"arch": arch}
    for i, k in enumerate(META_U32):
        meta[k] = struct.unpack_from("<I", b, 12 + 4 * i)[0]
    for i, k in enumerate(META_F32A):
        meta[k] = _f32(b, 44 + 4 * i)
    meta["flags"] = struct.unpack_from("<I", b, 68)[0]
    for i, k in enumerate(META_F32B):
        meta[k] = _f32(b, 72 + 4 * i)
    meta["name"] = b[88:136]
    tok_off, tok_size, table_off = struct.unpack_from("<QQQ", b, 136)
    count = struct.unpack_from("<I", b, 160)[0]
    data_off, data_size = struct.unpack_from("<QQ", b, 168)
    data_crc, meta_crc = struct.unpack_from("<II", b, 184)
    meta.update(tok_off=tok_off, tok_size=tok_size, table_off=table_off, tensor_count=count, data_off=data_off,
                data_size=data_size, data_crc=data_crc, meta_crc=meta_crc)
    # format.rs:316-327: scalar coherence
    es, at, rs, ls = (meta[k] for k in META_F32B)
    if (not math.isfinite(es) or not math.isfinite(at) or at < 0.0 or not math.isfinite(rs) or rs <= 0.0
            or not math.isfinite(ls) or ls <= 0.0):
        raise ParseError("BadTable")
    # format.rs:329-343: checked region ends (usize is 64-bit)
    table_len = count * ENTRY_SIZE
    if table_len > U64:
        raise ParseError("BadTable")
    table_end, data_end, tok_end = table_off + table_len, data_off + data_size, tok_off + tok_size
    if table_end > U64 or data_end > U64 or tok_end > U64:
        raise ParseError("TooShort")
    if len(b) < table_end or len(b) < data_end or len(b) < tok_end:
        raise ParseError("TooShort")
    # format.rs:345-357: meta CRC over header (crc fields zeroed) + tokenizer + table
    c = crc32(b[:HEADER_SIZE - 8])
    c = crc32(bytes(8), c)
    c = crc32(b[tok_off:tok_end], c)
    c = crc32(b[table_off:table_end], c)
    if c != meta_crc:
        raise ParseError("MetaCrc", (meta_crc, c))
    entries = []
    for i in range(count):
        o = table_off + ENTRY_SIZE * i
        kind, layer, dtype, _pad, offset, size, rows, cols = struct.unpack_from("<HHHHQQII", b, o)
        if dtype > Q6K:
            raise ParseError("BadTable")
        end = offset + size
        if end > U64 or end > data_size:
            raise ParseError("BadTable")
        if offset % DATA_ALIGN:
            raise ParseError("BadTable")
        if byte_size(dtype, rows * cols) != size:
            raise ParseError("BadTable")
        entries.append(dict(kind=kind, layer=layer, dtype=dtype, offset=offset, size=size, rows=rows, cols=cols))
    return meta, entries


def tensor(entries, kind: int, layer: int):
    """Model::tensor (format.rs:424-435): the first entry with this kind and layer, or None."""
    for e in entries:
        if e["kind"] == kind and e["layer"] == layer:
            return e
    return None


def meta_crc_of(b: bytes) -> int:
    """The seal of format_malformed.rs:75-94: regions clamped to the file."""
    tok_off, tok_size, table_off = struct.unpack_from("<QQQ", b, 136)
    count = struct.unpack_from("<I", b, 160)[0]
    c = crc32(b[:HEADER_SIZE - 8])
    c = crc32(bytes(8), c)
    t0 = min(tok_off, len(b))
    t1 = min(min(tok_off + tok_size, U64), len(b))
    c = crc32(b[t0:max(t1, t0)], c)
    e0 = min(table_off, len(b))
    e1 = min(min(table_off + min(count * ENTRY_SIZE, U64), U64), len(b))
    return crc32(b[e0:max(e1, e0)], c)


def reseal(b: bytearray) -> None:
    struct.pack_into("<I", b, 188, meta_crc_of(bytes(b)))


def default_meta(**kw) -> dict:
    m = dict(arch=ARCH_LLAMA3, dim=8, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=8, ffn_dim=8, vocab=16,
             ctx_train=128, rope_theta=0.0, norm_eps=0.0, rope_factor=0.0, rope_low=0.0, rope_high=0.0,
             rope_orig_ctx=0.0, flags=0, embed_scale=1.0, attn_scale=0.0, residual_scale=1.0, logit_scale=1.0,
             name=b"test")
    m.update(kw)
    return m


def write(meta: dict, tensors, tok_blob: bytes = b"\xee" * 16) -> bytearray:
    """A valid v3 file: header | tok_blob | table | data (64-byte aligned).
    tensors: [(kind, layer, dtype, rows, cols, payload bytes)]."""
    tok_off = HEADER_SIZE
    table_off = tok_off + len(tok_blob)
    data_off = -(-(table_off + ENTRY_SIZE * len(tensors)) // DATA_ALIGN) * DATA_ALIGN
    offs, pos = [], 0
    for t in tensors:
        offs.append(pos)
        pos = -(-(pos + len(t[5])) // DATA_ALIGN) * DATA_ALIGN
    data_size = offs[-1] + len(tensors[-1][5]) if tensors else 0
    b = bytearray(data_off + data_size)
    b[0:4] = MAGIC
    struct.pack_into("<II", b, 4, VERSION, meta["arch"])
    for i, k in enumerate(META_U32):
        struct.pack_into("<I", b, 12 + 4 * i, meta[k])
    for i, k in enumerate(META_F32A):
        struct.pack_into("<f", b, 44 + 4 * i, meta[k])
    struct.pack_into("<I", b, 68, meta["flags"])
    for i, k in enumerate(META_F32B):
        struct.pack_into("<f", b, 72 + 4 * i, meta[k])
    name = bytes(meta["name"])[:NAME_LEN]
    b[88:88 + len(name)] = name
    struct.pack_into("<QQQI", b, 136, tok_off, len(tok_blob), table_off, len(tensors))
    struct.pack_into("<QQ", b, 168, data_off, data_size)
    b[tok_off:tok_off + len(tok_blob)] = tok_blob
    for i, (t, off) in enumerate(zip(tensors, offs)):
        kind, layer, dtype, rows, cols, payload = t
        struct.pack_into("<HHHHQQII", b, table_off + ENTRY_SIZE * i, kind, layer, dtype, 0, off, len(payload), rows,
                         cols)
        b[data_off + off:data_off + off + len(payload)] = payload
    struct.pack_into("<I", b, 184, crc32(bytes(b[data_off:data_off + data_size])))
    reseal(b)
    return b


def tiny() -> bytearray:
    """The smallest valid file: one 8x8 F32 TokEmbed (format_malformed.rs:9-71)."""
    return write(default_meta(), [(TOK_EMBED, 0, F32, 8, 8, bytes(256))])


def model_tensors(cfg: dict, weights: dict, tied: bool = True, rope_factors=None):
    """The tensor list of a model in the oracle's weight dict (gen_model's layout),
    with Qwen3's per-head q/k norms when its layers carry them."""
    import numpy as np

    d, att, kvd, ffn = cfg["dim"], cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"], cfg["ffn_dim"]
    shapes = {"wq": (ATTN_Q, att, d), "wk": (ATTN_K, kvd, d), "wv": (ATTN_V, kvd, d), "wo": (ATTN_O, d, att),
              "w_gate": (FFN_GATE, ffn, d), "w_up": (FFN_UP, ffn, d), "w_down": (FFN_DOWN, d, ffn)}
    raw = lambda a: np.ascontiguousarray(a).tobytes()  # noqa: E731
    t = [(TOK_EMBED, 0, weights["embed_dtype"], cfg["vocab"], d, raw(weights["embed"])),
         (OUTPUT_NORM, 0, F32, 1, d, raw(weights["out_norm"]))]
    if not tied:
        t.append((OUTPUT, 0, weights["output_dtype"], cfg["vocab"], d, raw(weights["output"])))
    if rope_factors is not None:
        t.append((ROPE_FREQS, 0, F32, 1, cfg["head_dim"] // 2, raw(np.asarray(rope_factors, np.float32))))
    for l, lw in enumerate(weights["layers"]):
        t.append((ATTN_NORM, l, F32, 1, d, raw(lw["attn_norm"])))
        if "q_norm" in lw:
            t.append((ATTN_Q_NORM, l, F32, 1, cfg["head_dim"], raw(lw["q_norm"])))
            t.append((ATTN_K_NORM, l, F32, 1, cfg["head_dim"], raw(lw["k_norm"])))
        t.append((FFN_NORM, l, F32, 1, d, raw(lw["ffn_norm"])))
        for name, (kind, rows, cols) in shapes.items():
            t.append((kind, l, lw["dtypes"][name], rows, cols, raw(lw[name])))
    return t
