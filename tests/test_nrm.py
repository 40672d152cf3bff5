"""The .nrm container on the CPU: the oracle's CRC-32 and parser pinned against
the reference's own tests, and libnrq's host parser and host CRC checked
against the oracle (host logic only; no GPU call).

Pins (crates/nr-model/tests/verify.rs, format_malformed.rs):
* CRC-32 known values ("123456789" -> 0xCBF43926, "" -> 0, "a" -> 0xE8B7BE43),
  the slicing-by-8 form equal to the classic bitwise algorithm on the
  xorshift64 stream at lengths 0, 1, 7, 8, 9, 63, 100003, and to zlib.crc32
  (the textbook IEEE CRC-32 of the standard library);
* every malformed file of format_malformed.rs rejected, with MetaCrc for the
  flipped name byte, and the tiny valid file accepted with its values;
* libnrq's parser agreeing with the oracle's on accept/reject, the error
  variant, the meta and every entry, over those files and 3000 seeded
  mutations (byte flips, adversarial field values; half re-sealed so the
  meta-CRC gate is passed and the checks behind it are reached).
"""
import struct
import zlib

import numpy as np
import pytest

from oracle import nrm as ON

U64MAX = (1 << 64) - 1


def xorshift_bytes(n):
    """crates/nr-model/tests/verify.rs:31-39."""
    x, out = 0x12345678, bytearray(n)
    m = U64MAX
    for i in range(n):
        x ^= (x << 13) & m
        x ^= x >> 7
        x ^= (x << 17) & m
        out[i] = x & 0xFF
    return bytes(out)


def test_crc32_known_vectors(oracle):
    for f in (oracle.crc32, oracle.crc32_bitwise):
        assert f(b"123456789") == 0xCBF43926
        assert f(b"") == 0
        assert f(b"a") == 0xE8B7BE43


def test_crc32_slicing_equals_classic(oracle):
    data = xorshift_bytes(100_003)
    for n in (0, 1, 7, 8, 9, 63, 100_003):
        want = oracle.crc32_bitwise(data[:n])
        assert oracle.crc32(data[:n]) == want, n
        assert zlib.crc32(data[:n]) == want, n


def test_crc32_running_value(oracle):
    data = np.random.default_rng(5).integers(0, 256, 70_001, dtype=np.uint8).tobytes()
    whole = oracle.crc32(data)
    for cut in (0, 1, 8, 4097, 70_000, 70_001):
        assert oracle.crc32(data[cut:], oracle.crc32(data[:cut])) == whole


def test_host_crc32_matches_oracle(oracle):
    """libnrq's host CRC (nrq_crc32, the meta-CRC gate of its parser)."""
    from nightrun_amd import nrm

    data = np.random.default_rng(6).integers(0, 256, 300_007, dtype=np.uint8).tobytes()
    assert nrm.crc32(b"123456789") == 0xCBF43926
    assert nrm.crc32(b"") == 0
    for n in (0, 1, 7, 8, 9, 15, 16, 17, 63, 64, 1000, 300_007):
        assert nrm.crc32(data[:n]) == oracle.crc32(data[:n]), n
    assert nrm.crc32(data[77:], nrm.crc32(data[:77])) == oracle.crc32(data)


# ---- format_malformed.rs, restated ----------------------------------------------------

def _table_off(b):
    return struct.unpack_from("<Q", b, 152)[0]


def malformed_cases():
    """(name, bytes) for every case of format_malformed.rs:110-208."""
    cases = []
    b = bytes(ON.tiny())
    for cut in (0, 3, 4, 100, ON.HEADER_SIZE - 1, ON.HEADER_SIZE, len(b) - 1):
        cases.append((f"truncated to {cut}", b[:cut]))
    m = bytearray(b)
    m[0] = ord("X")
    cases.append(("magic", bytes(m)))
    m = bytearray(b)
    struct.pack_into("<I", m, 4, 99)
    cases.append(("version", bytes(m)))
    for name, edits in (("wrapping tok_off", [(136, "<Q", U64MAX - 4)]),
                        ("wrapping data_off", [(168, "<Q", U64MAX - 4)]),
                        ("wrapping table", [(152, "<Q", U64MAX - 31), (160, "<I", 0xFFFFFFFF)])):
        m = bytearray(b)
        for off, fmt, v in edits:
            struct.pack_into(fmt, m, off, v)
        ON.reseal(m)
        cases.append((name, bytes(m)))
    t = _table_off(b)
    for name, edits in (("entry offset+size wrap", [(t + 8, "<Q", U64MAX - 63)]),
                        ("misaligned tensor offset", [(t + 8, "<Q", 4)]),
                        ("rows*cols overflow", [(t + 24, "<I", 0xFFFFFFFF), (t + 28, "<I", 0xFFFFFFFF)]),
                        ("size/dtype mismatch", [(t + 16, "<Q", 8)])):
        m = bytearray(b)
        for off, fmt, v in edits:
            struct.pack_into(fmt, m, off, v)
        ON.reseal(m)
        cases.append((name, bytes(m)))
    m = bytearray(b)
    m[100] ^= 0x40
    cases.append(("meta crc flip", bytes(m)))
    m = bytearray(b)
    struct.pack_into("<f", m, 80, float("nan"))
    ON.reseal(m)
    cases.append(("NaN residual scale", bytes(m)))
    return cases


def oracle_outcome(blob):
    try:
        meta, entries = ON.parse(blob)
    except ON.ParseError as e:
        return ("err", e.variant)
    return ("ok", meta, entries)


def product_outcome(blob):
    from nightrun_amd import nrm

    try:
        f = nrm.NrmFile(blob)
    except nrm.ParseError as e:
        return ("err", e.variant)
    meta, entries = f.meta, f.entries()
    f.close()
    return ("ok", meta, entries)


def same_outcome(a, b):
    if a[0] != b[0]:
        return False
    if a[0] == "err":
        return a[1] == b[1]
    ma, ea = a[1], a[2]
    mb, eb = b[1], b[2]
    for k, v in ma.items():
        w = mb[k]
        if isinstance(v, float):
            if not (np.float32(v).view(np.uint32) == np.float32(w).view(np.uint32)):
                return False
        elif v != w:
            return False
    return ea == [{k: e[k] for k in ea[0]} for e in eb] if ea else not eb


def test_oracle_parses_tiny_file():
    """format_malformed.rs:96-103."""
    meta, entries = ON.parse(bytes(ON.tiny()))
    assert meta["dim"] == 8
    e = ON.tensor(entries, ON.TOK_EMBED, 0)
    assert (e["rows"], e["cols"]) == (8, 8) and e["size"] // 4 == 64


def test_oracle_rejects_every_malformed_file():
    for name, blob in malformed_cases():
        out = oracle_outcome(blob)
        assert out[0] == "err", name
        if name == "meta crc flip":
            assert out[1] == "MetaCrc"


def test_product_parser_matches_oracle_on_reference_cases():
    cases = [("tiny", bytes(ON.tiny()))] + malformed_cases()
    for name, blob in cases:
        a, b = oracle_outcome(blob), product_outcome(blob)
        assert same_outcome(a, b), (name, a, b)
    assert product_outcome(bytes(ON.tiny()))[0] == "ok"


def _multi_tensor_file():
    """Four tensors of every dtype, each 64-byte aligned."""
    t = [(ON.TOK_EMBED, 0, ON.Q8_0, 4, 64, bytes(range(256)) + bytes(16)),
         (ON.ATTN_NORM, 0, ON.F32, 1, 8, bytes(32)),
         (ON.ATTN_Q, 0, ON.Q4K, 1, 256, bytes(144)),
         (ON.FFN_DOWN, 3, ON.Q6K, 2, 256, bytes(420))]
    return ON.write(ON.default_meta(n_layers=4), t, tok_blob=b"tok" * 7)


FIELDS = [(4, "<I"), (8, "<I"), (12, "<I"), (72, "<f"), (76, "<f"), (80, "<f"), (84, "<f"), (136, "<Q"), (144, "<Q"),
          (152, "<Q"), (160, "<I"), (168, "<Q"), (176, "<Q"), (184, "<I")]
ENTRY_FIELDS = [(0, "<H"), (2, "<H"), (4, "<H"), (8, "<Q"), (16, "<Q"), (24, "<I"), (28, "<I")]


def _mutate(rng, b):
    m = bytearray(b)
    kind = rng.integers(0, 4)
    if kind == 0:  # byte flips anywhere
        for _ in range(int(rng.integers(1, 4))):
            i = int(rng.integers(0, len(m)))
            m[i] ^= 1 << int(rng.integers(0, 8))
    elif kind in (1, 2):  # a header or table field set to an adversarial value
        if kind == 1:
            off, fmt = FIELDS[int(rng.integers(0, len(FIELDS)))]
        else:
            n = struct.unpack_from("<I", b, 160)[0]
            eo, fmt = ENTRY_FIELDS[int(rng.integers(0, len(ENTRY_FIELDS)))]
            off = _table_off(b) + 32 * int(rng.integers(0, n)) + eo
        bits = {"<H": 16, "<I": 32, "<Q": 64, "<f": 32}[fmt]
        if fmt == "<f":
            vals = [np.nan, np.inf, -np.inf, -1.0, 0.0, 1.0, 2.5, 1e-30]
        else:
            top = (1 << bits) - 1
            vals = [0, 1, 3, 4, 63, 64, 65, 256, top, top - 4, top - 31, top - 63,
                    int(rng.integers(0, 1 << min(bits, 62)))]
        v = vals[int(rng.integers(0, len(vals)))]
        struct.pack_into(fmt, m, off, v)
    else:  # truncation
        m = m[:int(rng.integers(0, len(m)))]
    if rng.integers(0, 2) and len(m) >= ON.HEADER_SIZE:
        ON.reseal(m)
    return bytes(m)


def test_product_parser_matches_oracle_on_mutations():
    rng = np.random.default_rng(2024)
    bases = [bytes(ON.tiny()), bytes(_multi_tensor_file())]
    accepted = rejected = 0
    for i in range(3000):
        blob = _mutate(rng, bases[i % 2])
        a, b = oracle_outcome(blob), product_outcome(blob)
        assert same_outcome(a, b), (i, a, b)
        accepted += a[0] == "ok"
        rejected += a[0] == "err"
    assert accepted > 100 and rejected > 1000, (accepted, rejected)


def test_missing_tensor_is_reported_by_name():
    from nightrun_amd import nrm

    f = nrm.NrmFile(bytes(_multi_tensor_file()))
    assert f.tensor(ON.FFN_DOWN, 3)["rows"] == 2
    assert f.has_tensor(ON.ATTN_Q) and not f.has_tensor(ON.ATTN_K)
    with pytest.raises(nrm.ParseError, match="attn_k") as e:
        f.tensor(ON.ATTN_K, 0)
    assert e.value.variant == "MissingTensor"
    with pytest.raises(nrm.ParseError, match="ffn_down"):
        f.tensor(ON.FFN_DOWN, 0)


# ---- InferCtx::new's rope table --------------------------------------------------------

def test_infer_freqs_scaling_branches(oracle):
    """rope.rs:20-31 for Llama 3.2's scaling (factor 32, low 1, high 4, original
    context 8192, theta 500000, head_dim 64): frequencies whose wavelength is
    below 8192/4 are the unscaled ones bit for bit, those above 8192/1 are the
    unscaled ones divided by 32 exactly (IEEE division), and the blend in
    between lies strictly between the two and falls with i."""
    hd, theta = 64, 500000.0
    base = oracle.rope_freqs(hd, theta)
    got = oracle.infer_freqs(hd, theta, 32.0, 1.0, 4.0, 8192.0)
    wl = (np.float32(2.0) * np.float32(np.pi)) / base
    hi, lo, mid = wl < np.float32(2048.0), wl > np.float32(8192.0), (wl > np.float32(2048.0)) & (wl <= np.float32(8192.0))
    assert hi.sum() and lo.sum() and mid.sum()
    assert np.array_equal(got[hi].view(np.uint32), base[hi].view(np.uint32))
    assert np.array_equal(got[lo].view(np.uint32), (base[lo] / np.float32(32.0)).view(np.uint32))
    assert np.all(got[mid] < base[mid]) and np.all(got[mid] > base[mid] / np.float32(32.0))
    assert np.all(np.diff(got) < 0)
    # factor 0 is no scaling; a factors tensor divides the base spectrum and overrides scaling
    assert np.array_equal(oracle.infer_freqs(hd, theta).view(np.uint32), base.view(np.uint32))
    fac = np.linspace(1.0, 40.0, hd // 2).astype(np.float32)
    want = (base / fac).view(np.uint32)
    assert np.array_equal(oracle.infer_freqs(hd, theta, 32.0, 1.0, 4.0, 8192.0, factors=fac).view(np.uint32), want)


def test_loader_widths_do_not_wrap_32_bits():
    """InferCtx::new computes att_dim = n_heads * head_dim in usize
    (infer.rs:60-73, 401-404). A header with n_heads = 2^25 and head_dim = 128
    has att_dim = 2^32; a q matrix stored with 0 rows (what 2^32 wraps to in
    32 bits) is then a shape mismatch, MissingTensor("bad matrix shape"), and
    the loader must stop there, before any device allocation. Host-only: the
    check runs before the model is created."""
    import ctypes as C

    from nightrun_amd import _lib, nrm

    cfg = dict(dim=256, n_layers=1, n_heads=1 << 25, n_kv_heads=1 << 25, head_dim=128, ffn_dim=256, vocab=4)
    emb = bytes(4 * 256 // 32 * 34)
    t = [(ON.TOK_EMBED, 0, 1, 4, 256, emb), (ON.OUTPUT_NORM, 0, ON.F32, 1, 256, bytes(1024)),
         (ON.ATTN_NORM, 0, ON.F32, 1, 256, bytes(1024)), (ON.FFN_NORM, 0, ON.F32, 1, 256, bytes(1024))]
    # q/k/v with the wrapped row count 0 and o with the wrapped column count 0: 0-byte tensors
    t += [(ON.ATTN_Q, 0, 1, 0, 256, b""), (ON.ATTN_K, 0, 1, 0, 256, b""), (ON.ATTN_V, 0, 1, 0, 256, b""),
          (ON.ATTN_O, 0, 1, 256, 0, b"")]
    t += [(k, 0, 1, r, c, bytes(r * c // 32 * 34)) for k, r, c in
          ((ON.FFN_GATE, 256, 256), (ON.FFN_UP, 256, 256), (ON.FFN_DOWN, 256, 256))]
    blob = bytes(ON.write(ON.default_meta(**cfg, flags=ON.FLAG_TIED_EMBEDDINGS), t))
    f = nrm.NrmFile(blob)  # Model::parse accepts it: every entry's size is its block math
    h = C.c_void_p()
    rc = _lib.lib().nrq_model_load_nrm(f.h, 64, 0, C.byref(h))
    assert rc == -15 and not h.value  # NRQ_ERR_NRM_MISSING_TENSOR, no model
    assert "bad matrix shape" in _lib.lib().nrq_last_error().decode()
    f.close()
