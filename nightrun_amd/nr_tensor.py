"""Host-side mirror of the reference's nr-tensor API, over libnrq's C ABI.

Same function names, argument meaning and error behaviour as
crates/nr-tensor: `kernels.matvec_q8(y, w, x, rows, cols)` writes y in place,
and a shape mismatch raises NrPanic with the reference assertion's text (the
Rust functions panic). Block slices are numpy uint8 arrays of shape
(nblocks, block_bytes); `len(w)` is the slice length in blocks.

    from nightrun_amd.nr_tensor import kernels, kquant, q8
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import NrPanic, Q4_K, Q6_K, Q8_0  # noqa: F401  (re-exported)

QK8_0 = 32  # q8.rs:7
QK_K = 256  # kquant.rs:20
BLOCK_Q8_0_BYTES = 34
BLOCK_Q4K_BYTES = 144
BLOCK_Q6K_BYTES = 210
BLOCK_Q8K_BYTES = 292


def _ptr(a: np.ndarray):
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return C.c_void_p(a.ctypes.data) if a.size else None


def _blocks(a: np.ndarray, nbytes: int, what: str) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != np.uint8:
        raise TypeError(f"{what}: blocks must be uint8")
    if a.ndim == 1:
        if a.size % nbytes:
            raise ValueError(f"{what}: {a.size} bytes is not a whole number of {nbytes}-byte blocks")
        a = a.reshape(-1, nbytes)
    if a.ndim != 2 or a.shape[1] != nbytes:
        raise ValueError(f"{what}: expected shape (n, {nbytes}), got {a.shape}")
    return a


def _f32(y: np.ndarray, what: str) -> np.ndarray:
    if not isinstance(y, np.ndarray) or y.dtype != np.float32 or not y.flags["C_CONTIGUOUS"]:
        raise TypeError(f"{what}: expected a C-contiguous float32 array")
    return y


def _call_mv(fn, y, w, wb, x, xb, rows, cols, batch=None):
    _lib.init()
    y = _f32(y, "y")
    w = _blocks(w, wb, "w")
    x = _blocks(x, xb, "x")
    args = [_ptr(y), y.size, _ptr(w), w.shape[0], _ptr(x), x.shape[0], rows, cols]
    if batch is not None:
        args.append(batch)
    _lib.check(fn(*args))


class kernels:
    """crates/nr-tensor/src/kernels.rs"""

    @staticmethod
    def matvec_q8(y: np.ndarray, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> None:
        """kernels.rs:36-47"""
        _call_mv(_lib.lib().nrq_matvec_q8, y, w, BLOCK_Q8_0_BYTES, x, BLOCK_Q8_0_BYTES, rows, cols)

    @staticmethod
    def matmul_q8(y: np.ndarray, w: np.ndarray, xs: np.ndarray, rows: int, cols: int, batch: int) -> None:
        """kernels.rs:91-143; y is [batch][rows]."""
        _call_mv(_lib.lib().nrq_matmul_q8, y, w, BLOCK_Q8_0_BYTES, xs, BLOCK_Q8_0_BYTES, rows, cols, batch)


class kquant:
    """crates/nr-tensor/src/kquant.rs"""

    QK_K = QK_K

    @staticmethod
    def matvec_q4k(y, w, x, rows: int, cols: int) -> None:
        """kquant.rs:563 (kquant_matvec! instance)"""
        _call_mv(_lib.lib().nrq_matvec_q4k, y, w, BLOCK_Q4K_BYTES, x, BLOCK_Q8K_BYTES, rows, cols)

    @staticmethod
    def matvec_q6k(y, w, x, rows: int, cols: int) -> None:
        """kquant.rs:564"""
        _call_mv(_lib.lib().nrq_matvec_q6k, y, w, BLOCK_Q6K_BYTES, x, BLOCK_Q8K_BYTES, rows, cols)

    @staticmethod
    def matmul_q4k(y, w, xs, rows: int, cols: int, batch: int) -> None:
        """kquant.rs:626-632 (kquant_matmul! instance)"""
        _call_mv(_lib.lib().nrq_matmul_q4k, y, w, BLOCK_Q4K_BYTES, xs, BLOCK_Q8K_BYTES, rows, cols, batch)

    @staticmethod
    def matmul_q6k(y, w, xs, rows: int, cols: int, batch: int) -> None:
        """kquant.rs:633-639"""
        _call_mv(_lib.lib().nrq_matmul_q6k, y, w, BLOCK_Q6K_BYTES, xs, BLOCK_Q8K_BYTES, rows, cols, batch)

    @staticmethod
    def quantize_q8k(src: np.ndarray, out: np.ndarray) -> None:
        """kquant.rs:157-187; fills `out` (n, 292) in place."""
        _lib.init()
        src = np.ascontiguousarray(src, dtype=np.float32)
        out = _blocks(out, BLOCK_Q8K_BYTES, "out")
        _lib.check(_lib.lib().nrq_quantize_q8k(_ptr(src), src.size, _ptr(out), out.shape[0]))


class q8:
    """crates/nr-tensor/src/q8.rs"""

    QK8_0 = QK8_0

    @staticmethod
    def quantize(src: np.ndarray, out: np.ndarray) -> None:
        """q8.rs:27-44; fills `out` (n, 34) in place."""
        _lib.init()
        src = np.ascontiguousarray(src, dtype=np.float32)
        out = _blocks(out, BLOCK_Q8_0_BYTES, "out")
        _lib.check(_lib.lib().nrq_quantize(_ptr(src), src.size, _ptr(out), out.shape[0]))


def register_weights(w: np.ndarray) -> None:
    """Uploads a weight array to HBM once (InferCtx::new time)."""
    _lib.init()
    w = np.ascontiguousarray(w)
    _lib.check(_lib.lib().nrq_register_weights(_ptr(w), w.nbytes))


def unregister_weights(w: np.ndarray) -> None:
    _lib.check(_lib.lib().nrq_unregister_weights(_ptr(w)))
