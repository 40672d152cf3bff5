"""Device-resident entry points of libnrq over torch tensors.

torch supplies device memory and streams only; every computation is a libnrq
kernel launch on the given stream (default: torch's current stream).
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import ORDER_AVX2, ORDER_SCALAR, Q4_K, Q6_K, Q8_0  # noqa: F401

QK = {Q8_0: 32, Q4_K: 256, Q6_K: 256}
WBYTES = {Q8_0: 34, Q4_K: 144, Q6_K: 210}
XBYTES = {Q8_0: 34, Q4_K: 292, Q6_K: 292}


def _stream(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dev(t: torch.Tensor, what: str):
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{what}: expected a contiguous device tensor")
    return t.data_ptr()


def matvec(dtype: int, order: int, y: torch.Tensor, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
           stream=None) -> None:
    _lib.init(torch.cuda.current_device())
    _lib.check(_lib.lib().nrq_dev_matvec(dtype, order, _dev(y, "y"), _dev(w, "w"), _dev(x, "x"), rows, cols,
                                         _stream(stream)))


def matmul(dtype: int, order: int, y: torch.Tensor, w: torch.Tensor, xs: torch.Tensor, rows: int, cols: int,
           batch: int, stream=None) -> None:
    _lib.init(torch.cuda.current_device())
    _lib.check(_lib.lib().nrq_dev_matmul(dtype, order, _dev(y, "y"), _dev(w, "w"), _dev(xs, "xs"), rows, cols,
                                         batch, _stream(stream)))


def matmul_group(dtype: int, ys, ws, rows, xs: torch.Tensor, cols: int, batch: int, stream=None) -> None:
    """Acts::matmul_group (infer.rs:180-228): 1-3 matrices over one activation, scalar order."""
    import ctypes as C

    _lib.init(torch.cuda.current_device())
    n = len(ws)
    yp = (C.c_void_p * n)(*[_dev(y, "y") for y in ys])
    wp = (C.c_void_p * n)(*[_dev(w, "w") for w in ws])
    rp = (C.c_size_t * n)(*rows)
    _lib.check(_lib.lib().nrq_dev_matmul_group(dtype, n, yp, wp, rp, _dev(xs, "xs"), cols, batch, _stream(stream)))


def quantize_q8_0(src: torch.Tensor, out: torch.Tensor, stream=None) -> None:
    _lib.init(torch.cuda.current_device())
    _lib.check(_lib.lib().nrq_dev_quantize_q8_0(_dev(src, "src"), src.numel(), _dev(out, "out"), _stream(stream)))


def quantize_q8k(src: torch.Tensor, out: torch.Tensor, stream=None) -> None:
    _lib.init(torch.cuda.current_device())
    _lib.check(_lib.lib().nrq_dev_quantize_q8k(_dev(src, "src"), src.numel(), _dev(out, "out"), _stream(stream)))


def block_sums(dtype: int, out: torch.Tensor, w: torch.Tensor, x: torch.Tensor, rows: int, cols: int,
               stream=None) -> None:
    _lib.init(torch.cuda.current_device())
    _lib.check(_lib.lib().nrq_dev_block_sums(dtype, _dev(w, "w"), _dev(x, "x"), _dev(out, "out"), rows, cols,
                                             _stream(stream)))
