"""nightrun_amd: MI355X (gfx950) quantized matrix kernels, a drop-in for the
quantized matvec/matmul path of the reference's nr-tensor crate.

    nightrun_amd/csrc/     HIP kernels and the C ABI (include/nrq.h) -> libnrq.so
    nightrun_amd/build.py  builds libnrq.so for gfx950
    nightrun_amd/nr_tensor mirror of nr-tensor's API over host slices
    nightrun_amd/device    device-resident entry points over torch tensors
"""
from ._lib import (NRQ_ERR_ARG, NRQ_ERR_DEVICE, NRQ_ERR_NOT_INIT, NRQ_ERR_SHAPE,  # noqa: F401
                   NRQ_ERR_UNSUPPORTED, ORDER_AVX2, ORDER_SCALAR, Q4_K, Q6_K, Q8_0, NrPanic, NrqError,
                   device_info, get_order, init, set_order)
