"""ctypes binding of libnrq.so (the C ABI in include/nrq.h).

There is no CPU fallback: if the library is missing, or no gfx950 device is
present, calls raise. The library is built in-tree by nightrun_amd/build.py.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnrq.so")

NRQ_OK = 0
NRQ_ERR_ARG = -1
NRQ_ERR_SHAPE = -2
NRQ_ERR_DEVICE = -3
NRQ_ERR_UNSUPPORTED = -4
NRQ_ERR_NOT_INIT = -5
# .nrm files: Model::parse's ParseError variants, verify_data's failure
NRQ_ERR_NRM_TOO_SHORT = -10
NRQ_ERR_NRM_BAD_MAGIC = -11
NRQ_ERR_NRM_BAD_VERSION = -12
NRQ_ERR_NRM_META_CRC = -13
NRQ_ERR_NRM_BAD_TABLE = -14
NRQ_ERR_NRM_MISSING_TENSOR = -15
NRQ_ERR_NRM_DATA_CRC = -16

Q8_0, Q4_K, Q6_K = 1, 2, 3
ORDER_SCALAR, ORDER_AVX2 = 0, 1

# Every symbol include/nrq.h declares, with its ctypes signature.
_vp, _sz, _i, _fp = C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_float)
SIGNATURES = {
    "nrq_init": ([_i], _i),
    "nrq_shutdown": ([], _i),
    "nrq_last_error": ([], C.c_char_p),
    "nrq_device_info": ([C.c_char_p, _sz], _i),
    "nrq_set_order": ([_i], _i),
    "nrq_get_order": ([], _i),
    "nrq_register_weights": ([_vp, _sz], _i),
    "nrq_unregister_weights": ([_vp], _i),
    "nrq_matvec_q8": ([_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz], _i),
    "nrq_matmul_q8": ([_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz], _i),
    "nrq_matvec_q4k": ([_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz], _i),
    "nrq_matvec_q6k": ([_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz], _i),
    "nrq_matmul_q4k": ([_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz], _i),
    "nrq_matmul_q6k": ([_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz], _i),
    "nrq_quantize": ([_vp, _sz, _vp, _sz], _i),
    "nrq_quantize_q8k": ([_vp, _sz, _vp, _sz], _i),
    "nrq_dev_matvec": ([_i, _i, _vp, _vp, _vp, _sz, _sz, _vp], _i),
    "nrq_dev_matmul": ([_i, _i, _vp, _vp, _vp, _sz, _sz, _sz, _vp], _i),
    "nrq_dev_matmul_group": ([_i, _i, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(_sz), _vp, _sz, _sz, _vp], _i),
    "nrq_dev_quantize_q8_0": ([_vp, _sz, _vp, _vp], _i),
    "nrq_dev_quantize_q8k": ([_vp, _sz, _vp, _vp], _i),
    "nrq_dev_block_sums": ([_i, _vp, _vp, _vp, _sz, _sz, _vp], _i),
    "nrq_sync": ([_vp], _i),
    "nrq_dev_stream_read": ([_vp, _sz, _vp, _vp], _i),
    "nrq_dev_mathf": ([_i, _vp, _vp, _sz, _vp], _i),
    "nrq_dev_rmsnorm": ([_vp, _vp, _vp, _sz, _sz, C.c_float, _vp], _i),
    "nrq_model_create": ([_vp, C.POINTER(_vp)], _i),
    "nrq_model_set_tensor": ([_vp, _i, _i, _i, _vp], _i),
    "nrq_model_reset": ([_vp], _i),
    "nrq_model_pos": ([_vp], _i),
    "nrq_model_forward": ([_vp, C.c_uint32, _vp], _i),
    "nrq_model_generate": ([_vp, C.c_uint32, _i, _vp, _vp], _i),
    "nrq_model_step_profile": ([_vp, C.c_uint32, _vp, _i], _i),
    "nrq_model_kv_cache": ([_vp, _vp, _vp, _sz], _i),
    "nrq_model_destroy": ([_vp], _i),
    "nrq_model_set_rope_freqs": ([_vp, _vp, _i], _i),
    "nrq_model_set_recipe": ([_vp, _i, C.c_float, C.c_float, C.c_float, C.c_float], _i),
    "nrq_model_prefill": ([_vp, _vp, _i, _vp], _i),
    "nrq_model_set_sampler": ([_vp, C.c_float, C.c_float, C.c_uint64], _i),
    "nrq_model_sampler_state": ([_vp, C.POINTER(C.c_uint64)], _i),
    "nrq_dev_sample": ([_vp, _i, C.c_float, C.c_float, _vp, _vp, _vp], _i),
    "nrq_dev_sample_noalloc": ([_vp, _i, C.c_float, C.c_float, _vp, _vp, _vp], _i),
    "nrq_nrm_open": ([_vp, _sz, C.POINTER(_vp)], _i),
    "nrq_nrm_get_meta": ([_vp, _vp], _i),
    "nrq_nrm_entry": ([_vp, C.c_uint32, _vp], _i),
    "nrq_nrm_tensor": ([_vp, _i, _i, _vp], _i),
    "nrq_nrm_has_tensor": ([_vp, _i], _i),
    "nrq_nrm_verify_data": ([_vp, _vp, _vp], _i),
    "nrq_nrm_close": ([_vp], _i),
    "nrq_crc32": ([C.c_uint32, _vp, _sz], C.c_uint32),
    "nrq_dev_crc32": ([_vp, _sz, C.c_uint32, _vp, _vp], _i),
    "nrq_model_load_nrm": ([_vp, _i, _i, C.POINTER(_vp)], _i),
}


class NrqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code
        self.msg = msg


class NrPanic(AssertionError):
    """A shape assertion the reference would have panicked on."""


_lib = None


def lib():
    """Loads libnrq.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python -m nightrun_amd.build` (no CPU fallback exists)")
        # torch first: it ships its own HIP runtime, and libnrq (whose
        # libamdhip64.so.7 then resolves to that copy) must share it; loaded
        # the other way round, torch finds no GPU
        import torch  # noqa: F401

        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, res
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != NRQ_OK:
        msg = lib().nrq_last_error().decode(errors="replace")
        if rc == NRQ_ERR_SHAPE:
            raise NrPanic(msg)
        raise NrqError(rc, msg)


_initialised = False


def init(device: int = 0) -> None:
    global _initialised
    if not _initialised:
        check(lib().nrq_init(device))
        _initialised = True


def device_info() -> str:
    init()
    buf = C.create_string_buffer(256)
    check(lib().nrq_device_info(buf, 256))
    return buf.value.decode()


def set_order(order: int) -> None:
    init()
    check(lib().nrq_set_order(order))


def get_order() -> int:
    return lib().nrq_get_order()
