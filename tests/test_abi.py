"""The C-ABI library loads and exports every symbol include/nrq.h declares.

CPU only: no compute call is made. Without a GPU every entry point must
fail loudly (no CPU fallback exists).
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nrq.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|uint32_t|const char \*)\s*(nrq_\w+)\(", text, flags=re.M)))


def test_header_declares_the_c_abi():
    syms = declared_symbols()
    assert "nrq_init" in syms and "nrq_matvec_q8" in syms and "nrq_dev_matmul" in syms
    assert len(syms) == 52


def test_library_exports_every_declared_symbol():
    from nightrun_amd import _lib

    L = C.CDLL(_lib.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(L, name), name
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_library_is_gfx950_only():
    """The fat binary carries a gfx950 code object and no other GPU target."""
    from nightrun_amd import _lib

    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"--gfx942", b"--gfx90a", b"--gfx908", b"--gfx1100", b"sm_"):
        assert other not in blob


def _no_gpu():
    import torch

    return not torch.cuda.is_available()


@pytest.mark.skipif(not _no_gpu(), reason="checks the no-GPU failure path")
def test_no_gpu_fails_loudly():
    import nightrun_amd
    from nightrun_amd import _lib
    from nightrun_amd.nr_tensor import kernels

    L = _lib.lib()
    assert L.nrq_init(0) == _lib.NRQ_ERR_DEVICE
    assert L.nrq_last_error()
    y = np.zeros(4, dtype=np.float32)
    w = np.zeros((4, 34), dtype=np.uint8)
    x = np.zeros((1, 34), dtype=np.uint8)
    assert L.nrq_matvec_q8(y.ctypes.data, 4, w.ctypes.data, 4, x.ctypes.data, 1, 4, 32) == _lib.NRQ_ERR_NOT_INIT
    assert L.nrq_dev_matvec(1, 0, None, None, None, 4, 32, None) == _lib.NRQ_ERR_NOT_INIT
    with pytest.raises(nightrun_amd.NrqError):
        kernels.matvec_q8(y, w, x, 4, 32)


def test_oracle_is_not_reachable_from_the_product():
    """Nothing in nightrun_amd/ or the C sources names the oracle."""
    pkg = os.path.join(ROOT, "nightrun_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), os.path.join(dirpath, f)


def test_m0_is_written_only_by_the_dma_asm():
    """The LDS DMA helpers (nrq_wstream.hip, nrq_model.hip) set m0 in inline
    asm right before their global_load_lds instruction, without the compiler
    knowing (the compiler-tracked builtin adds vmcnt(0) waits that stall the
    DMA pipelines). That is sound only while no compiler-generated code keeps
    a value in m0: this disassembles the library's gfx950 code objects and
    checks that every instruction naming m0 is such an `s_mov_b32 m0, sN`
    directly followed by a global_load_lds, and that no instruction which
    reads m0 implicitly appears."""
    import glob
    import shutil
    import subprocess
    import tempfile

    from nightrun_amd import _lib

    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not installed")
    with tempfile.TemporaryDirectory() as tmp:
        lib = os.path.join(tmp, "libnrq.so")
        shutil.copy(_lib.LIB_PATH, lib)
        subprocess.run([objdump, "--offloading", lib], cwd=tmp, check=True, capture_output=True)
        cos = glob.glob(os.path.join(tmp, "libnrq.so.*gfx950"))
        assert cos, "no gfx950 code object in libnrq.so"
        lines = []
        for co in cos:
            out = subprocess.run([objdump, "-d", co], check=True, capture_output=True, text=True).stdout
            lines += [ln.split("//")[0].strip() for ln in out.splitlines() if ln.startswith(("\t", " "))]
    ins = [ln for ln in lines if ln]
    writes = 0
    for i, ln in enumerate(ins):
        assert not re.match(r"(s_sendmsg|s_movrel|v_movrel|s_set_gpr_idx|ds_gws|buffer_load\w*.*\blds\b)", ln), ln
        if re.search(r"\bm0\b", ln):
            assert re.match(r"s_mov_b32 m0, s\d+$", ln), ln
            assert ins[i + 1].startswith("global_load_lds_dword"), (ln, ins[i + 1])
            writes += 1
    assert writes > 0
