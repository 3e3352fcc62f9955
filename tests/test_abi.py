"""The C ABI loads and exports everything include/barq_rocm.h declares, and
its host-side logic (geometry, argument checks, status codes) behaves like
the reference's error conventions — without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "barq_rocm.h")


@pytest.fixture(scope="module")
def L():
    from barq_rocm import _lib
    _lib.lib()
    return _lib


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(barq_rocm_\w+)\s*\(", text)))


def test_header_declares_what_the_binding_declares(L):
    assert declared_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol(L):
    lib = ctypes.CDLL(L.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version(L):
    assert L.lib().barq_rocm_abi_version() == 1


def test_block_geometry_matches_gguf(L):
    lib = L.lib()
    # gguf.rs:168-186 block sizes, block bytes of gguf.rs:529-530,645,747,854
    for t, e, b in [(L.Q4_0, 32, 18), (L.Q4_0_BARQ, 32, 20), (L.Q8_0, 32, 34), (L.Q4_K, 256, 144),
                    (L.Q6_K, 256, 210), (L.Q8_K, 256, 292), (L.F16, 1, 2), (L.F32, 1, 4)]:
        assert lib.barq_rocm_block_elems(t) == e
        assert lib.barq_rocm_block_bytes(t) == b
    assert lib.barq_rocm_row_bytes(L.Q4_K, 4096) == 16 * 144
    assert lib.barq_rocm_row_bytes(L.Q6_K, 4096) == 16 * 210
    assert lib.barq_rocm_row_bytes(L.Q4_K, 100) == 0
    assert lib.barq_rocm_block_elems(999) == 0


def status(L, rc):
    return rc, L.lib().barq_rocm_last_error().decode()


def test_argument_errors_map_to_reference_error_variants(L):
    lib = L.lib()
    x = np.zeros(4096, np.float32)
    y = np.zeros(16, np.float32)
    w = np.zeros(16 * 144 * 16, np.uint8)
    # k not a whole number of blocks -> Error::Quantization
    rc, msg = status(L, lib.barq_rocm_matvec(None, L.Q4_K, w.ctypes.data, 16, 100, L.ACT_F32, x.ctypes.data,
                                             y.ctypes.data, L.MEM_HOST))
    assert rc == L.E_QUANT and "multiple" in msg
    # unknown weight type -> Error::Unsupported
    rc, _ = status(L, lib.barq_rocm_matvec(None, 13, w.ctypes.data, 16, 256, L.ACT_F32, x.ctypes.data,
                                           y.ctypes.data, L.MEM_HOST))
    assert rc == L.E_UNSUPPORTED
    # wrong activation partner -> Unsupported
    rc, msg = status(L, lib.barq_rocm_matvec(None, L.Q4_K, w.ctypes.data, 16, 256, L.Q8_0, x.ctypes.data,
                                             y.ctypes.data, L.MEM_HOST))
    assert rc == L.E_UNSUPPORTED and "pairs with" in msg
    # null buffers -> Error::Tensor
    rc, _ = status(L, lib.barq_rocm_matvec(None, L.Q4_K, None, 16, 256, L.ACT_F32, x.ctypes.data,
                                           y.ctypes.data, L.MEM_HOST))
    assert rc == L.E_INVALID
    # bad memory kind
    rc, _ = status(L, lib.barq_rocm_matvec(None, L.Q4_K, w.ctypes.data, 16, 256, L.ACT_F32, x.ctypes.data,
                                           y.ctypes.data, 7))
    assert rc == L.E_INVALID
    # valid arguments, no handle -> Error::Tensor("null handle")
    rc, msg = status(L, lib.barq_rocm_matvec(None, L.Q4_K, w.ctypes.data, 16, 256, L.ACT_F32, x.ctypes.data,
                                             y.ctypes.data, L.MEM_HOST))
    assert rc == L.E_INVALID and "handle" in msg
    # empty problems succeed without touching anything
    assert lib.barq_rocm_matvec(None, L.Q4_K, None, 0, 256, L.ACT_F32, None, None, L.MEM_HOST) == L.OK
    # dequantize of a partial block
    rc, _ = status(L, lib.barq_rocm_dequantize(None, L.Q4_K, w.ctypes.data, 100, y.ctypes.data, L.MEM_HOST))
    assert rc == L.E_QUANT
    # MoE: no experts -> the reference's "At least one expert function is required"
    rc, msg = status(L, lib.barq_rocm_moe_ffn(None, 0, L.Q4_K, None, L.Q4_K, None, L.Q6_K, None, 256, 256, None, 1,
                                              None, None, 1, L.ACT_F32, None, L.MEM_HOST))
    assert rc == L.E_INVALID and "expert" in msg
    rc, msg = status(L, lib.barq_rocm_moe_route(None, x.ctypes.data, 1, 0, 2, None, None, L.MEM_HOST))
    assert rc == L.E_INVALID and "at least one expert" in msg


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a ROCm device is visible")
def test_create_without_device_is_unsupported(L):
    # CudaBackend::new maps a missing device to Error::Unsupported
    # (backend/src/cuda.rs:64-77) so callers fall back to the CPU chain.
    h = ctypes.c_void_p()
    rc, msg = status(L, L.lib().barq_rocm_create(0, ctypes.byref(h)))
    assert rc == L.E_UNSUPPORTED and not h.value
    assert msg
