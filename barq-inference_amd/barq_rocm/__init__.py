"""barq_rocm — MI355X (gfx950) quantized-linear backend for barq-inference.

The compute lives in libbarq_rocm.so (hand-written HIP kernels behind the C
ABI in include/barq_rocm.h).  This package is the Python plumbing used by the
tests and the benchmark: a ctypes binding (_lib), a thin handle wrapper over
torch-allocated device buffers (backend) and the deterministic synthetic
inputs of the benchmark configurations (synth).
"""
from . import _lib
from ._lib import (ACT_F32, ACT_F32_Q8, BLOCK_BYTES, BLOCK_ELEMS, E_BACKEND, E_DIM, E_INVALID, E_QUANT,
                   E_UNSUPPORTED, F16, F32, MEM_DEVICE, MEM_HOST, NOALLOC_SCRATCH_BYTES, Q4_0, Q4_0_BARQ, Q4_K,
                   Q4_K_BARQ, Q6_K, Q8_0, Q8_K, Q8_PARTNER, BarqError)
from .backend import Backend

__all__ = [
    "_lib", "Backend", "BarqError", "ACT_F32", "ACT_F32_Q8", "BLOCK_BYTES", "BLOCK_ELEMS", "F16", "F32",
    "MEM_DEVICE", "MEM_HOST", "Q4_0", "Q4_0_BARQ", "Q4_K", "Q4_K_BARQ", "Q6_K", "Q8_0", "Q8_K", "Q8_PARTNER",
    "E_BACKEND", "E_DIM", "E_INVALID", "E_QUANT", "E_UNSUPPORTED", "NOALLOC_SCRATCH_BYTES",
]


def row_bytes(type_: int, k: int) -> int:
    return k // BLOCK_ELEMS[type_] * BLOCK_BYTES[type_]
