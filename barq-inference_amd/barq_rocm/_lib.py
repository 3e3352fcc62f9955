"""ctypes binding of libbarq_rocm.so (the C ABI in include/barq_rocm.h).

This module only loads the native library and declares its prototypes.  It
never falls back to another implementation: if the library is missing or the
device is unusable the calls raise.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "lib", "libbarq_rocm.so"))

# barq_status
OK = 0
E_BACKEND = 1
E_UNSUPPORTED = 2
E_DIM = 3
E_QUANT = 4
E_INVALID = 5
E_ALLOC = 6
E_GGUF = 7
E_IO = 8
STATUS_NAMES = {
    OK: "Ok", E_BACKEND: "Backend", E_UNSUPPORTED: "Unsupported", E_DIM: "DimensionMismatch",
    E_QUANT: "Quantization", E_INVALID: "Tensor", E_ALLOC: "Allocation", E_GGUF: "InvalidGguf", E_IO: "Io",
}

# barq_type (GgufTensorType discriminants, barq_core/src/gguf.rs:117-137)
F32 = 0
F16 = 1
Q4_0 = 2
Q8_0 = 8
Q4_K = 12
Q6_K = 14
Q8_K = 15
Q4_0_BARQ = 0x10002
Q4_K_BARQ = 0x1000C   # the quant crate's own Q4_K (quant/src/q4_k.rs), not GGUF
ACT_F32 = 0
ACT_F32_Q8 = 0x20000

MEM_HOST = 0
MEM_DEVICE = 1

BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_0_BARQ: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256, Q4_K_BARQ: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q4_0_BARQ: 20, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292, Q4_K_BARQ: 136}
Q8_PARTNER = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_0_BARQ: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K}

# every symbol include/barq_rocm.h declares
EXPORTS = (
    "barq_rocm_create", "barq_rocm_destroy", "barq_rocm_last_error", "barq_rocm_set_stream",
    "barq_rocm_get_stream", "barq_rocm_synchronize", "barq_rocm_abi_version",
    "barq_rocm_block_elems", "barq_rocm_block_bytes", "barq_rocm_row_bytes",
    "barq_rocm_dequantize", "barq_rocm_get_rows", "barq_rocm_quantize_act", "barq_rocm_rms_norm",
    "barq_rocm_rms_norm_quantize", "barq_rocm_add_rms_norm_quantize", "barq_rocm_add_bias",
    "barq_rocm_matvec", "barq_rocm_matmul", "barq_rocm_swiglu", "barq_rocm_ffn",
    "barq_rocm_gemm_f32", "barq_rocm_gemv_f32", "barq_rocm_dequantize_split",
    "barq_rocm_quantized_matmul_split", "barq_rocm_quantize_q4_0_barq", "barq_rocm_quantize_q4_k_barq",
    "barq_rocm_q4_k_barq_bytes", "barq_rocm_moe_route", "barq_rocm_moe_reduce", "barq_rocm_moe_route_reduce",
    "barq_rocm_moe_ffn", "barq_rocm_gguf_open", "barq_rocm_gguf_close", "barq_rocm_gguf_info",
    "barq_rocm_gguf_tensor", "barq_rocm_gguf_find_tensor", "barq_rocm_gguf_kv_type", "barq_rocm_gguf_kv_int",
    "barq_rocm_gguf_kv_number", "barq_rocm_gguf_kv_string", "barq_rocm_cache_create", "barq_rocm_cache_get",
    "barq_rocm_cache_bytes", "barq_rocm_cache_destroy",
    "barq_rocm_rope", "barq_rocm_transpose_heads", "barq_rocm_kv_cache_create", "barq_rocm_kv_cache_append",
    "barq_rocm_kv_cache_append_rope", "barq_rocm_kv_cache_size", "barq_rocm_kv_cache_layer_len",
    "barq_rocm_kv_cache_head", "barq_rocm_kv_cache_clear", "barq_rocm_kv_cache_destroy", "barq_rocm_attention",
    "barq_rocm_kv_cache_append_rope_q", "barq_rocm_attention_q8k", "barq_rocm_matvec_group",
    "barq_rocm_qkv_append_rope", "barq_rocm_matmul_noalloc", "barq_rocm_stream_read",
)

# bytes of the fixed per-GPU scratch behind barq_rocm_matmul_noalloc
NOALLOC_SCRATCH_BYTES = 32 << 20

ROPE_INTERLEAVED = 0
ROPE_SPLIT_HALF = 1


class BarqError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {msg}")
        self.code = code


_lib = None

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64


def _declare(lib):
    P = {
        "barq_rocm_create": (_i, [_i, ctypes.POINTER(_vp)]),
        "barq_rocm_destroy": (_i, [_vp]),
        "barq_rocm_last_error": (ctypes.c_char_p, []),
        "barq_rocm_set_stream": (_i, [_vp, _vp]),
        "barq_rocm_get_stream": (_vp, [_vp]),
        "barq_rocm_synchronize": (_i, [_vp]),
        "barq_rocm_abi_version": (_i, []),
        "barq_rocm_block_elems": (_sz, [_i]),
        "barq_rocm_block_bytes": (_sz, [_i]),
        "barq_rocm_row_bytes": (_sz, [_i, _sz]),
        "barq_rocm_dequantize": (_i, [_vp, _i, _vp, _sz, _vp, _i]),
        "barq_rocm_get_rows": (_i, [_vp, _i, _vp, _sz, _sz, _vp, _sz, _vp, _i]),
        "barq_rocm_add_bias": (_i, [_vp, _vp, _vp, _sz, _sz, _i]),
        "barq_rocm_stream_read": (_i, [_vp, _vp, _sz, _vp]),
        "barq_rocm_quantize_act": (_i, [_vp, _i, _vp, _sz, _sz, _vp, _i]),
        "barq_rocm_rms_norm": (_i, [_vp, _vp, _vp, _sz, _sz, ctypes.c_float, _vp, _i]),
        "barq_rocm_rms_norm_quantize": (_i, [_vp, _i, _vp, _vp, _sz, _sz, ctypes.c_float, _vp, _i]),
        "barq_rocm_add_rms_norm_quantize": (_i, [_vp, _i, _vp, _vp, _vp, _sz, _sz, ctypes.c_float, _vp, _vp, _i]),
        "barq_rocm_matvec": (_i, [_vp, _i, _vp, _sz, _sz, _i, _vp, _vp, _i]),
        "barq_rocm_matmul": (_i, [_vp, _i, _vp, _sz, _sz, _i, _vp, _sz, _vp, _i]),
        "barq_rocm_matvec_group": (_i, [_vp, _sz, _vp, _vp, _vp, _sz, _i, _vp, _vp, _i]),
        "barq_rocm_swiglu": (_i, [_vp, _i, _vp, _vp, _sz, _sz, _vp, _i]),
        "barq_rocm_ffn": (_i, [_vp, _i, _vp, _i, _vp, _i, _vp, _sz, _sz, _i, _vp, _sz, _vp, _i]),
        "barq_rocm_gemm_f32": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _vp, _i]),
        "barq_rocm_gemv_f32": (_i, [_vp, _vp, _vp, _sz, _sz, _vp, _i]),
        "barq_rocm_dequantize_split": (_i, [_vp, _i, _vp, _sz, _vp, _sz, _sz, _vp, _sz, _i]),
        "barq_rocm_quantized_matmul_split": (_i, [_vp, _vp, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _i, _sz, _i]),
        "barq_rocm_quantize_q4_0_barq": (_i, [_vp, _vp, _sz, _vp, _i]),
        "barq_rocm_quantize_q4_k_barq": (_i, [_vp, _vp, _sz, _vp, _i]),
        "barq_rocm_q4_k_barq_bytes": (_sz, [_sz]),
        "barq_rocm_moe_route": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _i]),
        "barq_rocm_moe_reduce": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_float, _vp, _vp, _i]),
        "barq_rocm_moe_route_reduce": (_i, [_vp, _vp, _sz, _sz, _sz, _sz, ctypes.c_float, _vp, _vp, _i]),
        "barq_rocm_moe_ffn": (_i, [_vp, _sz, _i, _vp, _i, _vp, _i, _vp, _sz, _sz, _vp, _sz, _vp, _vp, _sz, _i, _vp, _i]),
        "barq_rocm_gguf_open": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
        "barq_rocm_gguf_close": (_i, [_vp]),
        "barq_rocm_gguf_info": (_i, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                                     ctypes.POINTER(_u32), ctypes.POINTER(_u64)]),
        "barq_rocm_gguf_tensor": (_i, [_vp, _u64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i),
                                       ctypes.POINTER(_u32), ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                                       ctypes.POINTER(_u64), ctypes.POINTER(_vp)]),
        "barq_rocm_gguf_find_tensor": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
        "barq_rocm_gguf_kv_type": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_i), ctypes.POINTER(_i),
                                        ctypes.POINTER(_u64)]),
        "barq_rocm_gguf_kv_int": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
        "barq_rocm_gguf_kv_number": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
        "barq_rocm_gguf_kv_string": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.POINTER(_u64)]),
        "barq_rocm_cache_create": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
        "barq_rocm_cache_get": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_i), ctypes.POINTER(_u64),
                                     ctypes.POINTER(_u64), ctypes.POINTER(_vp)]),
        "barq_rocm_cache_bytes": (_u64, [_vp]),
        "barq_rocm_cache_destroy": (_i, [_vp]),
        "barq_rocm_rope": (_i, [_vp, _vp, _sz, _sz, _sz, _sz, ctypes.c_float, _vp, _i, _vp, _i]),
        "barq_rocm_transpose_heads": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _i]),
        "barq_rocm_kv_cache_create": (_i, [_vp, _sz, _sz, _sz, _sz, ctypes.POINTER(_vp)]),
        "barq_rocm_kv_cache_append": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _i]),
        "barq_rocm_kv_cache_append_rope": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, ctypes.c_float, _vp, _i, _i]),
        "barq_rocm_kv_cache_size": (_sz, [_vp]),
        "barq_rocm_kv_cache_layer_len": (_sz, [_vp, _sz]),
        "barq_rocm_kv_cache_head": (_i, [_vp, _sz, _sz, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]),
        "barq_rocm_kv_cache_clear": (_i, [_vp]),
        "barq_rocm_kv_cache_destroy": (_i, [_vp]),
        "barq_rocm_attention": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _i]),
        "barq_rocm_attention_q8k": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _i]),
        "barq_rocm_kv_cache_append_rope_q": (_i, [_vp, _vp, _sz, _vp, _sz, _vp, _vp, _vp, _sz, _sz, ctypes.c_float,
                                                  _vp, _i, _i]),
        "barq_rocm_qkv_append_rope": (_i, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _i, _vp, _vp, _sz, ctypes.c_float, _vp,
                                           _i, _i]),
        "barq_rocm_matmul_noalloc": (_i, [_vp, _i, _vp, _sz, _sz, _i, _vp, _sz, _vp]),
    }
    for name, (res, args) in P.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """Load libbarq_rocm.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        l = ctypes.CDLL(LIB_PATH)
        _declare(l)
        _lib = l
    return _lib


def check(rc: int):
    if rc != OK:
        raise BarqError(rc, lib().barq_rocm_last_error().decode(errors="replace"))
