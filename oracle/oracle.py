"""ctypes binding of the CPU oracle (oracle/_build/libbarq_oracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker for libbarq_rocm and the timed
CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module.  Every function restates the
reference (see the citations in barq_oracle.c).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libbarq_oracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, Q4_0_BARQ = 0, 1, 2, 8, 12, 14, 15, 0x10002

_lib = None
_vp, _sz, _i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        l = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_block_elems": (_sz, [_i]),
            "orc_block_bytes": (_sz, [_i]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_dequantize": (_sz, [_i, _vp, _sz, _vp]),
            "orc_get_scale_min_k4": (None, [_i, _vp, _vp, _vp]),
            "orc_pack_scale_min_k4": (None, [_vp, _vp, _vp]),
            "orc_q4_0_gguf_to_barq": (None, [_vp, _sz, _vp]),
            "orc_quantize_q8_0": (None, [_vp, _sz, _vp]),
            "orc_quantize_q8_k": (None, [_vp, _sz, _vp]),
            "orc_gemv_f32": (None, [_vp, _vp, _sz, _sz, _vp]),
            "orc_rms_norm": (None, [_vp, _vp, _sz, _sz, ctypes.c_float, _vp]),
            "orc_gemm_f32": (None, [_vp, _vp, _sz, _sz, _sz, _vp]),
            "orc_matvec": (_i, [_i, _vp, _sz, _sz, _i, _vp, _vp]),
            "orc_matmul": (_i, [_i, _vp, _sz, _sz, _i, _vp, _sz, _vp]),
            "orc_q4_0_quantize_barq": (_sz, [_vp, _sz, _vp]),
            "orc_dequantize_packed_4bit_split": (None, [_vp, _sz, _vp, _sz, _sz, _vp, _sz]),
            "orc_dequantize_signed_8bit_split": (None, [_vp, _sz, _vp, _sz, _sz, _vp, _sz]),
            "orc_quantized_matmul_split": (None, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _i, _sz, _vp]),
            "orc_moe_select_top_k": (_sz, [_vp, _sz, _sz, _sz, _vp, _vp]),
            "orc_moe_reduce_experts": (None, [_vp, _vp, _sz, _sz, _sz, ctypes.c_float, _vp, _vp]),
            "orc_moe_batch_by_expert": (None, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp]),
            "orc_moe_dispatch": (_i, [_vp, _sz, _sz, _sz, _vp, _vp, _sz, _vp, _vp, _vp]),
            "orc_moe_ffn": (_i, [_i, _vp, _i, _vp, _i, _vp, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _sz, _i, _vp]),
            "orc_ffn_swiglu": (None, [_vp, _vp, _sz, _vp]),
            "orc_ffn": (_i, [_i, _vp, _i, _vp, _i, _vp, _sz, _sz, _i, _vp, _sz, _vp]),
            "orc_q4_k_barq_quantize": (_sz, [_vp, _sz, _vp]),
            "orc_q4_k_barq_dequantize": (_sz, [_vp, _sz, _sz, _vp]),
            "orc_rope": (None, [_vp, _sz, _sz, _sz, _sz, ctypes.c_float, _vp, _i, _vp]),
            "orc_transpose_heads": (None, [_vp, _sz, _sz, _sz, _vp]),
            "orc_attention": (None, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp]),
            "cpub_gemm_literal_m1": (None, [_vp, _vp, _sz, _sz, _sz, _sz, _vp]),
            "cpub_gemv_simd": (None, [_vp, _vp, _sz, _sz, _sz, _vp]),
            "cpub_gemv_simd_threaded": (_i, [_vp, _vp, _sz, _sz, _sz, _vp, _i]),
            "cpub_simd_level": (_i, []),
            "cpub_gemm_rows": (None, [_vp, _vp, _sz, _sz, _sz, _sz, _vp]),
            "cpub_gemm_rows_threaded": (_i, [_vp, _vp, _sz, _sz, _sz, _sz, _vp, _i]),
            "cpub_moe_expert_ffn": (None, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def block_elems(t):
    return lib().orc_block_elems(t)


def block_bytes(t):
    return lib().orc_block_bytes(t)


def row_bytes(t, k):
    return k // block_elems(t) * block_bytes(t)


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def f32_to_f16(v: float) -> int:
    return lib().orc_f32_to_f16(v)


def dequantize(t: int, blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    r = lib().orc_dequantize(t, _p(blocks), n, _p(out))
    if r == ctypes.c_size_t(-1).value:
        raise ValueError(f"unsupported type {t}")
    return out


def get_scale_min_k4(j: int, q: np.ndarray):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    sc, m = ctypes.c_uint8(), ctypes.c_uint8()
    lib().orc_get_scale_min_k4(j, _p(q), ctypes.addressof(sc), ctypes.addressof(m))
    return sc.value, m.value


def pack_scale_min_k4(ls, lm) -> np.ndarray:
    ls = np.ascontiguousarray(ls, dtype=np.uint8)
    lm = np.ascontiguousarray(lm, dtype=np.uint8)
    out = np.empty(12, dtype=np.uint8)
    lib().orc_pack_scale_min_k4(_p(ls), _p(lm), _p(out))
    return out


def q4_0_gguf_to_barq(gguf: np.ndarray) -> np.ndarray:
    gguf = np.ascontiguousarray(gguf, dtype=np.uint8)
    nb = gguf.size // 18
    out = np.empty(nb * 20, dtype=np.uint8)
    lib().orc_q4_0_gguf_to_barq(_p(gguf), nb, _p(out))
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib().orc_quantize_q8_0(_p(x), x.size, _p(out))
    return out


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // 256 * 292, dtype=np.uint8)
    lib().orc_quantize_q8_k(_p(x), x.size, _p(out))
    return out


def quantize_act(act_type: int, x: np.ndarray) -> np.ndarray:
    return quantize_q8_0(x) if act_type == Q8_0 else quantize_q8_k(x)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """transformer.rs:148-172 on each row of x ([rows, n])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, n = (1, x.size) if x.ndim == 1 else x.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty((rows, n), dtype=np.float32)
    lib().orc_rms_norm(_p(x), _p(w), rows, n, eps, _p(y))
    return y


def q4_k_barq_quantize(x: np.ndarray) -> np.ndarray:
    """quant::Q4_K::quantize (quant/src/q4_k.rs:23-73)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    n = x.size
    out = np.zeros(n // 256 * 136 + (8 + (n % 256 + 1) // 2 if n % 256 else 0), dtype=np.uint8)
    got = lib().orc_q4_k_barq_quantize(_p(x), n, _p(out))
    assert got == out.size
    return out


def q4_k_barq_dequantize(data: np.ndarray, output_size: int) -> np.ndarray:
    """quant::Q4_K::dequantize (quant/src/q4_k.rs:75-133); may return fewer
    than output_size values, as the reference does."""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.zeros(max(output_size, 1), dtype=np.float32)
    w = lib().orc_q4_k_barq_dequantize(_p(data), data.size, output_size, _p(out))
    return out[:w]


def rope(x: np.ndarray, seq: int, heads: int, hd: int, start_pos: int, freq_scale: float, inv_freq: np.ndarray,
         layout: int) -> np.ndarray:
    """apply_rope (transformer.rs:514-562): [seq, heads*hd] -> [heads, seq, hd]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = np.ascontiguousarray(inv_freq, dtype=np.float32)
    out = np.empty((heads, seq, hd), dtype=np.float32)
    lib().orc_rope(_p(x), seq, heads, hd, start_pos, freq_scale, _p(f), layout, _p(out))
    return out


def transpose_heads(x: np.ndarray, seq: int, heads: int, hd: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((heads, seq, hd), dtype=np.float32)
    lib().orc_transpose_heads(_p(x), seq, heads, hd, _p(out))
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_head: int, q_len: int, kv_len: int,
              start_pos: int) -> np.ndarray:
    """compute_attention (transformer.rs:301-374).  q [n_head, q_len, hd];
    k, v [n_head_kv, positions >= kv_len, hd]; returns [q_len, n_head, hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n_head_kv, pos, hd = k.shape
    assert v.shape == k.shape and q.shape == (n_head, q_len, hd) and kv_len <= pos
    out = np.empty((q_len, n_head, hd), dtype=np.float32)
    lib().orc_attention(_p(q), _p(k), _p(v), pos * hd, n_head, n_head_kv, hd, q_len, kv_len, start_pos, _p(out))
    return out


def gemv_f32(a: np.ndarray, x: np.ndarray, m: int, n: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(m, dtype=np.float32)
    lib().orc_gemv_f32(_p(a), _p(x), m, n, _p(y))
    return y


def gemm_f32(a: np.ndarray, b: np.ndarray, m: int, k: int, n: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_gemm_f32(_p(a), _p(b), m, k, n, _p(c))
    return c


def matmul(w_type: int, w: np.ndarray, n_rows: int, k: int, act_type: int, x: np.ndarray, m: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x)
    y = np.empty((m, n_rows), dtype=np.float32)
    rc = lib().orc_matmul(w_type, _p(w), n_rows, k, act_type, _p(x), m, _p(y))
    if rc:
        raise ValueError("orc_matmul: bad type or shape")
    return y


def matvec(w_type, w, n_rows, k, act_type, x) -> np.ndarray:
    return matmul(w_type, w, n_rows, k, act_type, x, 1)[0]


def q4_0_quantize_barq(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = (x.size + 31) // 32
    out = np.zeros(nb * 20, dtype=np.uint8)
    n = lib().orc_q4_0_quantize_barq(_p(x), x.size, _p(out))
    return out[:n]


def dequantize_split(kind_q8_0: bool, quants, scales, block_size, n_out) -> np.ndarray:
    quants = np.ascontiguousarray(quants, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    out = np.zeros(n_out, dtype=np.float32)
    f = lib().orc_dequantize_signed_8bit_split if kind_q8_0 else lib().orc_dequantize_packed_4bit_split
    f(_p(quants), quants.size, _p(scales), scales.size, block_size, _p(out), n_out)
    return out


def quantized_matmul_split(a, bq, bs, m, n, k, kind_q8_0: bool, block_size) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    bq = np.ascontiguousarray(bq, dtype=np.uint8)
    bs = np.ascontiguousarray(bs, dtype=np.float32)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_quantized_matmul_split(_p(a), _p(bq), bq.size, _p(bs), bs.size, m, n, k, int(kind_q8_0), block_size, _p(c))
    return c


def moe_select_top_k(logits: np.ndarray, k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows, cols = logits.shape
    kk = max(1, min(k, cols))
    ids = np.empty((rows, kk), dtype=np.int32)
    w = np.empty((rows, kk), dtype=np.float32)
    got = lib().orc_moe_select_top_k(_p(logits), rows, cols, k, _p(ids), _p(w))
    assert got == kk
    return ids, w


def moe_reduce_experts(ids: np.ndarray, weights: np.ndarray, max_active: int, min_weight: float):
    """reduce_expert_assignments (moe_fused.rs:147-194) on rows x k slots
    (id < 0: absent); kept assignments first, then -1 / 0."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    rows, k = ids.shape
    oi = np.empty_like(ids)
    ow = np.empty_like(weights)
    lib().orc_moe_reduce_experts(_p(ids), _p(weights), rows, k, max_active, ctypes.c_float(min_weight), _p(oi), _p(ow))
    return oi, ow


def moe_batch_by_expert(ids: np.ndarray, weights: np.ndarray, n_experts: int):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    rows, k = ids.shape
    off = np.empty(n_experts + 1, dtype=np.int32)
    tok = np.full(rows * k, -1, dtype=np.int32)
    wts = np.zeros(rows * k, dtype=np.float32)
    lib().orc_moe_batch_by_expert(_p(ids), _p(weights), rows, k, n_experts, _p(off), _p(tok), _p(wts))
    return off, tok[: off[-1]], wts[: off[-1]]


EXPERT_FN = ctypes.CFUNCTYPE(_i, _i, ctypes.POINTER(ctypes.c_float), _sz, _sz, ctypes.POINTER(ctypes.c_float), _vp)


def moe_dispatch(x: np.ndarray, n_experts: int, ids: np.ndarray, weights: np.ndarray, expert_fns) -> np.ndarray:
    """dispatch_experts with Python expert closures f(batch [rows x hidden]) -> [rows x hidden]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    rows, hidden = x.shape

    def tramp(e, inp, r, h, outp, ctx):
        a = np.ctypeslib.as_array(inp, shape=(r, h)).copy()
        res = np.asarray(expert_fns[e](a), dtype=np.float32)
        np.ctypeslib.as_array(outp, shape=(r, h))[:] = res
        return 0

    cb = EXPERT_FN(tramp)
    out = np.empty((rows, hidden), dtype=np.float32)
    rc = lib().orc_moe_dispatch(_p(x), rows, hidden, n_experts, _p(ids), _p(weights), ids.shape[1],
                                ctypes.cast(cb, _vp), None, _p(out))
    if rc:
        raise ValueError("orc_moe_dispatch failed")
    return out


def moe_ffn(gate_type, gates, up_type, ups, down_type, downs, hidden, n_ff, x, ids, weights, act) -> np.ndarray:
    ne = len(gates)
    arr = _vp * ne
    gates = [np.ascontiguousarray(g, dtype=np.uint8) for g in gates]
    ups = [np.ascontiguousarray(g, dtype=np.uint8) for g in ups]
    downs = [np.ascontiguousarray(g, dtype=np.uint8) for g in downs]
    g = arr(*[_p(t) for t in gates])
    u = arr(*[_p(t) for t in ups])
    d = arr(*[_p(t) for t in downs])
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    rows = x.shape[0]
    out = np.empty((rows, hidden), dtype=np.float32)
    rc = lib().orc_moe_ffn(gate_type, g, up_type, u, down_type, d, ne, hidden, n_ff, _p(x), rows, _p(ids),
                           _p(weights), ids.shape[1], act, _p(out))
    if rc:
        raise ValueError("orc_moe_ffn failed")
    return out


def ffn_swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """transformer.rs:394-399 elementwise."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(g)
    lib().orc_ffn_swiglu(_p(g), _p(u), g.size, _p(h))
    return h


def ffn(gate_type, gate, up_type, up, down_type, down, n_embd, n_ff, act, x, m) -> np.ndarray:
    """feed_forward (transformer.rs:378-408): act F32 (x f32) or Q8_K / Q8_0
    (x quantized rows)."""
    gate = np.ascontiguousarray(gate, dtype=np.uint8)
    up = np.ascontiguousarray(up, dtype=np.uint8)
    down = np.ascontiguousarray(down, dtype=np.uint8)
    x = np.ascontiguousarray(x)
    out = np.empty((m, n_embd), dtype=np.float32)
    rc = lib().orc_ffn(gate_type, _p(gate), up_type, _p(up), down_type, _p(down), n_embd, n_ff, act, _p(x), m, _p(out))
    if rc:
        raise ValueError("orc_ffn failed")
    return out


# ---- CPU baseline variants (bench.py's cpu_baseline leg) -----------------
def cpub_gemm_literal_m1(x, w_t, k, n, j0, j1, y):
    lib().cpub_gemm_literal_m1(_p(x), _p(w_t), k, n, j0, j1, _p(y))


def cpub_gemv_simd(a, x, n, r0, r1, y):
    lib().cpub_gemv_simd(_p(a), _p(x), n, r0, r1, _p(y))


def cpub_gemv_simd_threaded(a, x, n, r0, r1, y, threads) -> int:
    return lib().cpub_gemv_simd_threaded(_p(a), _p(x), n, r0, r1, _p(y), threads)


def cpub_gemm_rows(a, b, k, n, i0, i1, c):
    """gemm_f32's per-row loop (blas.rs:202-210) for rows [i0, i1), one thread."""
    lib().cpub_gemm_rows(_p(a), _p(b), k, n, i0, i1, _p(c))


def cpub_gemm_rows_threaded(a, b, k, n, i0, i1, c, threads) -> int:
    """The same rows split over threads (rayon over rows of C)."""
    return lib().cpub_gemm_rows_threaded(_p(a), _p(b), k, n, i0, i1, _p(c), threads)


def cpub_moe_expert_ffn(x, t, hidden, n_ff, gt, ut, dt, g, u, out):
    """fused_ffn of one expert on t rows over f32 transposed weights."""
    lib().cpub_moe_expert_ffn(_p(x), t, hidden, n_ff, _p(gt), _p(ut), _p(dt), _p(g), _p(u), _p(out))


def cpub_simd_level() -> int:
    return lib().cpub_simd_level()
