"""Attention plumbing over the C ABI: RoPE, the device KV cache, attention.

Mirrors the reference's attention half of a layer
(models/src/transformer.rs:176-374) and its KVCache
(models/src/context.rs:245-340) with the same names and argument meanings.
Every compute call goes through libbarq_rocm.so; device buffers are torch
tensors, host buffers numpy arrays (``mem=MEM_HOST``).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L
from .backend import Backend, _ptr

ROPE_INTERLEAVED = L.ROPE_INTERLEAVED
ROPE_SPLIT_HALF = L.ROPE_SPLIT_HALF


def _empty(shape, like, mem, dtype="float32"):
    if mem == L.MEM_HOST:
        return np.empty(shape, dtype=np.dtype(dtype))
    import torch
    return torch.empty(shape, dtype=getattr(torch, dtype), device=like.device)


def apply_rope(be: Backend, x, seq_len, n_heads, head_dim, start_pos, rope_freq_scale, rope_inv_freq, layout,
               mem=L.MEM_DEVICE, sync=True):
    """apply_rope (transformer.rs:514-562): x [seq, n_heads*head_dim] -> [n_heads, seq, head_dim]."""
    out = _empty((n_heads, seq_len, head_dim), x, mem)
    L.check(be._lib.barq_rocm_rope(be.h, _ptr(x), seq_len, n_heads, head_dim, start_pos, rope_freq_scale,
                                   _ptr(rope_inv_freq), layout, _ptr(out), mem))
    if sync and mem == L.MEM_DEVICE:
        be.sync()
    return out


def transpose_heads(be: Backend, x, seq_len, n_heads, head_dim, mem=L.MEM_DEVICE, sync=True):
    """transpose_heads (transformer.rs:598-611)."""
    out = _empty((n_heads, seq_len, head_dim), x, mem)
    L.check(be._lib.barq_rocm_transpose_heads(be.h, _ptr(x), seq_len, n_heads, head_dim, _ptr(out), mem))
    if sync and mem == L.MEM_DEVICE:
        be.sync()
    return out


class KVCache:
    """KVCache (context.rs:245-340) in device memory, preallocated for
    max_size positions per layer and kv head."""

    def __init__(self, be: Backend, max_size: int, n_layers: int, n_head_kv: int, head_dim: int):
        self.be = be
        c = ctypes.c_void_p()
        L.check(be._lib.barq_rocm_kv_cache_create(be.h, max_size, n_layers, n_head_kv, head_dim, ctypes.byref(c)))
        self.c = c
        self.max_size, self.n_layers, self.n_head_kv, self.head_dim = max_size, n_layers, n_head_kv, head_dim

    def close(self):
        if self.c:
            self.be._lib.barq_rocm_kv_cache_destroy(self.c)
            self.c = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def append(self, layer, k, v, n_tokens, head_dim, mem=L.MEM_DEVICE):
        """KVCache::append (context.rs:272-291): k, v [n_head_kv, n_tokens, head_dim]."""
        L.check(self.be._lib.barq_rocm_kv_cache_append(self.be.h, self.c, layer, _ptr(k), _ptr(v), n_tokens,
                                                        head_dim, mem))

    def append_rope(self, layer, k_proj, v_proj, n_tokens, start_pos, rope_freq_scale, rope_inv_freq, layout,
                    mem=L.MEM_DEVICE):
        """apply_rope(k) + transpose_heads(v) + append, fused
        (transformer.rs:232-245): k_proj, v_proj [n_tokens, n_head_kv*head_dim]."""
        L.check(self.be._lib.barq_rocm_kv_cache_append_rope(self.be.h, self.c, layer, _ptr(k_proj), _ptr(v_proj),
                                                             n_tokens, start_pos, rope_freq_scale,
                                                             _ptr(rope_inv_freq), layout, mem))

    def append_rope_q(self, layer, q_proj, n_head, k_proj, v_proj, n_tokens, start_pos, rope_freq_scale,
                      rope_inv_freq, layout, mem=L.MEM_DEVICE, q_out=None):
        """apply_rope(q) + apply_rope(k) + transpose_heads(v) + append in one
        launch (transformer.rs:222-245); returns q rotated [n_head, n_tokens, head_dim]."""
        if q_out is None:
            q_out = _empty((n_head, n_tokens, self.head_dim), q_proj, mem)
        L.check(self.be._lib.barq_rocm_kv_cache_append_rope_q(self.be.h, self.c, layer, _ptr(q_proj), n_head,
                                                               _ptr(q_out), _ptr(k_proj), _ptr(v_proj), n_tokens,
                                                               start_pos, rope_freq_scale, _ptr(rope_inv_freq),
                                                               layout, mem))
        return q_out

    def qkv_append_rope(self, layer, w_types, ws, n_head, k, act_type, x, start_pos, rope_freq_scale, rope_inv_freq,
                        layout, mem=L.MEM_DEVICE, q_out=None):
        """The q/k/v projections of one token, apply_rope(q), apply_rope(k)
        and the append (transformer.rs:212-245) in one call; returns q rotated
        [n_head, 1, head_dim]."""
        if q_out is None:
            q_out = _empty((n_head, 1, self.head_dim), x, mem)
        tarr = (ctypes.c_int * 3)(*w_types)
        warr = (ctypes.c_void_p * 3)(*[_ptr(w) for w in ws])
        L.check(self.be._lib.barq_rocm_qkv_append_rope(self.be.h, self.c, layer, tarr, warr, n_head, k, act_type,
                                                        _ptr(x), _ptr(q_out), start_pos, rope_freq_scale,
                                                        _ptr(rope_inv_freq), layout, mem))
        return q_out

    def size(self) -> int:
        return self.be._lib.barq_rocm_kv_cache_size(self.c)

    def layer_len(self, layer) -> int:
        return self.be._lib.barq_rocm_kv_cache_layer_len(self.c, layer)

    def head_ptrs(self, layer, head):
        """Device pointers of get_k_head / get_v_head (context.rs:316-323)."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        L.check(self.be._lib.barq_rocm_kv_cache_head(self.c, layer, head, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value

    def get_head(self, layer, head):
        """(K, V) of a head as numpy [layer_len, head_dim], copied to the host
        after the backend's stream has finished."""
        n = self.layer_len(layer)
        self.be.sync()
        out = []
        for p in self.head_ptrs(layer, head):
            a = np.empty((n, self.head_dim), dtype=np.float32)
            if n:
                rc = _hip().hipMemcpy(ctypes.c_void_p(a.ctypes.data), ctypes.c_void_p(p), a.nbytes, 2)
                if rc != 0:
                    raise RuntimeError(f"hipMemcpy (device to host) failed: {rc}")
            out.append(a)
        return tuple(out)

    def clear(self):
        L.check(self.be._lib.barq_rocm_kv_cache_clear(self.c))


_hip_lib = None


def _hip():
    global _hip_lib
    if _hip_lib is None:
        _hip_lib = ctypes.CDLL("libamdhip64.so")
        _hip_lib.hipMemcpy.restype = ctypes.c_int
        _hip_lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _hip_lib


def compute_attention(be: Backend, q, cache: KVCache, layer, n_head, n_head_kv, head_dim, q_len, kv_len, start_pos,
                      mem=L.MEM_DEVICE, sync=True):
    """compute_attention (transformer.rs:301-374): q [n_head, q_len, head_dim] -> [q_len, n_head, head_dim]."""
    out = _empty((q_len, n_head, head_dim), q, mem)
    L.check(be._lib.barq_rocm_attention(be.h, _ptr(q), cache.c, layer, n_head, n_head_kv, head_dim, q_len, kv_len,
                                        start_pos, _ptr(out), mem))
    if sync and mem == L.MEM_DEVICE:
        be.sync()
    return out


def compute_attention_q8k(be: Backend, q, cache: KVCache, layer, n_head, n_head_kv, head_dim, q_len, kv_len,
                          start_pos, mem=L.MEM_DEVICE, sync=True, out=None):
    """compute_attention, then the Q8_K quantizer of its rows (the o
    projection's input): uint8 [q_len, n_head*head_dim/256 * 292]."""
    nb = n_head * head_dim // 256
    if out is None:
        out = _empty((q_len, nb * 292), q, mem, dtype="uint8")
    L.check(be._lib.barq_rocm_attention_q8k(be.h, _ptr(q), cache.c, layer, n_head, n_head_kv, head_dim, q_len,
                                            kv_len, start_pos, _ptr(out), mem))
    if sync and mem == L.MEM_DEVICE:
        be.sync()
    return out
