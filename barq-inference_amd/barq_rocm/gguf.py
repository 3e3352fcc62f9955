"""Python view of the packed GGUF loader and device weight cache of
libbarq_rocm (barq_rocm_gguf_* / barq_rocm_cache_*)."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L


class GgufFile:
    """A memory-mapped GGUF file read by the library (GgufReader analogue)."""

    def __init__(self, path: str):
        self._lib = L.lib()
        g = ctypes.c_void_p()
        L.check(self._lib.barq_rocm_gguf_open(path.encode(), ctypes.byref(g)))
        self.g = g

    def close(self):
        if self.g:
            self._lib.barq_rocm_gguf_close(self.g)
            self.g = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> dict:
        v, a = ctypes.c_uint32(), ctypes.c_uint32()
        nt, nk, off = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        L.check(self._lib.barq_rocm_gguf_info(self.g, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk),
                                              ctypes.byref(a), ctypes.byref(off)))
        return dict(version=v.value, n_tensors=nt.value, n_kv=nk.value, alignment=a.value, data_offset=off.value)

    def tensor(self, index: int) -> dict:
        name = ctypes.c_char_p()
        t, nd = ctypes.c_int(), ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        data = ctypes.c_void_p()
        L.check(self._lib.barq_rocm_gguf_tensor(self.g, index, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd),
                                                dims, ctypes.byref(off), ctypes.byref(nb), ctypes.byref(data)))
        raw = None
        if nb.value:
            raw = np.ctypeslib.as_array((ctypes.c_uint8 * nb.value).from_address(data.value)).copy()
        return dict(name=name.value.decode(), type=t.value, n_dims=nd.value, dims=list(dims), offset=off.value,
                    nbytes=nb.value, data=raw)

    def find(self, name: str) -> int:
        i = ctypes.c_uint64()
        L.check(self._lib.barq_rocm_gguf_find_tensor(self.g, name.encode(), ctypes.byref(i)))
        return i.value

    def kv_type(self, key: str):
        t, at, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        L.check(self._lib.barq_rocm_gguf_kv_type(self.g, key.encode(), ctypes.byref(t), ctypes.byref(at),
                                                 ctypes.byref(n)))
        return t.value, at.value, n.value

    def kv_int(self, key: str) -> int:
        v = ctypes.c_int64()
        L.check(self._lib.barq_rocm_gguf_kv_int(self.g, key.encode(), ctypes.byref(v)))
        return v.value

    def kv_number(self, key: str) -> float:
        v = ctypes.c_double()
        L.check(self._lib.barq_rocm_gguf_kv_number(self.g, key.encode(), ctypes.byref(v)))
        return v.value

    def kv_string(self, key: str) -> str:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        L.check(self._lib.barq_rocm_gguf_kv_string(self.g, key.encode(), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""


class WeightCache:
    """Packed device copies of a GGUF file's tensors (WeightCache analogue)."""

    def __init__(self, backend, gguf: GgufFile):
        self._lib = L.lib()
        c = ctypes.c_void_p()
        L.check(self._lib.barq_rocm_cache_create(backend.h, gguf.g, ctypes.byref(c)))
        self.c = c

    def get(self, name: str):
        """(type, n_rows, k, device pointer) of a cached tensor."""
        t, n, k, p = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_void_p()
        L.check(self._lib.barq_rocm_cache_get(self.c, name.encode(), ctypes.byref(t), ctypes.byref(n),
                                              ctypes.byref(k), ctypes.byref(p)))
        return t.value, n.value, k.value, p.value

    def find(self, name: str):
        """get(name), or None when the file has no such tensor."""
        t, n, k, p = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_void_p()
        rc = self._lib.barq_rocm_cache_get(self.c, name.encode(), ctypes.byref(t), ctypes.byref(n),
                                           ctypes.byref(k), ctypes.byref(p))
        if rc != L.OK:
            return None
        return t.value, n.value, k.value, p.value

    def nbytes(self) -> int:
        return self._lib.barq_rocm_cache_bytes(self.c)

    def close(self):
        if self.c:
            self._lib.barq_rocm_cache_destroy(self.c)
            self.c = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
