"""Python plumbing over the C ABI for tests and the benchmark.

Device buffers are torch tensors (PyTorch is only the allocator and stream
provider here); every compute call goes through libbarq_rocm.so.  Calls on
device buffers are enqueued on the backend's HIP stream; the helpers that
return tensors wait for it unless ``sync=False``.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L


def _ptr(t) -> int:
    if t is None:
        return 0
    if isinstance(t, int):   # a raw device pointer (e.g. from the weight cache)
        return t
    if isinstance(t, np.ndarray):
        return t.ctypes.data
    return t.data_ptr()


class Backend:
    """One libbarq_rocm handle bound to a device (CudaBackend::new analogue)."""

    def __init__(self, device: int = 0):
        self._lib = L.lib()
        h = ctypes.c_void_p()
        L.check(self._lib.barq_rocm_create(device, ctypes.byref(h)))
        self.h = h
        self.device = device

    def close(self):
        if self.h:
            self._lib.barq_rocm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- streams ---------------------------------------------------------
    def set_stream(self, stream_handle: int | None):
        L.check(self._lib.barq_rocm_set_stream(self.h, stream_handle or None))

    def sync(self):
        L.check(self._lib.barq_rocm_synchronize(self.h))

    # ---- raw calls (pointers) -------------------------------------------
    def dequantize_raw(self, type_, blocks, n, out, mem):
        L.check(self._lib.barq_rocm_dequantize(self.h, type_, _ptr(blocks), n, _ptr(out), mem))

    def quantize_act_raw(self, act_type, x, rows, k, out, mem):
        L.check(self._lib.barq_rocm_quantize_act(self.h, act_type, _ptr(x), rows, k, _ptr(out), mem))

    def rms_norm_raw(self, x, weight, rows, n, eps, y, mem):
        L.check(self._lib.barq_rocm_rms_norm(self.h, _ptr(x), _ptr(weight), rows, n, eps, _ptr(y), mem))

    def rms_norm_quantize_raw(self, act_type, x, weight, rows, n, eps, out, mem):
        L.check(self._lib.barq_rocm_rms_norm_quantize(self.h, act_type, _ptr(x), _ptr(weight), rows, n, eps,
                                                      _ptr(out), mem))

    def matvec_raw(self, w_type, w, n_rows, k, act_type, x, y, mem):
        L.check(self._lib.barq_rocm_matvec(self.h, w_type, _ptr(w), n_rows, k, act_type, _ptr(x), _ptr(y), mem))

    def matmul_raw(self, w_type, w, n_rows, k, act_type, x, m, y, mem):
        L.check(self._lib.barq_rocm_matmul(self.h, w_type, _ptr(w), n_rows, k, act_type, _ptr(x), m, _ptr(y), mem))

    def matvec_group_raw(self, w_types, ws, n_rows, k, act_type, x, ys, mem):
        """barq_rocm_matvec_group: ys[i] = ws[i] . x for every matrix (one launch where supported)."""
        n = len(ws)
        tarr = (ctypes.c_int * n)(*w_types)
        warr = (ctypes.c_void_p * n)(*[_ptr(w) for w in ws])
        rarr = (ctypes.c_size_t * n)(*n_rows)
        yarr = (ctypes.c_void_p * n)(*[_ptr(y) for y in ys])
        L.check(self._lib.barq_rocm_matvec_group(self.h, n, tarr, warr, rarr, k, act_type, _ptr(x), yarr, mem))

    def matmul_noalloc_raw(self, w_type, w, n_rows, k, act_type, x, m, y):
        """barq_rocm_matmul_noalloc: device buffers, the fixed per-GPU scratch."""
        L.check(self._lib.barq_rocm_matmul_noalloc(self.h, w_type, _ptr(w), n_rows, k, act_type, _ptr(x), m, _ptr(y)))

    # ---- torch-tensor conveniences (device memory) ----------------------
    def dequantize(self, type_, blocks, n, sync=True):
        import torch
        out = torch.empty(n, dtype=torch.float32, device=blocks.device)
        self.dequantize_raw(type_, blocks, n, out, L.MEM_DEVICE)
        if sync:
            self.sync()
        return out

    def get_rows(self, type_, table, n_rows, k, tokens, mem=L.MEM_DEVICE, sync=True, out=None):
        """get_embeddings (transformer.rs:96-119): the decoded rows `tokens` of
        an n_rows x k table; out-of-range ids give zero rows."""
        n = len(tokens)
        if out is None:
            if mem == L.MEM_HOST:
                out = np.empty((n, k), np.float32)
            else:
                import torch
                out = torch.empty((n, k), dtype=torch.float32, device=tokens.device)
        L.check(self._lib.barq_rocm_get_rows(self.h, type_, _ptr(table), n_rows, k, _ptr(tokens), n, _ptr(out), mem))
        if sync and mem == L.MEM_DEVICE:
            self.sync()
        return out

    def add_bias(self, y, bias, rows, dim, mem=L.MEM_DEVICE, sync=True):
        """add_bias (transformer.rs:444-465): y[r, j] += bias[j] in place."""
        L.check(self._lib.barq_rocm_add_bias(self.h, _ptr(y), _ptr(bias), rows, dim, mem))
        if sync and mem == L.MEM_DEVICE:
            self.sync()
        return y

    def quantize_act(self, act_type, x, sync=True):
        import torch
        rows, k = (1, x.numel()) if x.dim() == 1 else tuple(x.shape)
        nbytes = rows * (k // L.BLOCK_ELEMS[act_type]) * L.BLOCK_BYTES[act_type]
        out = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        self.quantize_act_raw(act_type, x, rows, k, out, L.MEM_DEVICE)
        if sync:
            self.sync()
        return out

    def rms_norm(self, x, weight, eps, mem=L.MEM_DEVICE, sync=True):
        """RMSNorm of each row of x ([rows, n]); numpy arrays with mem=MEM_HOST."""
        rows, n = (1, x.size if mem == L.MEM_HOST else x.numel()) if x.ndim == 1 else tuple(x.shape)
        if mem == L.MEM_HOST:
            y = np.empty((rows, n), dtype=np.float32)
        else:
            import torch
            y = torch.empty((rows, n), dtype=torch.float32, device=x.device)
        self.rms_norm_raw(x, weight, rows, n, eps, y, mem)
        if sync and mem == L.MEM_DEVICE:
            self.sync()
        return y

    def rms_norm_quantize(self, act_type, x, weight, eps, mem=L.MEM_DEVICE, sync=True):
        rows, n = (1, x.size if mem == L.MEM_HOST else x.numel()) if x.ndim == 1 else tuple(x.shape)
        nbytes = rows * (n // L.BLOCK_ELEMS[act_type]) * L.BLOCK_BYTES[act_type]
        if mem == L.MEM_HOST:
            out = np.empty(nbytes, dtype=np.uint8)
        else:
            import torch
            out = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        self.rms_norm_quantize_raw(act_type, x, weight, rows, n, eps, out, mem)
        if sync and mem == L.MEM_DEVICE:
            self.sync()
        return out

    def add_rms_norm_quantize(self, out_type, x, d, weight, eps, sum_out=None, out=None, mem=L.MEM_DEVICE,
                              sync=True):
        """rms_norm(x + d) as out_type (F32 rows or Q8 blocks); x + d to sum_out."""
        rows, n = (1, x.size if mem == L.MEM_HOST else x.numel()) if x.ndim == 1 else tuple(x.shape)
        if out is None:
            nbytes = rows * (n * 4 if out_type == L.F32 else n // L.BLOCK_ELEMS[out_type] * L.BLOCK_BYTES[out_type])
            if mem == L.MEM_HOST:
                out = np.empty((rows, n), np.float32) if out_type == L.F32 else np.empty(nbytes, np.uint8)
            else:
                import torch
                out = (torch.empty((rows, n), dtype=torch.float32, device=x.device) if out_type == L.F32
                       else torch.empty(nbytes, dtype=torch.uint8, device=x.device))
        L.check(self._lib.barq_rocm_add_rms_norm_quantize(self.h, out_type, _ptr(x), _ptr(d), _ptr(weight), rows, n,
                                                          eps, _ptr(sum_out), _ptr(out), mem))
        if sync and mem == L.MEM_DEVICE:
            self.sync()
        return out

    def matvec(self, w_type, w, n_rows, k, act_type, x, sync=True):
        import torch
        y = torch.empty(n_rows, dtype=torch.float32, device=w.device)
        self.matvec_raw(w_type, w, n_rows, k, act_type, x, y, L.MEM_DEVICE)
        if sync:
            self.sync()
        return y

    def matmul(self, w_type, w, n_rows, k, act_type, x, m, sync=True):
        import torch
        y = torch.empty((m, n_rows), dtype=torch.float32, device=w.device)
        self.matmul_raw(w_type, w, n_rows, k, act_type, x, m, y, L.MEM_DEVICE)
        if sync:
            self.sync()
        return y

    def swiglu(self, out_type, gate, up, mem=L.MEM_DEVICE, sync=True):
        """The dense FFN's SwiGLU (transformer.rs:394-399) of gate/up [rows, n]:
        f32 h (out_type F32) or its Q8_K / Q8_0 blocks."""
        rows, n = tuple(gate.shape)
        nbytes = rows * (n * 4 if out_type == L.F32 else n // L.BLOCK_ELEMS[out_type] * L.BLOCK_BYTES[out_type])
        if mem == L.MEM_HOST:
            out = np.empty((rows, n), np.float32) if out_type == L.F32 else np.empty(nbytes, np.uint8)
        else:
            import torch
            out = (torch.empty((rows, n), dtype=torch.float32, device=gate.device) if out_type == L.F32
                   else torch.empty(nbytes, dtype=torch.uint8, device=gate.device))
        L.check(self._lib.barq_rocm_swiglu(self.h, out_type, _ptr(gate), _ptr(up), rows, n, _ptr(out), mem))
        if mem == L.MEM_DEVICE and sync:
            self.sync()
        return out

    def ffn(self, gate_type, gate, up_type, up, down_type, down, n_embd, n_ff, act, x, m, mem=L.MEM_DEVICE,
            sync=True, out=None):
        """LlamaTransformer::feed_forward (transformer.rs:378-408) of m rows."""
        if out is None:
            if mem == L.MEM_HOST:
                out = np.empty((m, n_embd), np.float32)
            else:
                import torch
                out = torch.empty((m, n_embd), dtype=torch.float32, device=x.device)
        L.check(self._lib.barq_rocm_ffn(self.h, gate_type, _ptr(gate), up_type, _ptr(up), down_type, _ptr(down),
                                        n_embd, n_ff, act, _ptr(x), m, _ptr(out), mem))
        if mem == L.MEM_DEVICE and sync:
            self.sync()
        return out

    def gemm_f32(self, a, b, m, k, n, mem=L.MEM_DEVICE):
        if mem == L.MEM_HOST:
            c = np.empty((m, n), dtype=np.float32)
        else:
            import torch
            c = torch.empty((m, n), dtype=torch.float32, device=a.device)
        L.check(self._lib.barq_rocm_gemm_f32(self.h, _ptr(a), _ptr(b), m, k, n, _ptr(c), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return c

    def gemv_f32(self, a, x, m, n, mem=L.MEM_DEVICE):
        if mem == L.MEM_HOST:
            y = np.empty(m, dtype=np.float32)
        else:
            import torch
            y = torch.empty(m, dtype=torch.float32, device=a.device)
        L.check(self._lib.barq_rocm_gemv_f32(self.h, _ptr(a), _ptr(x), m, n, _ptr(y), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return y

    def dequantize_split(self, kind, quants, scales, block_size, n_out, mem=L.MEM_HOST):
        if mem == L.MEM_HOST:
            out = np.empty(n_out, dtype=np.float32)
            nq, ns = quants.size, scales.size
        else:
            import torch
            out = torch.empty(n_out, dtype=torch.float32, device=quants.device)
            nq, ns = quants.numel(), scales.numel()
        L.check(self._lib.barq_rocm_dequantize_split(self.h, kind, _ptr(quants), nq, _ptr(scales), ns,
                                                     block_size, _ptr(out), n_out, mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return out

    def quantized_matmul_split(self, a, bq, bs, m, n, k, kind, block_size, mem=L.MEM_HOST):
        if mem == L.MEM_HOST:
            c = np.empty((m, n), dtype=np.float32)
            nq, ns = bq.size, bs.size
        else:
            import torch
            c = torch.empty((m, n), dtype=torch.float32, device=a.device)
            nq, ns = bq.numel(), bs.numel()
        L.check(self._lib.barq_rocm_quantized_matmul_split(self.h, _ptr(a), _ptr(bq), nq, _ptr(bs), ns, _ptr(c),
                                                           m, n, k, kind, block_size, mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return c

    def quantize_q4_0_barq(self, x, mem=L.MEM_DEVICE):
        n = x.size if mem == L.MEM_HOST else x.numel()
        if mem == L.MEM_HOST:
            out = np.empty(n // 32 * 20, dtype=np.uint8)
        else:
            import torch
            out = torch.empty(n // 32 * 20, dtype=torch.uint8, device=x.device)
        L.check(self._lib.barq_rocm_quantize_q4_0_barq(self.h, _ptr(x), n, _ptr(out), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return out

    def quantize_q4_k_barq(self, x, mem=L.MEM_DEVICE):
        """quant::Q4_K::quantize (quant/src/q4_k.rs:23-73)."""
        n = x.size if mem == L.MEM_HOST else x.numel()
        nbytes = self._lib.barq_rocm_q4_k_barq_bytes(n)
        if mem == L.MEM_HOST:
            out = np.empty(nbytes, dtype=np.uint8)
        else:
            import torch
            out = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        L.check(self._lib.barq_rocm_quantize_q4_k_barq(self.h, _ptr(x), n, _ptr(out), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return out

    def moe_route(self, logits, rows, n_experts, top_k, mem=L.MEM_DEVICE):
        k = max(1, min(top_k, n_experts))
        if mem == L.MEM_HOST:
            ids = np.empty((rows, k), dtype=np.int32)
            w = np.empty((rows, k), dtype=np.float32)
        else:
            import torch
            ids = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
            w = torch.empty((rows, k), dtype=torch.float32, device=logits.device)
        L.check(self._lib.barq_rocm_moe_route(self.h, _ptr(logits), rows, n_experts, top_k, _ptr(ids), _ptr(w), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return ids, w

    def moe_route_reduce(self, logits, rows, n_experts, top_k, max_active, min_weight, mem=L.MEM_DEVICE):
        """Top-k routing followed by reduce_expert_assignments in one launch."""
        k = max(1, min(top_k, n_experts))
        if mem == L.MEM_HOST:
            ids = np.empty((rows, k), dtype=np.int32)
            w = np.empty((rows, k), dtype=np.float32)
        else:
            import torch
            ids = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
            w = torch.empty((rows, k), dtype=torch.float32, device=logits.device)
        L.check(self._lib.barq_rocm_moe_route_reduce(self.h, _ptr(logits), rows, n_experts, top_k, max_active,
                                                     min_weight, _ptr(ids), _ptr(w), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return ids, w

    def moe_reduce(self, ids, weights, max_active, min_weight, mem=L.MEM_DEVICE, out=None):
        """reduce_expert_assignments on rows x k slots; out=(ids, weights) may be the inputs."""
        rows, k = tuple(ids.shape)
        if out is not None:
            oi, ow = out
        elif mem == L.MEM_HOST:
            oi = np.empty((rows, k), dtype=np.int32)
            ow = np.empty((rows, k), dtype=np.float32)
        else:
            import torch
            oi = torch.empty((rows, k), dtype=torch.int32, device=ids.device)
            ow = torch.empty((rows, k), dtype=torch.float32, device=ids.device)
        L.check(self._lib.barq_rocm_moe_reduce(self.h, _ptr(ids), _ptr(weights), rows, k, max_active, min_weight,
                                               _ptr(oi), _ptr(ow), mem))
        if mem == L.MEM_DEVICE:
            self.sync()
        return oi, ow

    def moe_ffn(self, gate_type, gates, up_type, ups, down_type, downs, hidden, n_ff, x, rows, ids, weights,
                top_k, act, mem=L.MEM_DEVICE, sync=True, out=None):
        ne = len(gates)
        arr = ctypes.c_void_p * ne
        g = arr(*[_ptr(t) for t in gates])
        u = arr(*[_ptr(t) for t in ups])
        d = arr(*[_ptr(t) for t in downs])
        if out is not None:
            pass
        elif mem == L.MEM_HOST:
            out = np.empty((rows, hidden), dtype=np.float32)
        else:
            import torch
            out = torch.empty((rows, hidden), dtype=torch.float32, device=x.device)
        L.check(self._lib.barq_rocm_moe_ffn(self.h, ne, gate_type, g, up_type, u, down_type, d, hidden, n_ff,
                                            _ptr(x), rows, _ptr(ids), _ptr(weights), top_k, act, _ptr(out), mem))
        if mem == L.MEM_DEVICE and sync:
            self.sync()
        return out
