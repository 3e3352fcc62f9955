"""LlamaTransformer::forward (models/src/transformer.rs:81-94) on the device,
integer path: every projection takes Q8_K activation rows written by the
fused residual-add + RMSNorm quantizer, as a deployment runs it.

    get_embeddings (:96-119)              -> barq_rocm_get_rows
    forward_layer (:123-144), per layer:
      rms_norm(attn_norm) (:148-172)      -> barq_rocm_add_rms_norm_quantize
                                             (the previous layer's closing
                                             residual add fused in)
      q / k / v proj (:212-220) + biases  -> barq_rocm_qkv_append_rope (one
        (:206-220), RoPE (:222-240),         token, no biases) or matmul x3
        KV append (:243-245)                 [+ add_bias] + kv_cache_append_rope_q
      compute_attention (:301-374)        -> barq_rocm_attention_q8k (rows
                                             quantized for the o projection)
      o proj (:247-251)                   -> barq_rocm_matmul
      residual add + ffn_norm (:136-139)  -> barq_rocm_add_rms_norm_quantize
      feed_forward (:378-408)             -> barq_rocm_ffn
    final_output (:468-498): output_norm of the last row, the LM head
      (output.weight, else the tied token_embd.weight), output.bias when its
      length is the vocabulary's           -> add_rms_norm_quantize, matmul,
                                             barq_rocm_add_bias

Weights come from a lookup name -> (type, n_rows, k, device pointer) or
None: a WeightCache of a GGUF file (WeightCache.find) or any mapping with
the GGUF tensor names.  Every compute step is a libbarq_rocm call on the
backend's stream; torch only allocates the activation buffers.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib as L
from . import attention as A
from .backend import Backend


@dataclass
class LlamaConfig:
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_ff: int
    rope_freq_base: float = 500000.0
    rope_freq_scale: float = 1.0
    rms_norm_eps: float = 1e-5
    rope_layout: int = A.ROPE_INTERLEAVED

    def inv_freq(self) -> np.ndarray:
        """rope_inv_freq (transformer.rs:48-52): base^(-2i/head_dim) in f32."""
        hd = self.head_dim
        return np.array([np.float32(self.rope_freq_base) ** np.float32(-2.0 * i / hd) for i in range(hd // 2)],
                        dtype=np.float32)


class DeviceLlama:
    """forward(tokens, start_pos) -> logits of the last token, on the device.

    get(name) returns (type, n_rows, k, device pointer) or None.  The KV
    cache is the caller's (attention.KVCache with cfg.n_layer layers)."""

    def __init__(self, be: Backend, cfg: LlamaConfig, get, kv: A.KVCache):
        import torch
        self.be, self.cfg, self.get, self.kv = be, cfg, get, kv
        self.inv_freq = torch.from_numpy(cfg.inv_freq()).cuda()
        head = get("output.weight") or get("token_embd.weight")
        if head is None:
            raise KeyError("No output or token embedding weight found")
        self.head = head
        self.n_vocab = head[1]
        bias = get("output.bias")
        self.out_bias = bias if bias is not None and bias[2] * bias[1] == self.n_vocab else None
        self._bufs = {}

    def _need(self, name):
        w = self.get(name)
        if w is None:
            raise KeyError(f"{name} not found in cache")
        return w

    def _norm(self, name):
        w = self.get(name)
        if w is None:
            # rms_norm returns its input unchanged without a weight (:153-156);
            # the fused quantizer always normalises, so that form is not offered
            raise NotImplementedError(f"{name} absent: the integer path needs every norm weight")
        return w[3]

    def _buf(self, key, shape, dtype="float32"):
        """Activation buffers reused across calls (so a captured graph replays
        on the same addresses)."""
        import torch
        b = self._bufs.get(key)
        if b is None or tuple(b.shape) != tuple(shape):
            b = torch.empty(shape, dtype=getattr(torch, dtype), device="cuda")
            self._bufs[key] = b
        return b

    def embed(self, tokens):
        """get_embeddings: tokens (device int32 [seq]) -> [seq, n_embd] f32."""
        t, n_rows, k, p = self._need("token_embd.weight")
        out = self._buf(("emb", len(tokens)), (len(tokens), k))
        return self.be.get_rows(t, p, n_rows, k, tokens, sync=False, out=out)

    def forward(self, tokens, start_pos: int, trace=None):
        """Logits [n_vocab] (device f32) of the last of the tokens at
        positions start_pos .. start_pos + len(tokens) - 1."""
        return self.forward_hidden(self.embed(tokens), start_pos, trace)

    def forward_hidden(self, hidden, start_pos: int, trace=None):
        import torch
        """trace: a list that receives, per layer, device copies of the
        layer's input rows, its attention output (after the o projection) and
        the two addends of its output (residual, FFN output); the output sum
        itself is formed inside the next layer's norm."""
        be, c, kv = self.be, self.cfg, self.kv
        seq = int(hidden.shape[0])
        nbq = c.n_embd // 256 * 292
        q_rows = c.n_head * c.head_dim
        xq = self._buf(("xq", seq), (seq, nbq), "uint8")
        xq2 = self._buf(("xq2", seq), (seq, nbq), "uint8")
        aq = self._buf(("aq", seq), (seq, q_rows // 256 * 292), "uint8")
        qr = self._buf(("qr", seq), (c.n_head, seq, c.head_dim))
        o = self._buf(("o", seq), (seq, c.n_embd))
        res = [self._buf(("res0", seq), (seq, c.n_embd)), self._buf(("res1", seq), (seq, c.n_embd))]
        ff = self._buf(("ff", seq), (seq, c.n_embd))
        x, prev = hidden, None
        r_mid = res[1]
        for il in range(c.n_layer):
            pre = f"blk.{il}."
            r_in = res[0]
            # x + previous FFN output (the closing add of the last layer), normed
            be.add_rms_norm_quantize(L.Q8_K, x, prev, self._norm(pre + "attn_norm.weight"), c.rms_norm_eps,
                                     sum_out=r_in if prev is not None else None, out=xq, sync=False)
            if prev is None:
                r_in = x
            wq, wk, wv = (self._need(pre + f"attn_{m}.weight") for m in "qkv")
            biases = [self.get(pre + f"attn_{m}.bias") for m in "qkv"]
            if seq == 1 and all(b is None for b in biases):
                kv.qkv_append_rope(il, [wq[0], wk[0], wv[0]], [wq[3], wk[3], wv[3]], c.n_head, c.n_embd, L.Q8_K,
                                   xq, start_pos, c.rope_freq_scale, self.inv_freq, c.rope_layout, q_out=qr)
            else:
                outs = []
                for m, w, b in zip("qkv", (wq, wk, wv), biases):
                    y = self._buf((m, seq), (seq, w[1]))
                    be.matmul_raw(w[0], w[3], w[1], w[2], L.Q8_K, xq, seq, y, L.MEM_DEVICE)
                    if b is not None and b[1] * b[2] == w[1]:
                        be.add_bias(y, b[3], seq, w[1], sync=False)
                    outs.append(y)
                kv.append_rope_q(il, outs[0], c.n_head, outs[1], outs[2], seq, start_pos, c.rope_freq_scale,
                                 self.inv_freq, c.rope_layout, q_out=qr)
            A.compute_attention_q8k(be, qr, kv, il, c.n_head, c.n_head_kv, c.head_dim, seq, start_pos + seq,
                                    start_pos, sync=False, out=aq)
            wo = self._need(pre + "attn_output.weight")
            be.matmul_raw(wo[0], wo[3], wo[1], wo[2], L.Q8_K, aq, seq, o, L.MEM_DEVICE)
            be.add_rms_norm_quantize(L.Q8_K, r_in, o, self._norm(pre + "ffn_norm.weight"), c.rms_norm_eps,
                                     sum_out=r_mid, out=xq2, sync=False)
            g, u, d = (self._need(pre + f"ffn_{m}.weight") for m in ("gate", "up", "down"))
            be.ffn(g[0], g[3], u[0], u[3], d[0], d[3], c.n_embd, c.n_ff, L.Q8_K, xq2, seq, sync=False, out=ff)
            if trace is not None:
                be.sync()   # the copies run on torch's stream, the layer on the backend's
                trace.append((r_in.clone(), o.clone(), r_mid.clone(), ff.clone()))
                torch.cuda.synchronize()
            # the next layer sums x + ff into res[0] (x is res[1]: no buffer aliases another)
            x, prev = r_mid, ff
        return self.final_output(x[seq - 1:seq], prev[seq - 1:seq])

    def final_output(self, res_last, ff_last):
        """final_output of the last row: output_norm(res + ff) as Q8_K, the
        LM head, output.bias."""
        be, c = self.be, self.cfg
        xq = self._buf("xq_out", (1, c.n_embd // 256 * 292), "uint8")
        be.add_rms_norm_quantize(L.Q8_K, res_last, ff_last, self._norm("output_norm.weight"), c.rms_norm_eps,
                                 out=xq, sync=False)
        t, n, k, p = self.head
        logits = self._buf("logits", (1, n))
        be.matmul_raw(t, p, n, k, L.Q8_K, xq, 1, logits, L.MEM_DEVICE)
        if self.out_bias is not None:
            be.add_bias(logits, self.out_bias[3], 1, n, sync=False)
        return logits[0]
