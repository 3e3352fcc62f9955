"""One Llama-3-8B transformer layer (LlamaTransformer::forward_layer,
models/src/transformer.rs:123-144) chained through the C ABI from a GGUF
file and the device weight cache, against the oracle chained the same way:
a 3-token prompt chunk at position 0, then one decode token at position 3,
sharing one device KV cache.

    attn_norm (RMSNorm -> Q8_K) -> q / k / v projections -> RoPE(q),
    RoPE(k) + transpose(v) + KV append -> attention -> output projection
    -> residual add + ffn_norm (-> Q8_K) -> feed_forward -> residual add

Two chains: the integer path (activations quantized to Q8_K before every
projection, as a deployment runs it) and the literal f32 path (the
reference's own arithmetic).  Bars: the literal chain within 1e-4 of the
oracle (summation order, the device's sincosf and base-2 exponentials are
the only differences); the integer chain at the chained-quantization bar
of conftest.assert_close_chained; the KV cache rows within the RoPE bar
(2e-6 of max |k|) and V bit-exact for the literal chain."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import attention as A
from barq_rocm import synth
from barq_rocm.gguf import GgufFile, WeightCache
import gguf_writer as W
from conftest import assert_close_1e3, assert_close_chained

pytestmark = pytest.mark.gpu

N_EMBD, N_HEAD, N_KV, HD, N_FF = 4096, 32, 8, 128, 14336
EPS = 1e-5
LAYOUT = A.ROPE_INTERLEAVED
# Llama-3-8B Q4_K_M mix: (name, type, n_rows, k)
TENSORS = [
    ("blk.0.attn_q.weight", B.Q4_K, N_HEAD * HD, N_EMBD),
    ("blk.0.attn_k.weight", B.Q4_K, N_KV * HD, N_EMBD),
    ("blk.0.attn_v.weight", B.Q6_K, N_KV * HD, N_EMBD),
    ("blk.0.attn_output.weight", B.Q4_K, N_EMBD, N_HEAD * HD),
    ("blk.0.ffn_gate.weight", B.Q4_K, N_FF, N_EMBD),
    ("blk.0.ffn_up.weight", B.Q4_K, N_FF, N_EMBD),
    ("blk.0.ffn_down.weight", B.Q6_K, N_EMBD, N_FF),
]


def inv_freq(hd, base=500000.0):
    return np.array([np.float32(base) ** np.float32(-2.0 * i / hd) for i in range(hd // 2)], dtype=np.float32)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def layer(tmp_path_factory):
    w = {name: synth.gen_weights(t, n, k, 700 + i) for i, (name, t, n, k) in enumerate(TENSORS)}
    # the synthetic projections have large outputs; scale the norm weights so the
    # residual stream stays in a range where the softmax is not one-hot
    w["blk.0.attn_norm.weight"] = (0.01 * (1.0 + 0.1 * synth.gen_f32(N_EMBD, 720))).astype(np.float32)
    w["blk.0.ffn_norm.weight"] = (0.01 * (1.0 + 0.1 * synth.gen_f32(N_EMBD, 721))).astype(np.float32)
    w["output_norm.weight"] = np.ones(N_EMBD, np.float32)
    path = str(tmp_path_factory.mktemp("layer") / "llama3_layer.gguf")
    ts = [(name, [k, n], t, w[name].tobytes()) for name, t, n, k in TENSORS]
    ts += [(nm, [N_EMBD], 0, w[nm].tobytes()) for nm in ("blk.0.attn_norm.weight", "blk.0.ffn_norm.weight",
                                                         "output_norm.weight")]
    W.write(path, [("general.architecture", W.STRING, "llama")], ts)
    return path, w


def oracle_layer(orc, w, x, cache, start, q8):
    """forward_layer in the oracle's arithmetic; cache = [K, V] numpy arrays
    [N_KV, positions, HD] extended in place."""
    seq = x.shape[0]
    f = inv_freq(HD)
    t = {name: (tt, n, k) for name, tt, n, k in TENSORS}

    def proj(name, inp):
        tt, n, k = t[name]
        if q8:
            a = B.Q8_PARTNER[tt]
            return orc.matmul(tt, w[name], n, k, a, orc.quantize_act(a, inp), inp.shape[0])
        return orc.matmul(tt, w[name], n, k, orc.F32, inp, inp.shape[0])

    normed = orc.rms_norm(x, w["blk.0.attn_norm.weight"], EPS)
    q, k, v = proj("blk.0.attn_q.weight", normed), proj("blk.0.attn_k.weight", normed), proj("blk.0.attn_v.weight", normed)
    q_rope = orc.rope(q, seq, N_HEAD, HD, start, 1.0, f, LAYOUT)
    k_rope = orc.rope(k, seq, N_KV, HD, start, 1.0, f, LAYOUT)
    v_t = orc.transpose_heads(v, seq, N_KV, HD)
    cache[0] = np.concatenate([cache[0], k_rope], axis=1)
    cache[1] = np.concatenate([cache[1], v_t], axis=1)
    attn = orc.attention(q_rope, cache[0], cache[1], N_HEAD, seq, start + seq, start).reshape(seq, N_EMBD)
    o = proj("blk.0.attn_output.weight", attn)
    res = x + o
    n2 = orc.rms_norm(res, w["blk.0.ffn_norm.weight"], EPS)
    gt = t["blk.0.ffn_gate.weight"][0]
    if q8:
        ff = orc.ffn(gt, w["blk.0.ffn_gate.weight"], gt, w["blk.0.ffn_up.weight"], B.Q6_K, w["blk.0.ffn_down.weight"],
                     N_EMBD, N_FF, orc.Q8_K, orc.quantize_act(orc.Q8_K, n2), seq)
    else:
        ff = orc.ffn(gt, w["blk.0.ffn_gate.weight"], gt, w["blk.0.ffn_up.weight"], B.Q6_K, w["blk.0.ffn_down.weight"],
                     N_EMBD, N_FF, orc.F32, n2, seq)
    return res + ff


def device_layer(be, wc, norms, kv, x, start, q8):
    """forward_layer through the C ABI on device buffers."""
    import torch
    seq = x.shape[0]
    f = dev(inv_freq(HD))
    get = {name: wc.get(name) for name, *_ in TENSORS}

    def proj(name, inp, act):
        tt, n, k, ptr = get[name]
        y = torch.empty((inp_rows, n), dtype=torch.float32, device="cuda")
        be.matmul_raw(tt, ptr, n, k, act, inp, inp_rows, y, B.MEM_DEVICE)
        return y

    inp_rows = seq
    if q8:
        xin = be.add_rms_norm_quantize(B.Q8_K, x, None, norms["blk.0.attn_norm.weight"], EPS, sync=False)
        act = B.Q8_K
    else:
        xin = be.add_rms_norm_quantize(B.F32, x, None, norms["blk.0.attn_norm.weight"], EPS, sync=False)
        act = B.ACT_F32
    q = proj("blk.0.attn_q.weight", xin, act)
    k = proj("blk.0.attn_k.weight", xin, act)
    v = proj("blk.0.attn_v.weight", xin, act)
    q_rope = A.apply_rope(be, q, seq, N_HEAD, HD, start, 1.0, f, LAYOUT, sync=False)
    kv.append_rope(0, k, v, seq, start, 1.0, f, LAYOUT)
    attn = A.compute_attention(be, q_rope, kv, 0, N_HEAD, N_KV, HD, seq, start + seq, start, sync=False)
    o = proj("blk.0.attn_output.weight", attn.reshape(seq, N_EMBD), B.ACT_F32_Q8 if q8 else B.ACT_F32)
    res = torch.empty_like(x)
    gt, _, _, gp = get["blk.0.ffn_gate.weight"]
    ut, _, _, up = get["blk.0.ffn_up.weight"]
    dt, _, _, dp = get["blk.0.ffn_down.weight"]
    if q8:
        x2 = be.add_rms_norm_quantize(B.Q8_K, x, o, norms["blk.0.ffn_norm.weight"], EPS, sum_out=res, sync=False)
        ff = be.ffn(gt, gp, ut, up, dt, dp, N_EMBD, N_FF, B.Q8_K, x2, seq, sync=False)
    else:
        x2 = be.add_rms_norm_quantize(B.F32, x, o, norms["blk.0.ffn_norm.weight"], EPS, sum_out=res, sync=False)
        ff = be.ffn(gt, gp, ut, up, dt, dp, N_EMBD, N_FF, B.ACT_F32, x2, seq, sync=False)
    # the closing residual add: as the next layer would run it, fused with its norm
    out = torch.empty_like(x)
    be.add_rms_norm_quantize(B.Q8_K, res, ff, norms["output_norm.weight"], EPS, sum_out=out, sync=False)
    be.sync()
    return out


@pytest.mark.parametrize("q8", [True, False], ids=["integer", "literal_f32"])
def test_decode_layer_chain(be, orc, layer, q8):
    path, w = layer
    with GgufFile(path) as g:
        wc = WeightCache(be, g)
        norms = {}
        for nm in ("blk.0.attn_norm.weight", "blk.0.ffn_norm.weight", "output_norm.weight"):
            t, n_rows, k, ptr = wc.get(nm)
            assert (t, n_rows, k) == (0, 1, N_EMBD)
            norms[nm] = ptr
        kv = A.KVCache(be, 64, 1, N_KV, HD)
        cache = [np.zeros((N_KV, 0, HD), np.float32), np.zeros((N_KV, 0, HD), np.float32)]
        x_all = synth.gen_f32(4 * N_EMBD, 730).reshape(4, N_EMBD)
        for step, (start, seq) in enumerate([(0, 3), (3, 1)]):
            x = x_all[start:start + seq]
            print(f"layer chain {'integer' if q8 else 'literal'}: step {step}, positions {start}..{start + seq - 1}",
                  flush=True)
            got = device_layer(be, wc, norms, kv, dev(x), start, q8).cpu().numpy()
            ref = oracle_layer(orc, w, x, cache, start, q8)
            if q8:
                assert_close_chained(got, ref)
            else:
                assert_close_1e3(got, ref, tol=1e-4)
            for h in (0, N_KV - 1):
                kd, vd = kv.get_head(0, h)
                assert kd.shape[0] == start + seq and vd.shape[0] == start + seq
                if q8:
                    assert_close_chained(kd, cache[0][h])
                    assert_close_chained(vd, cache[1][h])
                else:
                    assert_close_1e3(kd, cache[0][h], tol=1e-5)
                    assert_close_1e3(vd, cache[1][h], tol=1e-5)
        kv.close()
        wc.close()
