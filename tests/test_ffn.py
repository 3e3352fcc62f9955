"""The dense FFN's oracle (LlamaTransformer::feed_forward,
models/src/transformer.rs:378-408) pinned without a GPU: the SwiGLU's
rounding order (transformer.rs:394-399 against ops::Silu's form), its
closed forms, and the whole FFN against a float64 brute force over the
dequantized weights (a gate/up swap or a dropped term fails it)."""
import ctypes

import numpy as np
import pytest

from barq_rocm import synth

import barq_rocm as B

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def expf(v):
    return np.float32([_libm.expf(float(t)) for t in np.ravel(v)]).reshape(np.shape(v))


def test_swiglu_rounds_as_transformer_not_as_ops_silu(orc):
    # (g * (1 / (1 + e))) * u and (g / (1 + e)) * u differ in the last bit for
    # some g; the dense FFN must take the first form
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    e = expf(-g)
    one = np.float32(1.0)
    dense = (g * (one / (one + e))) * u
    moe = (g / (one + e)) * u
    assert np.count_nonzero(dense != moe) > 50        # the two roundings are distinguishable here
    h = orc.ffn_swiglu(g, u)
    assert np.array_equal(h.view(np.uint32), dense.view(np.uint32))


def test_swiglu_closed_forms(orc):
    g = np.float32([0.0, -0.0, 30.0, 100.0, -100.0, -1000.0, 1.0, -1.0])
    u = np.float32([5.0, 5.0, 2.0, -3.0, 7.0, 1.0, 1.0, 1.0])
    h = orc.ffn_swiglu(g, u)
    assert h[0] == 0.0 and h[1] == 0.0                 # silu(0) = 0
    assert h[2] == np.float32(60.0)                    # exp(-30) vanishes against 1 in f32
    assert h[3] == np.float32(-300.0)
    assert h[4] == 0.0 and h[5] == 0.0                 # exp(100) overflows: 1 / inf = 0
    ref = np.float64(g[6:]) * np.float64(u[6:]) / (1.0 + np.exp(-np.float64(g[6:])))
    assert np.allclose(h[6:], ref, rtol=3e-7, atol=0)  # silu(1) = 0.7311, silu(-1) = -0.2689


def ffn_case(n_embd, n_ff, m, seed, gt=B.Q4_K, ut=B.Q4_K, dt=B.Q6_K):
    gate = synth.gen_weights(gt, n_ff, n_embd, seed)
    up = synth.gen_weights(ut, n_ff, n_embd, seed + 1)
    down = synth.gen_weights(dt, n_embd, n_ff, seed + 2)
    x = synth.gen_f32(m * n_embd, seed + 3).reshape(m, n_embd)
    return gate, up, down, x


def brute_force(orc, gt, gate, ut, up, dt, down, n_embd, n_ff, x):
    G = orc.dequantize(gt, gate, n_ff * n_embd).reshape(n_ff, n_embd).astype(np.float64)
    U = orc.dequantize(ut, up, n_ff * n_embd).reshape(n_ff, n_embd).astype(np.float64)
    D = orc.dequantize(dt, down, n_embd * n_ff).reshape(n_embd, n_ff).astype(np.float64)
    xx = np.asarray(x, np.float64)
    g, u = xx @ G.T, xx @ U.T
    h = g / (1.0 + np.exp(-g)) * u
    return h @ D.T


@pytest.mark.parametrize("types", [(B.Q4_K, B.Q4_K, B.Q6_K), (B.Q4_0, B.Q4_0, B.Q8_0), (B.Q6_K, B.Q4_K, B.Q4_K)])
def test_ffn_literal_equals_float64_brute_force(orc, types):
    gt, ut, dt = types
    n_embd, n_ff, m = 256, 512, 3
    gate, up, down, x = ffn_case(n_embd, n_ff, m, 60 + gt, gt, ut, dt)
    out = orc.ffn(gt, gate, ut, up, dt, down, n_embd, n_ff, orc.F32, x, m)
    ref = brute_force(orc, gt, gate, ut, up, dt, down, n_embd, n_ff, x)
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert err < 2e-5, err
    # gate and up swapped is a different function: the check above would fail it
    swapped = brute_force(orc, ut, up, gt, gate, dt, down, n_embd, n_ff, x)
    assert np.max(np.abs(swapped - ref)) / np.max(np.abs(ref)) > 1e-2


def test_ffn_q8_is_the_literal_ffn_on_quantized_rows(orc):
    # act Q8_K: x and h pass through Q8_K; against float64 the only extra error
    # is that quantization noise, and the Q8 result equals its pieces chained
    n_embd, n_ff, m = 512, 768, 2
    gate, up, down, x = ffn_case(n_embd, n_ff, m, 70)
    xq = orc.quantize_act(orc.Q8_K, x)
    out = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.Q8_K, xq, m)
    g = orc.matmul(B.Q4_K, gate, n_ff, n_embd, orc.Q8_K, xq, m)
    u = orc.matmul(B.Q4_K, up, n_ff, n_embd, orc.Q8_K, xq, m)
    h = orc.ffn_swiglu(g, u)
    hq = np.concatenate([orc.quantize_q8_k(h[r]) for r in range(m)])
    chained = orc.matmul(B.Q6_K, down, n_embd, n_ff, orc.Q8_K, hq, m)
    assert np.array_equal(out.view(np.uint32), chained.view(np.uint32))
    ref = brute_force(orc, B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, x)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 3e-2
