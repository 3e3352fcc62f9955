"""GPU parity of the batched (M >= 16) int8-MFMA GEMM against the CPU oracle.

The oracle is gemm_f32(dequant(Q8_K(X)), dequant(W)^T) in sequential f32
(barq_core/src/blas.rs:199-210 over gguf.rs decoders); the bar is the north
star's 1e-3 (relative L2 and max-abs relative to max |y|)."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth
from conftest import assert_close_1e3

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def q6k_full_range(n, k, seed):
    """Q6_K blocks whose int8 sub-block scales span [-128, 127] (real
    llama.cpp Q6_K files use the whole range), so w' = sc*(q-32) reaches
    +4096 and -4064."""
    w = synth.gen_q6_k(n, k, seed).reshape(-1, 210).copy()
    rng = np.random.default_rng(seed)
    w[:, 192:208] = rng.integers(0, 256, size=(w.shape[0], 16), dtype=np.uint8)
    w[0, 192:208] = 0x80          # sc = -128 everywhere in block 0
    w[0, 0:192] = 0               # q = 0 -> q - 32 = -32 -> w' = 4096
    return w.reshape(-1)


def run(be, orc, t, w, n, k, m, seed):
    at = B.Q8_PARTNER[t]
    x = synth.gen_f32(m * k, seed).reshape(m, k)
    xq = be.quantize_act(at, dev(x))
    y = host(be.matmul(t, dev(w), n, k, at, xq, m))
    ref = orc.matmul(t, w, n, k, at, host(xq), m)
    assert_close_1e3(y, ref)
    return y, host(xq)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("n,k,m", [(64, 256, 16), (130, 768, 47), (512, 1024, 128), (1000, 512, 300), (64, 256, 513)])
def test_gemm_mfma_shapes(be, orc, name, n, k, m):
    t = {"Q4_K": B.Q4_K, "Q6_K": B.Q6_K}[name]
    print(f"gemm {name} n={n} k={k} m={m}", flush=True)
    w = synth.gen_weights(t, n, k, 900 + n + m)
    run(be, orc, t, w, n, k, m, 901 + m)


def test_gemm_mfma_q6k_full_scale_range(be, orc):
    n, k, m = 96, 512, 40
    print("gemm Q6_K full-range scales", flush=True)
    run(be, orc, B.Q6_K, q6k_full_range(n, k, 5), n, k, m, 6)


def test_gemm_q6k_128_row_tiles(be, orc):
    """Q6_K prompts of 256+ rows against long K take 128 x 128 tiles (four
    waves of 128 x 32, K slices): ragged M and N, and scales over the whole
    int8 range (w' = sc*(q - 32) up to +4096 and down to -4064)."""
    for n, k, m, full in [(520, 8192, 260, False), (136, 8192, 300, True)]:
        print(f"gemm Q6_K 128-row tiles n={n} k={k} m={m} full-range={full}", flush=True)
        w = q6k_full_range(n, k, 11) if full else synth.gen_weights(B.Q6_K, n, k, 10)
        run(be, orc, B.Q6_K, w, n, k, m, 12 + m)


def test_gemm_mfma_q4k_extreme_blocks(be, orc):
    # all-0xFF scale bytes (sc = m = 63), all-0xFF quants, f16 extremes for d / dmin
    n, k, m = 80, 512, 33
    w = synth.gen_q4_k(n, k, 9).reshape(-1, 144).copy()
    f16s = np.float16([0.0, 2.0 ** -24, 6.1e-5, 4.0, -1.5, 1.0]).view(np.uint8).reshape(-1, 2)
    for i in range(0, w.shape[0], 5):
        w[i, 0:2] = f16s[i % 6]
        w[i, 2:4] = f16s[(i + 3) % 6]
        if i % 3 == 0:
            w[i, 4:] = 0xFF
    print("gemm Q4_K extreme blocks", flush=True)
    run(be, orc, B.Q4_K, w.reshape(-1), n, k, m, 10)


def test_gemm_rows_equal_gemv(be):
    # a matmul row is the matvec of that activation row (same Q8_K blocks)
    t, n, k, m = B.Q4_K, 384, 2048, 64
    w = synth.gen_q4_k(n, k, 11)
    x = synth.gen_f32(m * k, 12).reshape(m, k)
    wd = dev(w)
    xq = be.quantize_act(B.Q8_K, dev(x))
    y = host(be.matmul(t, wd, n, k, B.Q8_K, xq, m))
    rb = B.row_bytes(B.Q8_K, k)
    for r in (0, 17, 63):
        yr = host(be.matvec(t, wd, n, k, B.Q8_K, xq[r * rb:(r + 1) * rb]))
        assert_close_1e3(y[r], yr, tol=1e-5)


def test_gemm_c4_config(be, orc):
    """BASELINE config 4 at full size (Q4_K 4096x4096, 512 tokens); the oracle
    checks a spread of 48 token rows (all 4096 outputs each)."""
    t, w, x = synth.linear_inputs(4)
    c = synth.CONFIGS[4]
    n, k, m = c["n_rows"], c["k"], c["m"]
    print("gemm full config C4", flush=True)
    xq = be.quantize_act(B.Q8_K, dev(x))
    xq_h = host(xq)
    assert np.array_equal(xq_h, orc.quantize_act(B.Q8_K, x))
    y = host(be.matmul(t, dev(w), n, k, B.Q8_K, xq, m))
    rows = np.linspace(0, m - 1, 48).astype(int)
    rb = B.row_bytes(B.Q8_K, k)
    sub = np.concatenate([xq_h[r * rb:(r + 1) * rb] for r in rows])
    ref = orc.matmul(t, w, n, k, B.Q8_K, sub, len(rows))
    assert_close_1e3(y[rows], ref)
