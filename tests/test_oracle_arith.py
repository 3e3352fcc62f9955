"""Pins the oracle's activation quantizers, f32 BLAS, quantized matvec,
split-scale operator API and MoE helpers."""
import numpy as np
import pytest

from conftest import assert_close_1e3


def q8k_fields(blk):
    d = blk[0:4].view(np.float32)[0]
    qs = blk[4:260].view(np.int8)
    bs = blk[260:292].view(np.int16)
    return d, qs, bs


# ---- Q8_K activation quantizer (llama.cpp quantize_row_q8_K_ref) ----------

def test_q8_k_zero_block(orc):
    out = orc.quantize_q8_k(np.zeros(256, np.float32))
    assert np.all(out == 0)


def test_q8_k_invariants_random(orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(256 * 64) * 10.0 ** rng.integers(-3, 3, 256 * 64)).astype(np.float32)
    out = orc.quantize_q8_k(x).reshape(64, 292)
    for b in range(64):
        xb = x[256 * b: 256 * (b + 1)]
        d, qs, bs = q8k_fields(out[b])
        j = int(np.argmax(np.abs(xb)))          # first index of the largest |x|
        assert qs[j] == -127                    # iscale = -127/max maps max to -127
        iscale = np.float32(-127.0) / xb[j]
        assert d == np.float32(1.0) / iscale
        v = np.rint(iscale * xb).astype(np.int64)   # ties to even
        assert np.array_equal(qs.astype(np.int64), np.minimum(127, v))
        assert np.array_equal(bs, qs.reshape(16, 16).sum(axis=1).astype(np.int16))
        # reconstruction error at most half a step
        assert np.all(np.abs(xb - d * qs) <= np.abs(d) * 0.5 * (1 + 1e-5) + 1e-30)


def test_q8_k_first_index_wins_ties_and_sign(orc):
    x = np.zeros(256, np.float32)
    x[5], x[10] = 2.0, -2.0
    d, qs, _ = q8k_fields(orc.quantize_q8_k(x))
    assert qs[5] == -127 and qs[10] == 127 and d < 0
    x[5], x[10] = -2.0, 2.0
    d, qs, _ = q8k_fields(orc.quantize_q8_k(x))
    assert qs[5] == -127 and qs[10] == 127 and d > 0


def test_q8_k_round_half_to_even(orc):
    # max = -127 -> iscale = 1 exactly; x = 2.5 -> 2, 3.5 -> 4, -0.5 -> -0
    x = np.zeros(256, np.float32)
    x[0] = -127.0
    x[1], x[2], x[3], x[4] = 2.5, 3.5, -0.5, 126.5
    _, qs, _ = q8k_fields(orc.quantize_q8_k(x))
    assert list(qs[:5]) == [-127, 2, 4, 0, 126]


# ---- Q8_0 activation quantizer (llama.cpp quantize_row_q8_0_ref) ----------

def test_q8_0_invariants(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(32 * 100).astype(np.float32)
    x[32:64] = 0.0
    out = orc.quantize_q8_0(x).reshape(100, 34)
    for b in range(100):
        xb = x[32 * b: 32 * (b + 1)]
        amax = np.max(np.abs(xb))
        d = np.float32(amax) / np.float32(127.0)
        assert out[b, 0:2].view(np.float16)[0] == np.float16(d)
        qs = out[b, 2:].view(np.int8)
        if amax == 0:
            assert np.all(qs == 0)
            continue
        idv = np.float32(1.0) / d
        prod = (xb * idv).astype(np.float32)
        exp = np.where(prod >= 0, np.floor(prod + 0.5), np.ceil(prod - 0.5))  # roundf: half away
        assert np.array_equal(qs, exp.astype(np.int8))
        assert np.max(np.abs(qs)) == 127


def test_q8_0_round_half_away_from_zero(orc):
    x = np.zeros(32, np.float32)
    x[0] = 127.0          # d = 1, id = 1
    x[1], x[2] = 2.5, -2.5
    qs = orc.quantize_q8_0(x)[2:].view(np.int8)
    assert qs[1] == 3 and qs[2] == -3


# ---- f32 BLAS (blas.rs, gemm.rs, ops.rs reference tests) ------------------

def test_gemm_f32_reference_known_answers(orc):
    # blas.rs:314-325, gemm.rs:498-517, ops.rs MatMul
    c = orc.gemm_f32(np.float32([1, 2, 3, 4]), np.float32([5, 6, 7, 8]), 2, 2, 2)
    assert c.reshape(-1).tolist() == [19, 22, 43, 50]
    # blas.rs:327-341, gemm.rs:519-537
    c = orc.gemm_f32(np.float32([1, 2, 3, 4, 5, 6]), np.float32([7, 8, 9, 10, 11, 12]), 2, 3, 2)
    assert c.reshape(-1).tolist() == [58, 64, 139, 154]


def test_gemv_f32_reference_known_answer(orc):
    # blas.rs:343-353
    assert orc.gemv_f32(np.float32([1, 2, 3, 4]), np.float32([5, 6]), 2, 2).tolist() == [17, 39]


def test_sums_are_sequential_in_k_order(orc):
    # blas.rs:204-207 adds left to right in f32: (1e8 + 1) - 1e8 == 0
    a = np.float32([1e8, 1.0, -1e8])
    assert orc.gemv_f32(a, np.float32([1, 1, 1]), 1, 3)[0] == 0.0
    assert orc.gemm_f32(a, np.float32([1, 1, 1]), 1, 3, 1)[0, 0] == 0.0


def test_gemm_matches_f64_brute_force(orc):
    rng = np.random.default_rng(6)
    a = rng.standard_normal((7, 33)).astype(np.float32)
    b = rng.standard_normal((33, 5)).astype(np.float32)
    c = orc.gemm_f32(a, b, 7, 33, 5)
    assert np.allclose(c, a.astype(np.float64) @ b.astype(np.float64), rtol=1e-5, atol=1e-5)


# ---- quantized matvec / matmul -----------------------------------------------

@pytest.mark.parametrize("wt", ["Q4_0", "Q4_0_BARQ", "Q8_0", "Q4_K", "Q6_K"])
def test_matvec_equals_gemv_over_dequantized(orc, wt):
    from barq_rocm import synth
    import barq_rocm as B
    t = getattr(B, wt)
    n, k = 37, 512
    w = synth.gen_weights(t, n, k, 77)
    x = synth.gen_f32(k, 78)
    wf = orc.dequantize(t, w, n * k)
    # literal path == blas::gemv_f32(dequant(W), x), bit for bit
    assert np.array_equal(orc.matvec(t, w, n, k, orc.F32, x), orc.gemv_f32(wf, x, n, k))
    # and == gemm_f32(x, W^T) (weight_cache.rs transpose + blas.rs:199-210)
    assert np.array_equal(orc.matvec(t, w, n, k, orc.F32, x), orc.gemm_f32(x, wf.reshape(n, k).T.copy(), 1, k, n)[0])
    # the Q8 path == gemv over dequant(W) and dequant(Q8(x)); close to f64 truth
    at = B.Q8_PARTNER[t]
    xq = orc.quantize_act(at, x)
    y = orc.matvec(t, w, n, k, at, xq)
    xd = orc.dequantize(at, xq, k)
    assert np.array_equal(y, orc.gemv_f32(wf, xd, n, k))
    assert_close_1e3(y, wf.reshape(n, k).astype(np.float64) @ xd.astype(np.float64), tol=1e-5)


def test_matmul_rows_equal_matvec(orc):
    from barq_rocm import synth
    import barq_rocm as B
    n, k, m = 19, 512, 3
    w = synth.gen_q4_k(n, k, 5)
    x = synth.gen_f32(m * k, 6).reshape(m, k)
    y = orc.matmul(B.Q4_K, w, n, k, orc.F32, x, m)
    for r in range(m):
        assert np.array_equal(y[r], orc.matvec(B.Q4_K, w, n, k, orc.F32, x[r]))


# ---- split-scale operator API (backend/src/cuda_quant.rs) -------------------

def test_split_packed_4bit_reference_test(orc):
    # cuda_quant.rs:345-353: [0x88, 0x88], scale 1, block 4 -> -8 x4
    assert orc.dequantize_split(False, np.uint8([0x88, 0x88]), np.float32([1.0]), 4, 4).tolist() == [-8.0] * 4


def test_split_quantized_matmul_reference_test(orc):
    # cuda_quant.rs:355-373 (the reference checks the length only); the values
    # follow from B = dequant([0x11,0x11], 1.0, block 4) = [[1,1],[1,1]]
    c = orc.quantized_matmul_split(np.float32([1, 2, 3, 4]), np.uint8([0x11, 0x11]), np.float32([1.0]), 2, 2, 2, False, 4)
    assert c.size == 4 and c.reshape(-1).tolist() == [3.0, 3.0, 7.0, 7.0]


def test_split_uncovered_outputs_are_zero(orc):
    out = orc.dequantize_split(True, np.int8([1, -2, 3]).view(np.uint8), np.float32([2.0]), 4, 10)
    assert out.tolist() == [2.0, -4.0, 6.0] + [0.0] * 7


# ---- MoE (models/src/moe_fused.rs) ----------------------------------------

def test_select_top_k_reference_test(orc):
    # moe_fused.rs:326-337
    ids, w = orc.moe_select_top_k(np.float32([[0.1, 2.0, 1.0, -1.0], [3.0, 0.0, 1.5, 1.0]]), 2)
    assert ids.tolist() == [[1, 2], [0, 2]]
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_select_top_k_is_renormalised_softmax(orc):
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((50, 8)).astype(np.float32)
    ids, w = orc.moe_select_top_k(logits, 2)
    full = np.exp(logits.astype(np.float64) - logits.max(axis=1, keepdims=True))
    full /= full.sum(axis=1, keepdims=True)
    for r in range(50):
        order = sorted(range(8), key=lambda e: (-logits[r, e], e))[:2]
        assert ids[r].tolist() == order
        p = full[r, order] / full[r, order].sum()
        assert np.allclose(w[r], p, rtol=1e-6)


def test_select_top_k_ties_keep_index_order_and_clamp(orc):
    ids, w = orc.moe_select_top_k(np.float32([[1.0, 3.0, 3.0, 0.0]]), 9)   # k clamps to 4
    assert ids.tolist() == [[1, 2, 0, 3]]
    ids, _ = orc.moe_select_top_k(np.float32([[1.0, 3.0]]), 0)             # k clamps to 1
    assert ids.tolist() == [[1]]


def test_batch_by_expert(orc):
    ids = np.int32([[1, 0], [1, 2], [0, 1]])
    w = np.float32([[0.6, 0.4], [0.7, 0.3], [0.5, 0.5]])
    off, tok, wts = orc.moe_batch_by_expert(ids, w, 4)
    assert off.tolist() == [0, 2, 5, 6, 6]
    assert tok.tolist() == [0, 2, 0, 1, 2, 1]
    assert np.allclose(wts, [0.4, 0.5, 0.6, 0.7, 0.5, 0.3])


def test_dispatch_experts_reference_test(orc):
    # moe_fused.rs:351-395
    x = np.float32([[1, 2, 3], [4, 5, 6]])
    out = orc.moe_dispatch(x, 2, np.int32([[0], [1]]), np.float32([[1.0], [1.0]]), [lambda a: a * 2, lambda a: a * 3])
    assert out.reshape(-1).tolist() == [2, 4, 6, 12, 15, 18]


def test_dispatch_matches_naive_per_token(orc):
    # moe_fused.rs:433-516: batched dispatch == per-token naive loop
    x = (np.arange(512, dtype=np.float32) % 13.0 / 13.0).reshape(32, 16)
    fns = [lambda a, s=s: a * s for s in (2.0, 3.0, 4.0, 5.0)]
    ids = np.int32([[t % 4, (t + 1) % 4] for t in range(32)])
    w = np.tile(np.float32([0.7, 0.3]), (32, 1))
    out = orc.moe_dispatch(x, 4, ids, w, fns)
    naive = np.zeros_like(x)
    for t in range(32):
        for e, wt in sorted(zip(ids[t], w[t]), key=lambda p: p[0]):
            naive[t] = naive[t] + (fns[e](x[t:t + 1])[0] * wt).astype(np.float32)
    assert np.allclose(out, naive, atol=1e-6)


def test_moe_ffn_literal_equals_dispatch_with_fused_ffn(orc):
    # orc_moe_ffn (act f32) == dispatch_experts with fused_ffn built from the
    # oracle's matmul and the elementwise SiLU*up, computed independently
    from barq_rocm import synth
    import barq_rocm as B
    ne, hid, nff, rows = 3, 256, 512, 6
    gates = [synth.gen_q4_k(nff, hid, 10 + e) for e in range(ne)]
    ups = [synth.gen_q4_k(nff, hid, 20 + e) for e in range(ne)]
    downs = [synth.gen_q6_k(hid, nff, 30 + e) for e in range(ne)]
    x = synth.gen_f32(rows * hid, 40).reshape(rows, hid)
    ids, w = orc.moe_select_top_k(synth.gen_f32(rows * ne, 41).reshape(rows, ne), 2)
    out = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x, ids, w, orc.F32)

    def ffn(e):
        def f(a):
            g = orc.matmul(B.Q4_K, gates[e], nff, hid, orc.F32, a, a.shape[0])
            u = orc.matmul(B.Q4_K, ups[e], nff, hid, orc.F32, a, a.shape[0])
            with np.errstate(over="ignore"):
                h = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32) * u
            return orc.matmul(B.Q6_K, downs[e], hid, nff, orc.F32, h.astype(np.float32), a.shape[0])
        return f
    ref = orc.moe_dispatch(x, ne, ids, w, [ffn(e) for e in range(ne)])
    assert_close_1e3(out, ref, tol=1e-5)
