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


@pytest.mark.parametrize("bs", [5, 7, 3])
def test_split_packed_4bit_odd_block_size_placement(orc, bs):
    # cuda_quant.rs:44-75: block b's quants start div_ceil(bs, 2) bytes after
    # block b-1's; an odd block leaves the high nibble of its last byte unused.
    # One nibble at a time is set to 3: it must land on exactly the element the
    # byte-to-element map gives (or on none for the padding nibble), scaled by
    # its block's scale.  A stride of bs // 2 bytes fails this.
    n_blocks = 4
    stride = (bs + 1) // 2
    n_out = n_blocks * bs
    scales = np.float32([1.0, 2.0, -0.5, 4.0])
    for j in range(n_blocks * stride):
        for shift in (0, 4):
            q = np.zeros(n_blocks * stride, np.uint8)
            q[j] = 3 << shift
            out = orc.dequantize_split(False, q, scales, bs, n_out)
            b, rel = j // stride, 2 * (j % stride) + shift // 4
            expect = np.zeros(n_out, np.float32)
            if rel < bs:
                expect[b * bs + rel] = 3.0 * scales[b]
            assert np.array_equal(out, expect), (bs, j, shift)


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


def test_reduce_experts_threshold_cap_and_renormalisation(orc):
    # moe_fused.rs:147-194, checked against closed forms rather than a retyped loop
    w = np.float32([[0.5, 0.3, 0.15, 0.05]])
    ids = np.int32([[3, 1, 0, 2]])
    # nothing below the threshold, cap above k: order kept, weights unchanged up to the
    # division by their float sum (exactly 1.0 here)
    oi, ow = orc.moe_reduce_experts(ids, w, 8, 0.0)
    assert oi.tolist() == [[3, 1, 0, 2]]
    assert np.float32(np.float32(np.float32(0.5 + np.float32(0.3)) + np.float32(0.15)) + np.float32(0.05)) == 1.0
    assert np.array_equal(ow, w)
    # the threshold drops the last two, the rest renormalise to 0.5/0.8, 0.3/0.8
    oi, ow = orc.moe_reduce_experts(ids, w, 8, 0.1)
    assert oi.tolist() == [[3, 1, 0, -1]]
    assert ow[0, 3] == 0.0
    oi, ow = orc.moe_reduce_experts(ids, w, 2, 0.1)          # the cap keeps the two largest
    assert oi.tolist() == [[3, 1, -1, -1]]
    assert np.allclose(ow[0, :2], [0.625, 0.375], rtol=1e-6, atol=0)
    oi, ow = orc.moe_reduce_experts(ids, w, 0, 0.0)          # max_active 0 keeps one (.max(1))
    assert oi.tolist() == [[3, -1, -1, -1]] and ow[0, 0] == 1.0


def test_reduce_experts_sorts_descending_and_stable(orc):
    # unsorted input is sorted by weight, equal weights keep slot order
    ids = np.int32([[4, 7, 2, 9, 5]])
    w = np.float32([[0.1, 0.3, 0.2, 0.3, 0.1]])
    oi, ow = orc.moe_reduce_experts(ids, w, 5, 0.0)
    assert oi.tolist() == [[7, 9, 2, 4, 5]]
    assert np.all(np.diff(ow[0]) <= 0)


def test_reduce_experts_all_below_threshold_keeps_the_last_maximum(orc):
    # Iterator::max_by returns the last of equal maxima (moe_fused.rs:165-171)
    ids = np.int32([[1, 2, 3], [6, 5, 4]])
    w = np.float32([[0.02, 0.04, 0.04], [0.03, 0.01, 0.02]])
    oi, ow = orc.moe_reduce_experts(ids, w, 2, 0.05)
    assert oi.tolist() == [[3, -1, -1], [6, -1, -1]]
    assert ow[:, 0].tolist() == [1.0, 1.0]


def test_reduce_experts_absent_slots_and_alias(orc):
    ids = np.int32([[-1, 2, -1, 0]])
    w = np.float32([[0.9, 0.3, 0.9, 0.7]])    # weights of absent slots are ignored
    oi, ow = orc.moe_reduce_experts(ids, w, 4, 0.0)
    assert oi.tolist() == [[0, 2, -1, -1]]
    assert np.allclose(ow, [[0.7, 0.3, 0.0, 0.0]], rtol=1e-6)
    oi2, ow2 = orc.moe_reduce_experts(oi, ow, 4, 0.0)        # reducing again changes nothing
    assert np.array_equal(oi2, oi) and np.allclose(ow2, ow, rtol=1e-6)


def test_reduce_experts_sum_is_floored_at_epsilon(orc):
    ids = np.int32([[0, 1]])
    w = np.float32([[0.0, 0.0]])
    oi, ow = orc.moe_reduce_experts(ids, w, 2, 0.0)
    assert oi.tolist() == [[0, 1]] and ow.tolist() == [[0.0, 0.0]]
    w = np.float32([[1e-8, 0.0]])              # 1e-8 / EPSILON, not 1e-8 / 1e-8
    oi, ow = orc.moe_reduce_experts(ids, w, 2, 0.0)
    assert ow[0, 0] == np.float32(np.float32(1e-8) / np.float32(1.1920929e-7))


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


def test_moe_ffn_q8k_equals_dispatch_with_quantized_ffn(orc):
    # orc_moe_ffn (act Q8_K, the GPU's integer path) == dispatch_experts with an
    # expert built from independent pieces: Q8_K rows by quantize_q8_k, the
    # Q8_K matmul, SiLU as ops.rs:191-211 computes it (x / (1 + exp(-x)), with
    # the same libm expf the oracle links), the up product, Q8_K again, down.
    # Bit-equal.
    import ctypes
    from barq_rocm import synth
    import barq_rocm as B
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    ne, hid, nff, rows = 3, 256, 512, 5
    gates = [synth.gen_q4_k(nff, hid, 110 + e) for e in range(ne)]
    ups = [synth.gen_q4_k(nff, hid, 120 + e) for e in range(ne)]
    downs = [synth.gen_q6_k(hid, nff, 130 + e) for e in range(ne)]
    x = synth.gen_f32(rows * hid, 140).reshape(rows, hid)
    ids, w = orc.moe_select_top_k(synth.gen_f32(rows * ne, 141).reshape(rows, ne), 2)
    out = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x, ids, w, orc.Q8_K)

    def ffn(e):
        def f(a):
            r = a.shape[0]
            xq = np.concatenate([orc.quantize_q8_k(a[i]) for i in range(r)])
            g = orc.matmul(B.Q4_K, gates[e], nff, hid, orc.Q8_K, xq, r).reshape(-1)
            u = orc.matmul(B.Q4_K, ups[e], nff, hid, orc.Q8_K, xq, r).reshape(-1)
            ex = np.float32([libm.expf(float(-v)) for v in g])
            h = (g / (np.float32(1.0) + ex)) * u
            hq = np.concatenate([orc.quantize_q8_k(h[i * nff:(i + 1) * nff]) for i in range(r)])
            return orc.matmul(B.Q6_K, downs[e], hid, nff, orc.Q8_K, hq, r)
        return f
    ref = orc.moe_dispatch(x, ne, ids, w, [ffn(e) for e in range(ne)])
    assert np.array_equal(out.view(np.uint32), ref.astype(np.float32).view(np.uint32))


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


# ---- the timed CPU baseline (oracle/cpu_baseline.c) is the reference arithmetic ----

def test_cpu_baseline_literal_equals_gemm_f32(orc):
    # variant (i), blas.rs:199-210 at M = 1: bit-exact with the oracle's gemm_f32
    rng = np.random.default_rng(3)
    k, n = 640, 300
    x = rng.standard_normal(k).astype(np.float32)
    w_t = rng.standard_normal((k, n)).astype(np.float32)
    y = np.zeros(n, np.float32)
    orc.cpub_gemm_literal_m1(x, w_t, k, n, 0, 170, y)
    orc.cpub_gemm_literal_m1(x, w_t, k, n, 170, n, y)
    ref = orc.gemm_f32(x, w_t.reshape(-1), 1, k, n).reshape(-1)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_cpu_baseline_simd_dot_matches_gemv_f32(orc, threads):
    # variants (ii)/(iii), simd.rs:115-168: an FMA-blocked dot, so equal to the
    # sequential gemv_f32 only to float rounding; the threaded form computes
    # the same rows bit for bit
    rng = np.random.default_rng(4)
    m, n = 257, 1000            # n not a multiple of the vector width: the scalar tail runs
    a = rng.standard_normal((m, n)).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    ref = orc.gemv_f32(a.reshape(-1), x, m, n)
    y1 = np.zeros(m, np.float32)
    orc.cpub_gemv_simd(a, x, n, 0, m, y1)
    bound = 4 * n * np.finfo(np.float32).eps * (np.abs(a) @ np.abs(x))
    assert np.all(np.abs(y1.astype(np.float64) - ref) <= bound)
    y2 = np.zeros(m, np.float32)
    used = orc.cpub_gemv_simd_threaded(a, x, n, 0, m, y2, threads)
    assert used == threads
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_cpu_baseline_gemm_rows_equals_gemm_f32(orc, threads):
    # the C4 leg: gemm_f32 at M > 1 (blas.rs:193-212), rows split over
    # threads, bit-exact with the oracle's gemm_f32 whatever the split
    rng = np.random.default_rng(6)
    m, k, n = 11, 300, 257
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    ref = orc.gemm_f32(a, b, m, k, n)
    c = np.zeros((m, n), np.float32)
    used = orc.cpub_gemm_rows_threaded(a, b, k, n, 0, m, c, threads)
    per = -(-m // threads)                 # rows per range, as the split makes them
    assert used == -(-m // per)
    assert np.array_equal(c.view(np.uint32), ref.view(np.uint32))
    c1 = np.zeros((m, n), np.float32)
    orc.cpub_gemm_rows(a, b, k, n, 3, 7, c1)
    assert np.array_equal(c1[3:7].view(np.uint32), ref[3:7].view(np.uint32))


def test_cpu_baseline_moe_expert_equals_oracle_moe(orc):
    import barq_rocm as B
    from barq_rocm import synth
    # the C5 leg: one expert's fused_ffn over f32 weights transposed at load
    # equals the oracle's F32 MoE (moe_fused.rs:84-92, 226-308) for tokens
    # routed to that expert alone with weight 1 (out = 0 + 1 * y), bit for bit
    hid, nff, rows = 256, 512, 3
    gate = synth.gen_weights(B.Q4_K, nff, hid, 31)
    up = synth.gen_weights(B.Q4_K, nff, hid, 32)
    down = synth.gen_weights(B.Q6_K, hid, nff, 33)
    x = synth.gen_f32(rows * hid, 34).reshape(rows, hid)
    ref = orc.moe_ffn(B.Q4_K, [gate], B.Q4_K, [up], B.Q6_K, [down], hid, nff, x, np.zeros((rows, 1), np.int32),
                      np.ones((rows, 1), np.float32), orc.F32)
    gt = np.ascontiguousarray(orc.dequantize(B.Q4_K, gate, nff * hid).reshape(nff, hid).T)
    ut = np.ascontiguousarray(orc.dequantize(B.Q4_K, up, nff * hid).reshape(nff, hid).T)
    dt = np.ascontiguousarray(orc.dequantize(B.Q6_K, down, hid * nff).reshape(hid, nff).T)
    g = np.empty((rows, nff), np.float32)
    u = np.empty_like(g)
    out = np.empty((rows, hid), np.float32)
    orc.cpub_moe_expert_ffn(x, rows, hid, nff, gt, ut, dt, g, u, out)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
