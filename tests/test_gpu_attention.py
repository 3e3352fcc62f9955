"""GPU parity of RoPE, the device KV cache and attention against the oracle
(models/src/transformer.rs:176-374, models/src/context.rs:245-340).

Bars:
  - transpose_heads, KV-cache appends and reads: bit-exact.
  - RoPE: within 2e-6 * max|x| of the oracle (the device's sincosf against
    glibc's sinf/cosf, a few ulp apart).
  - attention: max |out - ref| <= 2e-5 * max|V| (outputs are convex
    combinations of V rows; the device sums in a different order and takes
    base-2 exponentials of pre-scaled scores).
"""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import attention as A

pytestmark = pytest.mark.gpu
F32 = np.float32


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def inv_freq(hd, base=500000.0):
    return np.array([np.float32(base) ** np.float32(-2.0 * i / hd) for i in range(hd // 2)], dtype=F32)


def rng_f32(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape).astype(F32)


@pytest.mark.parametrize("layout", [A.ROPE_INTERLEAVED, A.ROPE_SPLIT_HALF])
@pytest.mark.parametrize("seq,heads,hd,start", [(1, 32, 128, 4095), (7, 8, 128, 0), (33, 4, 64, 100000),
                                                (2, 3, 256, 17), (5, 2, 4, 1)])
def test_rope_matches_oracle(be, orc, layout, seq, heads, hd, start):
    x = rng_f32(seq * 31 + hd, seq, heads * hd)
    f = inv_freq(hd)
    ref = orc.rope(x, seq, heads, hd, start, 1.0, f, layout)
    got = A.apply_rope(be, dev(x), seq, heads, hd, start, 1.0, dev(f), layout).cpu().numpy()
    assert np.max(np.abs(got - ref)) <= 2e-6 * np.max(np.abs(x))
    host = A.apply_rope(be, x, seq, heads, hd, start, 1.0, f, layout, mem=B.MEM_HOST)
    assert np.array_equal(host, got)


def test_rope_reference_known_answers(be):
    # transformer.rs:623-684 on the device
    x = np.array([1.0, 2.0, 3.0, 4.0], dtype=F32)
    f = np.array([1.0, np.float32(10000.0) ** np.float32(-0.5)], dtype=F32)
    s0, c0, s1, c1 = np.sin(f[0]), np.cos(f[0]), np.sin(f[1]), np.cos(f[1])
    r0 = A.apply_rope(be, x, 1, 1, 4, 0, 1.0, f, A.ROPE_INTERLEAVED, mem=B.MEM_HOST).ravel()
    assert np.allclose(r0, x, atol=1e-6)
    r = A.apply_rope(be, x, 1, 1, 4, 1, 1.0, f, A.ROPE_INTERLEAVED, mem=B.MEM_HOST).ravel()
    assert np.allclose(r, [c0 - 2 * s0, s0 + 2 * c0, 3 * c1 - 4 * s1, 3 * s1 + 4 * c1], atol=1e-6)
    r = A.apply_rope(be, x, 1, 1, 4, 1, 1.0, f, A.ROPE_SPLIT_HALF, mem=B.MEM_HOST).ravel()
    assert np.allclose(r, [c0 - 3 * s0, 2 * c1 - 4 * s1, s0 + 3 * c0, 2 * s1 + 4 * c1], atol=1e-6)


def test_transpose_heads_bit_exact(be, orc):
    x = rng_f32(5, 9, 4 * 64)
    got = A.transpose_heads(be, dev(x), 9, 4, 64).cpu().numpy()
    assert np.array_equal(got, orc.transpose_heads(x, 9, 4, 64))
    assert np.array_equal(A.transpose_heads(be, x, 9, 4, 64, mem=B.MEM_HOST), got)


def test_kv_cache_semantics(be):
    n_kv, hd = 2, 64
    c = A.KVCache(be, 16, 3, n_kv, hd)
    assert c.size() == 0
    k0, v0 = rng_f32(1, n_kv, 5, hd), rng_f32(2, n_kv, 5, hd)
    c.append(0, dev(k0), dev(v0), 5, hd)
    k1, v1 = rng_f32(3, n_kv, 4, hd), rng_f32(4, n_kv, 4, hd)
    c.append(1, k1, v1, 4, hd, mem=B.MEM_HOST)
    assert c.size() == 5 and c.layer_len(0) == 5 and c.layer_len(1) == 4   # only layer 0 moves size
    c.append(7, k1, v1, 4, hd, mem=B.MEM_HOST)                           # out-of-range layer: ignored
    assert c.size() == 5
    k2, v2 = rng_f32(5, n_kv, 3, hd), rng_f32(6, n_kv, 3, hd)
    c.append(0, dev(k2), dev(v2), 3, hd)
    for h in range(n_kv):
        kh, vh = c.get_head(0, h)
        assert np.array_equal(kh, np.concatenate([k0[h], k2[h]]))
        assert np.array_equal(vh, np.concatenate([v0[h], v2[h]]))
        kh, vh = c.get_head(1, h)
        assert np.array_equal(kh, k1[h]) and np.array_equal(vh, v1[h])
    with pytest.raises(B.BarqError) as e:
        c.append(0, rng_f32(7, n_kv, 9, hd), rng_f32(8, n_kv, 9, hd), 9, hd, mem=B.MEM_HOST)
    assert e.value.code == B._lib.E_INVALID
    with pytest.raises(B.BarqError) as e:
        c.append(0, k2, v2, 3, 32, mem=B.MEM_HOST)
    assert e.value.code == B._lib.E_DIM
    c.clear()
    assert c.size() == 0 and c.layer_len(1) == 0
    c.close()


@pytest.mark.parametrize("layout", [A.ROPE_INTERLEAVED, A.ROPE_SPLIT_HALF])
def test_append_rope_equals_rope_then_append(be, layout):
    n_kv, hd, n = 4, 128, 6
    f = inv_freq(hd)
    kp, vp = rng_f32(11, n, n_kv * hd), rng_f32(12, n, n_kv * hd)
    c1 = A.KVCache(be, 32, 2, n_kv, hd)
    c2 = A.KVCache(be, 32, 2, n_kv, hd)
    for layer in range(2):
        c1.append_rope(layer, dev(kp), dev(vp), n, 3, 1.0, dev(f), layout)
        kr = A.apply_rope(be, dev(kp), n, n_kv, hd, 3, 1.0, dev(f), layout)
        vt = A.transpose_heads(be, dev(vp), n, n_kv, hd)
        c2.append(layer, kr, vt, n, hd)
    c1.append_rope(1, kp, vp, n, 3 + n, 1.0, f, layout, mem=B.MEM_HOST)
    kr = A.apply_rope(be, dev(kp), n, n_kv, hd, 3 + n, 1.0, dev(f), layout)
    c2.append(1, kr, A.transpose_heads(be, dev(vp), n, n_kv, hd), n, hd)
    assert c1.size() == c2.size() == n and c1.layer_len(1) == 2 * n
    for layer in range(2):
        for h in range(n_kv):
            a, b = c1.get_head(layer, h), c2.get_head(layer, h)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


ATTN_CASES = [
    # n_head, n_kv, hd, q_len, kv_len, start_pos, cache positions
    (32, 8, 128, 1, 4096, 4095, 4096),    # Llama-3-8B decode
    (32, 8, 128, 1, 1, 0, 1),
    (32, 8, 128, 1, 63, 62, 63),
    (32, 8, 128, 1, 65, 64, 80),
    (32, 8, 128, 1, 1000, 999, 1000),
    (32, 8, 128, 1, 4097, 4096, 4100),    # one position past 4096: a short last split
    (32, 8, 128, 1, 20000, 19999, 20000),
    (8, 8, 64, 1, 300, 299, 300),         # no grouping
    (16, 2, 128, 1, 700, 699, 700),       # 8 query heads per kv head
    (12, 6, 128, 1, 500, 499, 512),       # 2 per kv head
    (6, 4, 128, 1, 129, 128, 129),        # irregular grouping (kv = h * 4 / 6)
    (8, 2, 256, 1, 517, 516, 517),
    (32, 8, 128, 7, 40, 33, 40),          # a chunk of 7 new tokens
    (4, 2, 64, 16, 16, 0, 16),            # a prompt from position 0
    (8, 2, 128, 3, 10, 2, 10),            # start_pos + q_len < kv_len: masked tail
    (8, 2, 128, 1, 50, 49, 80),           # kv_len below the layer length
    # prompt chunks of 32+ rows (head_dim 128: the MFMA kernel)
    (32, 8, 128, 32, 32, 0, 32),          # one query block from position 0
    (32, 8, 128, 100, 150, 50, 160),      # ragged last block, chunk after a prefix
    (8, 2, 128, 64, 64, 0, 64),
    (12, 6, 128, 40, 300, 260, 300),      # 2 per kv head
    (6, 4, 128, 33, 33, 0, 40),           # irregular grouping
    (8, 2, 128, 40, 100, 20, 100),        # start_pos + q_len < kv_len: masked tail
    (32, 8, 128, 512, 512, 0, 512),       # a Llama-3-8B prompt of 512 tokens
    (32, 8, 128, 768, 768, 0, 768),       # pieces of 6 position blocks, two workgroups per CU
    (32, 8, 128, 200, 1000, 800, 1000),   # a chunk after a long prefix: every query block in pieces
    (4, 2, 64, 48, 48, 0, 48),            # head_dim 64 stays on the split kernel
    (32, 32, 128, 512, 512, 0, 512),      # query blocks paired (long + short) per workgroup
    (64, 64, 128, 288, 300, 12, 300),     # paired, odd block count (the middle block alone)
]


def fill_cache(be, n_kv, hd, pos, seed, layers=2, layer=1):
    k = rng_f32(seed, n_kv, pos, hd)
    v = rng_f32(seed + 1, n_kv, pos, hd)
    c = A.KVCache(be, pos + 5, layers, n_kv, hd)
    c.append(0, dev(k), dev(v), pos, hd)
    c.append(layer, dev(k), dev(v), pos, hd)
    return c, k, v


@pytest.mark.parametrize("n_head,n_kv,hd,q_len,kv_len,start,pos", ATTN_CASES)
def test_attention_matches_oracle(be, orc, n_head, n_kv, hd, q_len, kv_len, start, pos):
    c, k, v = fill_cache(be, n_kv, hd, pos, n_head * 7 + kv_len)
    q = rng_f32(kv_len + 3, n_head, q_len, hd)
    print(f"attention case n_head={n_head} n_kv={n_kv} hd={hd} q_len={q_len} kv_len={kv_len} start={start}",
          flush=True)
    got = A.compute_attention(be, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start).cpu().numpy()
    ref = orc.attention(q, k, v, n_head, q_len, kv_len, start)
    err = np.max(np.abs(got - ref))
    assert err <= 2e-5 * np.max(np.abs(v)), err
    host = A.compute_attention(be, q, c, 1, n_head, n_kv, hd, q_len, kv_len, start, mem=B.MEM_HOST)
    assert np.array_equal(host, got)
    c.close()


def test_attention_argument_errors(be):
    c, k, v = fill_cache(be, 2, 128, 20, 3)
    q = rng_f32(1, 4, 1, 128)
    with pytest.raises(B.BarqError) as e:
        A.compute_attention(be, q, c, 1, 4, 2, 128, 1, 21, 20, mem=B.MEM_HOST)
    assert e.value.code == B._lib.E_DIM
    with pytest.raises(B.BarqError) as e:
        A.compute_attention(be, q, c, 1, 4, 4, 128, 1, 20, 19, mem=B.MEM_HOST)
    assert e.value.code == B._lib.E_DIM
    c.close()
    c80 = A.KVCache(be, 8, 1, 1, 80)
    c80.append(0, rng_f32(2, 1, 4, 80), rng_f32(3, 1, 4, 80), 4, 80, mem=B.MEM_HOST)
    with pytest.raises(B.BarqError) as e:
        A.compute_attention(be, rng_f32(4, 1, 1, 80), c80, 0, 1, 1, 80, 1, 4, 3, mem=B.MEM_HOST)
    assert e.value.code == B._lib.E_UNSUPPORTED
    c80.close()


@pytest.mark.parametrize("layout", [A.ROPE_INTERLEAVED, A.ROPE_SPLIT_HALF])
@pytest.mark.parametrize("n_head,n_kv,hd,n", [(32, 8, 128, 1), (8, 2, 128, 6), (6, 4, 64, 3), (4, 2, 256, 2)])
def test_append_rope_q_equals_separate_steps(be, layout, n_head, n_kv, hd, n):
    """The fused q/k RoPE + cache append is bit-identical to barq_rocm_rope on q
    then append_rope on k and v (device and host buffers, an out-of-range
    layer that still rotates q)."""
    f = inv_freq(hd)
    qp, kp, vp = rng_f32(21, n, n_head * hd), rng_f32(22, n, n_kv * hd), rng_f32(23, n, n_kv * hd)
    c1 = A.KVCache(be, 40, 2, n_kv, hd)
    c2 = A.KVCache(be, 40, 2, n_kv, hd)
    for layer in range(2):
        q1 = c1.append_rope_q(layer, dev(qp), n_head, dev(kp), dev(vp), n, 5, 1.0, dev(f), layout)
        be.sync()
        q2 = A.apply_rope(be, dev(qp), n, n_head, hd, 5, 1.0, dev(f), layout)
        c2.append_rope(layer, dev(kp), dev(vp), n, 5, 1.0, dev(f), layout)
        assert np.array_equal(q1.cpu().numpy(), q2.cpu().numpy())
    qh = c1.append_rope_q(1, qp, n_head, kp, vp, n, 5 + n, 1.0, f, layout, mem=B.MEM_HOST)
    c2.append_rope(1, dev(kp), dev(vp), n, 5 + n, 1.0, dev(f), layout)
    q2 = A.apply_rope(be, dev(qp), n, n_head, hd, 5 + n, 1.0, dev(f), layout)
    assert np.array_equal(qh, q2.cpu().numpy())
    q3 = c1.append_rope_q(7, dev(qp), n_head, dev(kp), dev(vp), n, 9, 1.0, dev(f), layout)   # layer out of range
    be.sync()
    assert np.array_equal(q3.cpu().numpy(), A.apply_rope(be, dev(qp), n, n_head, hd, 9, 1.0, dev(f), layout).cpu().numpy())
    assert c1.size() == c2.size() == n and c1.layer_len(1) == c2.layer_len(1) == 2 * n
    for layer in range(2):
        for h in range(n_kv):
            a, b = c1.get_head(layer, h), c2.get_head(layer, h)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    c1.close()
    c2.close()


@pytest.mark.parametrize("n_head,n_kv,hd,q_len,kv_len,start,pos", [
    (32, 8, 128, 1, 4096, 4095, 4096),    # decode: the merge writes Q8_K blocks
    (32, 8, 128, 1, 40, 39, 40),          # one split: attention, then the quantizer
    (32, 8, 128, 7, 300, 293, 300),       # a chunk of 7 rows
    (32, 8, 128, 40, 100, 60, 100),       # a prompt chunk on the MFMA kernel
    (8, 2, 64, 1, 1000, 999, 1000),       # head_dim 64: four heads per block
    (4, 2, 256, 1, 517, 516, 517),        # head_dim 256: one head per block
    (8, 1, 64, 1, 20000, 19999, 20000),   # 157 splits (test_attention_q8k_many_splits: more than the merge's threads)
])
def test_attention_q8k_equals_quantized_attention(be, n_head, n_kv, hd, q_len, kv_len, start, pos):
    """attention_q8k writes the bytes quantize_act(Q8_K) writes for the f32
    attention rows, whichever path (merge kernel or quantizer after) runs."""
    c, k, v = fill_cache(be, n_kv, hd, pos, n_head * 3 + kv_len)
    q = rng_f32(kv_len + 5, n_head, q_len, hd)
    print(f"attention_q8k case n_head={n_head} hd={hd} q_len={q_len} kv_len={kv_len}", flush=True)
    y = A.compute_attention(be, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start)
    ref = be.quantize_act(B.Q8_K, y.reshape(q_len, n_head * hd)).cpu().numpy().reshape(-1)
    got = A.compute_attention_q8k(be, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start).cpu().numpy().reshape(-1)
    assert np.array_equal(got, ref)
    host = A.compute_attention_q8k(be, q, c, 1, n_head, n_kv, hd, q_len, kv_len, start, mem=B.MEM_HOST)
    assert np.array_equal(host.reshape(-1), ref)
    c.close()


def test_attention_prompt_pieces_random_shapes(be, orc):
    """Prompt chunks of seeded random lengths after random cached prefixes
    (some with a masked tail: start_pos + q_len < kv_len) on the MFMA prompt
    kernel, whose pieces per query block follow the launch simulation's chunk:
    the f32 rows against the oracle, and the Q8_K merge against quantizing
    them."""
    rng = np.random.default_rng(2024)
    for case in range(10):
        n_head, n_kv = [(8, 2), (12, 6), (16, 4), (32, 8)][case % 4]
        hd = 128
        q_len = int(rng.integers(32, 200))
        prefix = int(rng.integers(0, 400))
        kv_len = prefix + q_len
        start = prefix if case % 3 else max(0, prefix - int(rng.integers(1, 40)))
        print(f"prompt pieces case {case}: n_head={n_head} n_kv={n_kv} q_len={q_len} kv_len={kv_len} "
              f"start={start}", flush=True)
        c, k, v = fill_cache(be, n_kv, hd, kv_len, 900 + case)
        q = rng_f32(950 + case, n_head, q_len, hd)
        y = A.compute_attention(be, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start)
        ref = orc.attention(q, k, v, n_head, q_len, kv_len, start)
        err = np.max(np.abs(y.cpu().numpy() - ref))
        assert err <= 2e-5 * np.max(np.abs(v)), (case, err)
        if (n_head * hd) % 256 == 0:
            q8 = A.compute_attention_q8k(be, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start)
            want = be.quantize_act(B.Q8_K, y.reshape(q_len, n_head * hd)).cpu().numpy().reshape(-1)
            assert np.array_equal(q8.cpu().numpy().reshape(-1), want), case
        c.close()


def test_attention_q8k_argument_errors(be):
    c, k, v = fill_cache(be, 2, 64, 20, 3)
    q = rng_f32(1, 3, 1, 64)
    with pytest.raises(B.BarqError):   # 3 * 64 is not a multiple of 256
        A.compute_attention_q8k(be, dev(q), c, 1, 3, 2, 64, 1, 20, 19)
    c.close()


@pytest.mark.parametrize("n_head,n_kv,q_len,kv_len,start,pos", [
    (32, 8, 1, 300, 299, 300),    # a decode row on the MFMA kernel
    (32, 8, 7, 40, 33, 40),       # a short chunk: one block, 25 rows unused
    (8, 2, 16, 16, 0, 16),
    (12, 6, 3, 10, 2, 10),        # masked tail
])
def test_attention_mfma_kernel_small_chunks(be, orc, n_head, n_kv, q_len, kv_len, start, pos):
    """The MFMA prompt kernel with its threshold lowered (BARQ_ATTN_MFMA_MIN_Q,
    read at handle creation) on chunks shorter than a query block."""
    import os
    hd = 128
    c, k, v = fill_cache(be, n_kv, hd, pos, n_head * 5 + kv_len)
    q = rng_f32(kv_len + 9, n_head, q_len, hd)
    old = os.environ.get("BARQ_ATTN_MFMA_MIN_Q")
    os.environ["BARQ_ATTN_MFMA_MIN_Q"] = "1"
    try:
        b2 = B.Backend(0)
    finally:
        if old is None:
            os.environ.pop("BARQ_ATTN_MFMA_MIN_Q", None)
        else:
            os.environ["BARQ_ATTN_MFMA_MIN_Q"] = old
    try:
        got = A.compute_attention(b2, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start).cpu().numpy()
        got_q8 = A.compute_attention_q8k(b2, dev(q), c, 1, n_head, n_kv, hd, q_len, kv_len, start).cpu().numpy()
        ref_q8 = b2.quantize_act(B.Q8_K, dev(got.reshape(q_len, n_head * hd))).cpu().numpy()
    finally:
        b2.close()
    ref = orc.attention(q, k, v, n_head, q_len, kv_len, start)
    assert np.max(np.abs(got - ref)) <= 2e-5 * np.max(np.abs(v))
    assert np.array_equal(got_q8.reshape(-1), ref_q8.reshape(-1))
    c.close()


@pytest.mark.parametrize("hd,kv_len", [(128, 40000), (64, 20000)])
def test_attention_q8k_many_splits(be, hd, kv_len):
    """More splits than the Q8_K merge's threads per head (512 at head_dim
    128, 256 at 64; 625 and 313 splits with BARQ_ATTN_WG=2048, read at handle
    creation): the merge still writes the bytes the f32 merge's rows quantize
    to."""
    import os
    n_head, n_kv = 8, 1
    print(f"attention_q8k many splits hd={hd} kv_len={kv_len}", flush=True)
    c, k, v = fill_cache(be, n_kv, hd, kv_len, 77)
    q = rng_f32(78, n_head, 1, hd)
    old = os.environ.get("BARQ_ATTN_WG")
    os.environ["BARQ_ATTN_WG"] = "2048"
    try:
        b2 = B.Backend(0)
    finally:
        if old is None:
            os.environ.pop("BARQ_ATTN_WG", None)
        else:
            os.environ["BARQ_ATTN_WG"] = old
    try:
        y = A.compute_attention(b2, dev(q), c, 1, n_head, n_kv, hd, 1, kv_len, kv_len - 1)
        ref = b2.quantize_act(B.Q8_K, y.reshape(1, n_head * hd)).cpu().numpy().reshape(-1)
        got = A.compute_attention_q8k(b2, dev(q), c, 1, n_head, n_kv, hd, 1, kv_len, kv_len - 1).cpu().numpy()
    finally:
        b2.close()
    assert np.array_equal(got.reshape(-1), ref)
    c.close()
