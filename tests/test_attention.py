"""CPU pins of the attention oracle (oracle/barq_oracle.c orc_rope,
orc_transpose_heads, orc_attention) and the host logic of the attention
plumbing.

What pins each function:
  - orc_rope: the reference's own known-answer tests
    (models/src/transformer.rs:623-684: position 0 is the identity; position
    1 rotates pair i by inv_freq[i], consecutive pairs or split halves), and
    a float64 rotation of random rows at large positions.
  - orc_transpose_heads: exact index identity.
  - orc_attention: closed forms (one visible position -> V[0] exactly;
    identical keys -> the mean of V; the causal row 0 sees only position 0;
    a shift of all scores changes nothing) and a float64 brute force that
    restates the GQA mapping, the mask and the softmax independently.
A planted mistake (mask off by one, wrong kv head) fails the brute force; see
test_brute_force_catches_planted_mistakes.
"""
import math

import numpy as np
import pytest

F32 = np.float32


def inv_freq(hd, base=10000.0):
    # transformer.rs:52-54: base.powf(-2 i / head_dim) in f32
    return np.array([np.float32(base) ** np.float32(-2.0 * i / hd) for i in range(hd // 2)], dtype=F32)


# ---- RoPE: the reference's own tests -------------------------------------------------
def test_rope_consecutive_pairs_reference_test(orc):
    # transformer.rs:623-661
    x = np.array([1.0, 2.0, 3.0, 4.0], dtype=F32)
    f = np.array([1.0, np.float32(10000.0) ** np.float32(-1.0 / 2.0)], dtype=F32)
    out = orc.rope(x, 1, 1, 4, 0, 1.0, f, 0).ravel()
    assert np.allclose(out, [1.0, 2.0, 3.0, 4.0], atol=1e-6)
    r = orc.rope(x, 1, 1, 4, 1, 1.0, f, 0).ravel()
    s0, c0 = math.sin(f[0]), math.cos(f[0])
    s1, c1 = math.sin(f[1]), math.cos(f[1])
    assert abs(r[0] - (1.0 * c0 - 2.0 * s0)) < 1e-6
    assert abs(r[1] - (1.0 * s0 + 2.0 * c0)) < 1e-6
    assert abs(r[2] - (3.0 * c1 - 4.0 * s1)) < 1e-6
    assert abs(r[3] - (3.0 * s1 + 4.0 * c1)) < 1e-6


def test_rope_split_half_reference_test(orc):
    # transformer.rs:663-684
    x = np.array([1.0, 2.0, 3.0, 4.0], dtype=F32)
    f = np.array([1.0, np.float32(10000.0) ** np.float32(-1.0 / 2.0)], dtype=F32)
    r = orc.rope(x, 1, 1, 4, 1, 1.0, f, 1).ravel()
    s0, c0 = math.sin(f[0]), math.cos(f[0])
    s1, c1 = math.sin(f[1]), math.cos(f[1])
    assert abs(r[0] - (1.0 * c0 - 3.0 * s0)) < 1e-6
    assert abs(r[2] - (1.0 * s0 + 3.0 * c0)) < 1e-6
    assert abs(r[1] - (2.0 * c1 - 4.0 * s1)) < 1e-6
    assert abs(r[3] - (2.0 * s1 + 4.0 * c1)) < 1e-6


@pytest.mark.parametrize("layout", [0, 1])
def test_rope_is_a_rotation_at_large_positions(orc, layout):
    rng = np.random.default_rng(7 + layout)
    seq, heads, hd, start = 5, 3, 64, 100000
    x = rng.standard_normal((seq, heads * hd)).astype(F32)
    f = inv_freq(hd)
    out = orc.rope(x, seq, heads, hd, start, 0.5, f, layout)
    half = hd // 2
    for h in range(heads):
        for p in range(seq):
            src = x[p, h * hd:(h + 1) * hd].astype(np.float64)
            ang = (np.float32(np.float32(start + p) * np.float32(0.5)) * f).astype(np.float64)
            i0 = np.arange(half) * 2 if layout == 0 else np.arange(half)
            i1 = i0 + 1 if layout == 0 else i0 + half
            exp = np.empty(hd)
            exp[i0] = src[i0] * np.cos(ang) - src[i1] * np.sin(ang)
            exp[i1] = src[i0] * np.sin(ang) + src[i1] * np.cos(ang)
            assert np.max(np.abs(out[h, p] - exp)) <= 2e-6 * np.max(np.abs(src)) + 1e-7
            # a rotation keeps each pair's length
            n_in = src[i0] ** 2 + src[i1] ** 2
            n_out = out[h, p][i0].astype(np.float64) ** 2 + out[h, p][i1].astype(np.float64) ** 2
            assert np.allclose(n_in, n_out, rtol=1e-5, atol=1e-9)


def test_transpose_heads_index_identity(orc):
    seq, heads, hd = 3, 4, 8
    x = np.arange(seq * heads * hd, dtype=F32).reshape(seq, heads * hd)
    out = orc.transpose_heads(x, seq, heads, hd)
    for h in range(heads):
        for p in range(seq):
            assert np.array_equal(out[h, p], x[p, h * hd:(h + 1) * hd])


# ---- attention -----------------------------------------------------------------------
def brute_attention(q, k, v, n_head, q_len, kv_len, start_pos, mask_shift=0, kv_map=None):
    """float64 restatement, written independently of the oracle."""
    n_kv, _, hd = k.shape
    out = np.zeros((q_len, n_head, hd))
    for h in range(n_head):
        kh = (h * n_kv) // n_head if kv_map is None else kv_map(h, n_head, n_kv)
        K = k[kh, :kv_len].astype(np.float64)
        V = v[kh, :kv_len].astype(np.float64)
        for i in range(q_len):
            s = K @ q[h, i].astype(np.float64) / math.sqrt(hd)
            vis = min(kv_len, start_pos + i + 1 + mask_shift)
            s = s[:vis]
            p = np.exp(s - s.max())
            p /= p.sum()
            out[i, h] = p @ V[:vis]
    return out


def rand_qkv(seed, n_head, n_kv, q_len, pos, hd):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_head, q_len, hd)).astype(F32)
    k = rng.standard_normal((n_kv, pos, hd)).astype(F32)
    v = rng.standard_normal((n_kv, pos, hd)).astype(F32)
    return q, k, v


@pytest.mark.parametrize("n_head,n_kv,hd,q_len,kv_len,start", [
    (4, 2, 16, 1, 9, 8), (4, 4, 8, 3, 3, 0), (6, 4, 8, 2, 7, 5), (8, 1, 32, 4, 20, 16), (2, 2, 64, 5, 12, 0)])
def test_attention_matches_float64_brute_force(orc, n_head, n_kv, hd, q_len, kv_len, start):
    q, k, v = rand_qkv(n_head * 100 + kv_len, n_head, n_kv, q_len, kv_len + 3, hd)
    got = orc.attention(q, k, v, n_head, q_len, kv_len, start)
    ref = brute_attention(q, k, v, n_head, q_len, kv_len, start)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(v))


def test_brute_force_catches_planted_mistakes(orc):
    n_head, n_kv, hd, q_len, kv_len, start = 6, 4, 8, 3, 6, 3
    q, k, v = rand_qkv(11, n_head, n_kv, q_len, kv_len, hd)
    got = orc.attention(q, k, v, n_head, q_len, kv_len, start)
    tol = 1e-5 * np.max(np.abs(v))
    assert np.max(np.abs(got - brute_attention(q, k, v, n_head, q_len, kv_len, start))) <= tol
    # a mask that admits one more position, or a kv head taken as h % n_kv, is caught
    assert np.max(np.abs(got - brute_attention(q, k, v, n_head, q_len, kv_len, start, mask_shift=1))) > tol
    assert np.max(np.abs(got - brute_attention(q, k, v, n_head, q_len, kv_len, start,
                                               kv_map=lambda h, nh, nk: h % nk))) > tol


def test_attention_closed_forms(orc):
    hd = 16
    rng = np.random.default_rng(3)
    # one visible position: out = V[0] exactly
    q, k, v = rand_qkv(5, 2, 1, 1, 4, hd)
    out = orc.attention(q, k, v, 2, 1, 1, 0)
    assert np.array_equal(out[0, 0], v[0, 0]) and np.array_equal(out[0, 1], v[0, 0])
    # causal row 0 of a prompt (start 0) sees only position 0
    q, k, v = rand_qkv(6, 1, 1, 4, 4, hd)
    out = orc.attention(q, k, v, 1, 4, 4, 0)
    assert np.array_equal(out[0, 0], v[0, 0])
    # identical keys: uniform weights, out = mean of V
    krow = rng.standard_normal(hd).astype(F32)
    k = np.tile(krow, (1, 10, 1)).astype(F32)
    v = rng.standard_normal((1, 10, hd)).astype(F32)
    qq = rng.standard_normal((1, 1, hd)).astype(F32)
    out = orc.attention(qq, k, v, 1, 1, 10, 9)
    assert np.allclose(out[0, 0], v[0].astype(np.float64).mean(axis=0), atol=1e-6)
    # the same vector added to every key shifts every score by q.u / sqrt(hd):
    # the softmax, and so the output, does not change
    q, k, v = rand_qkv(8, 1, 1, 1, 6, hd)
    u = (0.5 * rng.standard_normal(hd)).astype(F32)
    base = orc.attention(q, k, v, 1, 1, 6, 5)
    shifted = orc.attention(q, (k + u).astype(F32), v, 1, 1, 6, 5)
    assert np.max(np.abs(shifted - base)) <= 1e-5 * np.max(np.abs(v))
