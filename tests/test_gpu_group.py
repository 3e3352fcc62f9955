"""GPU parity of barq_rocm_matvec_group (the q/k/v projections of one
activation row in one launch) through the C ABI.

Each output of the grouped launch must equal, bit for bit, the matvec the
register GEMV computes for that matrix alone (same lane slicing and
reduction order), and be within the 1e-3 bar of the oracle.  The Q6_K
matrix is compared with a handle that keeps Q6_K on the register GEMV
(BARQ_GEMV_DMA_TYPES=0), since the default single matvec streams Q6_K
through the LDS kernel, whose reduction order differs."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth
from conftest import assert_bits_equal, assert_close_1e3
from test_gpu_parity import dev, host, tuned

pytestmark = pytest.mark.gpu

GROUPS = [
    # (types, rows, k)
    ([B.Q4_K, B.Q4_K, B.Q6_K], [4096, 1024, 1024], 4096),    # Llama-3-8B q, k, v
    ([B.Q4_K, B.Q4_K, B.Q4_K], [4096, 1024, 1024], 4096),
    ([B.Q4_K, B.Q4_K, B.Q6_K], [37, 9, 13], 512),             # ragged: partial workgroups and waves
    ([B.Q4_K, B.Q6_K], [1, 1], 256),
    ([B.Q4_K, B.Q4_K, B.Q4_K, B.Q6_K], [100, 7, 65, 33], 2048),
    ([B.Q4_K, B.Q4_K, B.Q4_K, B.Q4_K], [8, 9, 15, 17], 4096),
]


def _inputs(types, rows, k, seed):
    ws = [synth.gen_weights(t, n, k, seed + 10 * i) for i, (t, n) in enumerate(zip(types, rows))]
    x = synth.gen_f32(k, seed + 1)
    return ws, x


@pytest.mark.parametrize("case", range(len(GROUPS)))
def test_matvec_group_equals_separate_matvecs(be, orc, case):
    import torch
    types, rows, k = GROUPS[case]
    print(f"matvec_group types={types} rows={rows} k={k}", flush=True)
    ws, x = _inputs(types, rows, k, 500 + case)
    xq = be.quantize_act(B.Q8_K, dev(x))
    wd = [dev(w) for w in ws]
    ys = [torch.full((n,), float("nan"), dtype=torch.float32, device="cuda") for n in rows]
    be.matvec_group_raw(types, wd, rows, k, B.Q8_K, xq, ys, B.MEM_DEVICE)
    be.sync()
    got = [host(y) for y in ys]
    with tuned(BARQ_GEMV_DMA_TYPES=0) as reg:
        for i, (t, n) in enumerate(zip(types, rows)):
            sep = host(reg.matvec(t, wd[i], n, k, B.Q8_K, xq))
            assert_bits_equal(got[i], sep)
            assert_close_1e3(got[i], orc.matvec(t, ws[i], n, k, B.Q8_K, host(xq)))


def test_matvec_group_fallback_cases(be, orc):
    """Cases outside the one-launch path (host memory, f32 activation, a Q6_K
    matrix that is not last, k > 4096) give the separate matvecs' results."""
    import torch
    k = 4352
    types, rows = [B.Q6_K, B.Q4_K], [19, 40]
    ws, x = _inputs(types, rows, k, 777)
    # host memory, library-side quantization
    ys = [np.empty(n, np.float32) for n in rows]
    be.matvec_group_raw(types, ws, rows, k, B.ACT_F32_Q8, x, ys, B.MEM_HOST)
    xq = orc.quantize_q8_k(x)
    for i, (t, n) in enumerate(zip(types, rows)):
        assert_close_1e3(ys[i], orc.matvec(t, ws[i], n, k, B.Q8_K, xq))
    # device memory: equal to the single matvecs of the same handle
    wd = [dev(w) for w in ws]
    xqd = be.quantize_act(B.Q8_K, dev(x))
    yd = [torch.empty(n, dtype=torch.float32, device="cuda") for n in rows]
    be.matvec_group_raw(types, wd, rows, k, B.Q8_K, xqd, yd, B.MEM_DEVICE)
    be.sync()
    for i, (t, n) in enumerate(zip(types, rows)):
        assert_bits_equal(host(yd[i]), host(be.matvec(t, wd[i], n, k, B.Q8_K, xqd)))


def test_matvec_group_argument_errors(be):
    import torch
    k = 256
    w = dev(synth.gen_q4_k(4, k, 1))
    xq = be.quantize_act(B.Q8_K, dev(synth.gen_f32(k, 2)))
    y = torch.empty(4, dtype=torch.float32, device="cuda")
    with pytest.raises(B.BarqError):
        be.matvec_group_raw([B.Q4_K, B.Q4_K], [w, w], [4, 4], 100, B.Q8_K, xq, [y, y], B.MEM_DEVICE)
    with pytest.raises(B.BarqError):
        be.matvec_group_raw([B.Q4_K, 99], [w, w], [4, 4], k, B.Q8_K, xq, [y, y], B.MEM_DEVICE)
    with pytest.raises(B.BarqError):
        be.matvec_group_raw([B.Q4_K, B.Q4_K], [w, None], [4, 4], k, B.Q8_K, xq, [y, y], B.MEM_DEVICE)
    # zero matrices: nothing to do
    be.matvec_group_raw([], [], [], k, B.Q8_K, xq, [], B.MEM_DEVICE)


# ---- the q/k/v projections + RoPE + cache append of one token -------------

QKV_CASES = [
    # (n_head, n_kv, hd, k, v_type, layout, mem)
    (32, 8, 128, 4096, B.Q6_K, "interleaved", "device"),   # Llama-3-8B: one launch
    (32, 8, 128, 4096, B.Q4_K, "interleaved", "device"),
    (8, 2, 64, 512, B.Q6_K, "interleaved", "device"),
    (6, 3, 64, 256, B.Q4_K, "interleaved", "device"),
    (8, 2, 64, 512, B.Q6_K, "split_half", "device"),       # the two separate calls
    (8, 2, 64, 4352, B.Q6_K, "interleaved", "device"),     # k > 4096: the two separate calls
    (4, 2, 64, 512, B.Q6_K, "interleaved", "host"),
    (4, 4, 256, 1024, B.Q6_K, "interleaved", "device"),       # head_dim 256, one query head per kv head
    (16, 2, 128, 2048, B.Q4_K, "interleaved", "device"),      # GQA 8
]


@pytest.mark.parametrize("case", range(len(QKV_CASES)))
def test_qkv_append_rope_equals_separate_calls(be, case):
    """barq_rocm_qkv_append_rope against barq_rocm_matvec_group followed by
    barq_rocm_kv_cache_append_rope_q on a second cache with the same prefix:
    q_out and every cached K/V row bit for bit, two tokens in a row."""
    import torch
    from barq_rocm import attention as A
    from test_gpu_attention import fill_cache, inv_freq
    n_head, n_kv, hd, k, vt, layout, mem = QKV_CASES[case]
    lay = A.ROPE_INTERLEAVED if layout == "interleaved" else A.ROPE_SPLIT_HALF
    types = [B.Q4_K, B.Q4_K, vt]
    rows = [n_head * hd, n_kv * hd, n_kv * hd]
    print(f"qkv_append_rope n_head={n_head} n_kv={n_kv} hd={hd} k={k} v={vt} {layout} {mem}", flush=True)
    ws = [synth.gen_weights(t, n, k, 900 + 7 * i + case) for i, (t, n) in enumerate(zip(types, rows))]
    pos = 9
    c_ref, _, _ = fill_cache(be, n_kv, hd, pos, 40 + case)
    c_got, _, _ = fill_cache(be, n_kv, hd, pos, 40 + case)
    f = inv_freq(hd)
    # the rotation angle of the new position (large positions take sincosf's long argument reduction)
    rope_pos = [pos, pos + 1] if case % 2 == 0 else [100000, 131071]
    for step in range(2):
        x = synth.gen_f32(k, 70 + 3 * case + step)
        xq = be.quantize_act(B.Q8_K, dev(x))
        if mem == "device":
            wd = [dev(w) for w in ws]
            ys = [torch.empty(n, dtype=torch.float32, device="cuda") for n in rows]
            be.matvec_group_raw(types, wd, rows, k, B.Q8_K, xq, ys, B.MEM_DEVICE)
            q_ref = c_ref.append_rope_q(1, ys[0], n_head, ys[1], ys[2], 1, rope_pos[step], 1.0, dev(f), lay)
            q_got = c_got.qkv_append_rope(1, types, wd, n_head, k, B.Q8_K, xq, rope_pos[step], 1.0, dev(f), lay)
            be.sync()
            q_ref, q_got = host(q_ref), host(q_got)
        else:
            xh = host(xq)
            ys = [np.empty(n, np.float32) for n in rows]
            be.matvec_group_raw(types, ws, rows, k, B.Q8_K, xh, ys, B.MEM_HOST)
            q_ref = c_ref.append_rope_q(1, ys[0], n_head, ys[1], ys[2], 1, rope_pos[step], 1.0, f, lay,
                                        mem=B.MEM_HOST)
            q_got = c_got.qkv_append_rope(1, types, ws, n_head, k, B.Q8_K, xh, rope_pos[step], 1.0, f, lay,
                                          mem=B.MEM_HOST)
        assert_bits_equal(np.asarray(q_got).reshape(-1), np.asarray(q_ref).reshape(-1))
        assert c_got.layer_len(1) == c_ref.layer_len(1) == pos + step + 1
        for hk in range(n_kv):
            kg, vg = c_got.get_head(1, hk)
            kr, vr = c_ref.get_head(1, hk)
            assert_bits_equal(kg.reshape(-1), kr.reshape(-1))
            assert_bits_equal(vg.reshape(-1), vr.reshape(-1))
    c_ref.close()
    c_got.close()


def test_qkv_append_rope_edge_cases(be):
    """An out-of-range layer appends nothing and still writes q; a full
    layer and null buffers are errors; f32 rows on device buffers are not
    taken."""
    from barq_rocm import attention as A
    from test_gpu_attention import fill_cache, inv_freq
    n_head, n_kv, hd, k = 4, 2, 64, 256
    types = [B.Q4_K, B.Q4_K, B.Q6_K]
    rows = [n_head * hd, n_kv * hd, n_kv * hd]
    wd = [dev(synth.gen_weights(t, n, k, 5 + i)) for i, (t, n) in enumerate(zip(types, rows))]
    x = synth.gen_f32(k, 6)
    xq = be.quantize_act(B.Q8_K, dev(x))
    f = dev(inv_freq(hd))
    c, _, _ = fill_cache(be, n_kv, hd, 4, 7)   # max_size 9, layers 0 and 1 hold 4 positions
    q5 = c.qkv_append_rope(5, types, wd, n_head, k, B.Q8_K, xq, 4, 1.0, f, A.ROPE_INTERLEAVED)
    be.sync()
    q1 = c.qkv_append_rope(1, types, wd, n_head, k, B.Q8_K, xq, 4, 1.0, f, A.ROPE_INTERLEAVED)
    be.sync()
    assert_bits_equal(host(q5).reshape(-1), host(q1).reshape(-1))
    assert c.layer_len(1) == 5 and c.layer_len(0) == 4
    for _ in range(4):
        c.qkv_append_rope(1, types, wd, n_head, k, B.Q8_K, xq, 5, 1.0, f, A.ROPE_INTERLEAVED)
    assert c.layer_len(1) == 9
    with pytest.raises(B.BarqError):   # the layer is full
        c.qkv_append_rope(1, types, wd, n_head, k, B.Q8_K, xq, 9, 1.0, f, A.ROPE_INTERLEAVED)
    with pytest.raises(B.BarqError):   # f32 rows on device buffers
        c.qkv_append_rope(0, types, wd, n_head, k, B.ACT_F32, dev(x), 4, 1.0, f, A.ROPE_INTERLEAVED)
    with pytest.raises(B.BarqError):
        c.qkv_append_rope(0, types, [wd[0], None, wd[2]], n_head, k, B.Q8_K, xq, 4, 1.0, f, A.ROPE_INTERLEAVED)
    c.close()
