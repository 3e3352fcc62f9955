"""The dense FFN on the device (barq_rocm_swiglu, barq_rocm_ffn) against the
oracle of LlamaTransformer::feed_forward (transformer.rs:378-408).

Bars: h within 4 ulp of the oracle's (the device expf against libm's
expf, both within an ulp of exp); h's Q8 blocks byte-identical to
quantizing the device's own f32 h; FFN outputs with Q8 activations within
1e-3 relative L2 error, the north star's bar, and max-abs within 5e-3 of
max |y| (conftest.assert_close_chained: h is quantized a second time, so an
ulp of exp can move one element of h by one Q8 quantum); the down
projection, and the FFN output, within 1e-3 on both measures of the
oracle's down projection fed the device's own h blocks; the literal f32
FFN within 1e-5 on both measures."""
import contextlib
import os

import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth
from conftest import assert_close_1e3, assert_close_chained

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


@contextlib.contextmanager
def tuned(**kv):
    old = {k: os.environ.get(k) for k in kv}
    os.environ.update({k: str(v) for k, v in kv.items()})
    try:
        b = B.Backend(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    try:
        yield b
    finally:
        b.close()


def test_swiglu_f32_and_blocks(be, orc):
    rows, n = 3, 14336
    g = (synth.gen_f32(rows * n, 1) * 4).reshape(rows, n)
    u = synth.gen_f32(rows * n, 2).reshape(rows, n)
    g[0, :8] = [0.0, -0.0, 30.0, 100.0, -100.0, -1000.0, 1.0, -1.0]
    ref = orc.ffn_swiglu(g, u)
    h = host(be.swiglu(B.F32, dev(g), dev(u)))
    ulp = np.spacing(np.abs(ref).astype(np.float32))
    assert np.all(np.abs(h - ref) <= 4 * ulp), np.max(np.abs(h - ref) / np.maximum(ulp, 1e-45))
    for t in (B.Q8_K, B.Q8_0):
        blocks = host(be.swiglu(t, dev(g), dev(u)))
        assert np.array_equal(blocks, host(be.quantize_act(t, dev(h))))
        assert np.array_equal(be.swiglu(t, g, u, mem=B.MEM_HOST), blocks)
    assert np.array_equal(be.swiglu(B.F32, g, u, mem=B.MEM_HOST), h)


def ffn_case(n_embd, n_ff, m, seed, gt, ut, dt):
    gate = synth.gen_weights(gt, n_ff, n_embd, seed)
    up = synth.gen_weights(ut, n_ff, n_embd, seed + 1)
    down = synth.gen_weights(dt, n_embd, n_ff, seed + 2)
    x = synth.gen_f32(m * n_embd, seed + 3).reshape(m, n_embd)
    return gate, up, down, x


# (n_embd, n_ff, m, gate, up, down): Llama-3-8B's FFN at one token (the fused
# gate/up launch) and at 3 and 16 tokens (multi-token GEMV, MFMA GEMM), the
# 32-element formats, mixed types, k above one 4096-element chunk
CASES = {
    "llama3_decode": (4096, 14336, 1, B.Q4_K, B.Q4_K, B.Q6_K),
    "llama3_decode_q4k_down": (4096, 14336, 1, B.Q4_K, B.Q4_K, B.Q4_K),
    "llama3_3tok": (4096, 14336, 3, B.Q4_K, B.Q4_K, B.Q6_K),
    "prefill16": (1024, 2816, 16, B.Q4_K, B.Q4_K, B.Q6_K),
    "q4_0": (1024, 2048, 1, B.Q4_0, B.Q4_0, B.Q8_0),
    "q4_0_m5": (1024, 2048, 5, B.Q4_0, B.Q4_0, B.Q4_0),
    "mixed": (512, 1536, 2, B.Q6_K, B.Q4_K, B.Q4_K),
    "long_k": (5120, 1280, 1, B.Q4_K, B.Q4_K, B.Q6_K),
}


@pytest.mark.parametrize("name", list(CASES))
def test_ffn_q8(be, orc, name):
    n_embd, n_ff, m, gt, ut, dt = CASES[name]
    gate, up, down, x = ffn_case(n_embd, n_ff, m, 300 + len(name), gt, ut, dt)
    pa = B.Q8_PARTNER[gt]
    xq = orc.quantize_act(pa, x)
    ref = orc.ffn(gt, gate, ut, up, dt, down, n_embd, n_ff, pa, xq, m)
    print(f"ffn {name}", flush=True)
    gd, ud, dd = dev(gate), dev(up), dev(down)
    got = host(be.ffn(gt, gd, ut, ud, dt, dd, n_embd, n_ff, B.ACT_F32_Q8, dev(x), m))
    assert_close_chained(got, ref)
    # already-quantized input rows give the same result bit for bit
    got_q = host(be.ffn(gt, gd, ut, ud, dt, dd, n_embd, n_ff, pa, dev(xq), m))
    assert np.array_equal(got_q, got)
    # the down projection at the north star's 1e-3 bar: the oracle's down
    # projection fed the device's own h blocks (swiglu of the device's gate
    # and up products), so h's second quantization is out of the comparison;
    # the FFN's output is held to the same bar against it (its h comes from
    # the same products, up to the f32 summation order of a fused launch)
    pd = B.Q8_PARTNER[dt]
    g_dev = be.matmul(gt, gd, n_ff, n_embd, pa, dev(xq), m)
    u_dev = be.matmul(ut, ud, n_ff, n_embd, pa, dev(xq), m)
    hq = be.swiglu(pd, g_dev, u_dev)
    down_ref = orc.matmul(dt, down, n_embd, n_ff, pd, host(hq), m)
    assert_close_1e3(host(be.matmul(dt, dd, n_embd, n_ff, pd, hq, m)), down_ref)
    assert_close_1e3(got, down_ref)


def test_ffn_fused_gate_up_matches_separate_path(be, orc):
    """m = 1 with Q4_K gate/up takes the fused launch; the same row as part of
    a 2-row call takes the separate projections.  Each is checked against the
    oracle; the launch shapes of the fused kernel as well."""
    n_embd, n_ff = 4096, 14336
    gate, up, down, x = ffn_case(n_embd, n_ff, 1, 410, B.Q4_K, B.Q4_K, B.Q6_K)
    xq = orc.quantize_act(B.Q8_K, x)
    ref = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.Q8_K, xq, 1)
    gd, ud, dd = dev(gate), dev(up), dev(down)
    x2 = np.concatenate([xq, xq])
    two = host(be.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K, dev(x2), 2))
    assert_close_chained(two[:1], ref)
    assert np.array_equal(two[0], two[1])
    for glu in (14, 12, 18, 24, 22, 28):
        print(f"ffn glu shape {glu}", flush=True)
        with tuned(BARQ_GEMV_GLU=glu, BARQ_GEMV_LDS=0) as b:
            got = host(b.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K, dev(xq), 1))
        assert_close_chained(got, ref)
    # odd n_ff: the last wave of the two-output shape has one output
    n_ff2 = 256 * 9
    gate2, up2, down2, x2 = ffn_case(1024, n_ff2, 1, 420, B.Q4_K, B.Q4_K, B.Q4_K)
    xq2 = orc.quantize_act(B.Q8_K, x2)
    ref2 = orc.ffn(B.Q4_K, gate2, B.Q4_K, up2, B.Q4_K, down2, 1024, n_ff2, orc.Q8_K, xq2, 1)
    with tuned(BARQ_GEMV_GLU=24, BARQ_GEMV_LDS=0) as b:
        got2 = host(b.ffn(B.Q4_K, dev(gate2), B.Q4_K, dev(up2), B.Q4_K, dev(down2), 1024, n_ff2, B.Q8_K, dev(xq2), 1))
    assert_close_chained(got2, ref2)


def test_ffn_lds_gate_up_equals_register_gate_up(be, orc):
    """The LDS-staged fused gate/up GEMV (the default for k <= 4096) gives
    the register kernel's h (BARQ_GEMV_LDS=0) bit for bit, so the whole FFN
    output matches; short k leaves lanes idle, and n_ff is not a multiple of
    the rows per workgroup."""
    for n_embd, n_ff in [(4096, 14336), (1024, 256 * 9), (768, 512)]:
        print(f"ffn lds glu {n_embd} {n_ff}", flush=True)
        gate, up, down, x = ffn_case(n_embd, n_ff, 1, 440 + n_embd, B.Q4_K, B.Q4_K, B.Q6_K)
        xq = orc.quantize_act(B.Q8_K, x)
        gd, ud, dd = dev(gate), dev(up), dev(down)
        got = host(be.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K, dev(xq), 1))
        with tuned(BARQ_GEMV_LDS=0) as b:
            base = host(b.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K, dev(xq), 1))
        assert np.array_equal(got, base)
        ref = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.Q8_K, xq, 1)
        assert_close_chained(got, ref)


def test_ffn_small_batch_equals_one_token_ffn(be, orc):
    """2-4 tokens (gate and up in one launch over every row, then h's
    quantizer and the down GEMV over every row): each token's output equals
    the one-token FFN of that row bit for bit, and the oracle within the
    chained bar.  n_ff is a multiple of 512, so the Q6_K down projection of
    2-4 tokens is a GEMV too (otherwise 3-4 tokens take the MFMA GEMM, whose
    sums are ordered differently)."""
    from conftest import assert_bits_equal
    for n_embd, n_ff in [(4096, 14336), (1024, 2560), (768, 512)]:
        gate, up, down, _ = ffn_case(n_embd, n_ff, 1, 520 + n_embd, B.Q4_K, B.Q4_K, B.Q6_K)
        gd, ud, dd = dev(gate), dev(up), dev(down)
        for m in (2, 3, 4):
            print(f"ffn small batch {n_embd} {n_ff} m={m}", flush=True)
            x = synth.gen_f32(m * n_embd, 530 + m).reshape(m, n_embd)
            xq = orc.quantize_act(B.Q8_K, x)
            got = host(be.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K, dev(xq), m))
            rb = B.row_bytes(B.Q8_K, n_embd)
            for j in range(m):
                one = host(be.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K,
                                  dev(xq[j * rb:(j + 1) * rb]), 1))
                assert_bits_equal(got[j], one[0])
            ref = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.Q8_K, xq, m)
            assert_close_chained(got, ref)


@pytest.mark.parametrize("m", [1, 3])
def test_ffn_literal_f32(be, orc, m):
    n_embd, n_ff = 1024, 2816
    gate, up, down, x = ffn_case(n_embd, n_ff, m, 500 + m, B.Q4_K, B.Q4_K, B.Q6_K)
    ref = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.F32, x, m)
    got = host(be.ffn(B.Q4_K, dev(gate), B.Q4_K, dev(up), B.Q6_K, dev(down), n_embd, n_ff, B.ACT_F32, dev(x), m))
    assert_close_1e3(got, ref, tol=1e-5)


def test_ffn_host_buffers(be, orc):
    n_embd, n_ff, m = 512, 1024, 2
    gate, up, down, x = ffn_case(n_embd, n_ff, m, 600, B.Q4_K, B.Q4_K, B.Q6_K)
    xq = orc.quantize_act(B.Q8_K, x)
    ref = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.Q8_K, xq, m)
    got = be.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, B.ACT_F32_Q8, x, m, mem=B.MEM_HOST)
    assert_close_chained(got, ref)
