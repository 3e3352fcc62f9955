"""GPU parity of RMSNorm and the fused RMSNorm -> Q8_K / Q8_0 quantizer
(models/src/transformer.rs:148-172) against the oracle.

Bars: the normalized rows within 1e-5 (relative L2 and max-abs relative to
max |y|; the GPU sums the squares in a tree, the reference sequentially); the
fused quantizer byte-identical to quantize_act applied to the GPU's own f32
rows (on the GPU and in the oracle); against the oracle's sequential
normalization, quantized values differ by at most one step, in a small
fraction of positions."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth

pytestmark = pytest.mark.gpu

SHAPES = [(1, 4096), (7, 4096), (3, 5120), (2, 16384), (5, 100), (1, 4), (64, 1024)]


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def inputs(rows, n, seed):
    x = synth.gen_f32(rows * n, seed).reshape(rows, n)
    w = (1.0 + 0.25 * synth.gen_f32(n, seed + 1)).astype(np.float32)
    return x, w


@pytest.mark.parametrize("rows,n", SHAPES)
def test_rms_norm_matches_oracle(be, orc, rows, n):
    x, w = inputs(rows, n, 100 + n + rows)
    got = be.rms_norm(dev(x), dev(w), 1e-5).cpu().numpy()
    ref = orc.rms_norm(x, w, 1e-5)
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    host = be.rms_norm(x, w, 1e-5, mem=B.MEM_HOST)
    assert np.array_equal(host, got)


@pytest.mark.parametrize("act", ["Q8_K", "Q8_0"])
@pytest.mark.parametrize("rows,n", [(1, 4096), (7, 4096), (3, 5120), (2, 16384), (64, 1024), (1, 256)])
def test_fused_quantizer_equals_quantize_of_norm(be, orc, act, rows, n):
    t = B.Q8_K if act == "Q8_K" else B.Q8_0
    x, w = inputs(rows, n, 200 + n + rows)
    xd, wd = dev(x), dev(w)
    fused = be.rms_norm_quantize(t, xd, wd, 1e-5).cpu().numpy()
    y = be.rms_norm(xd, wd, 1e-5)
    unfused = be.quantize_act(t, y).cpu().numpy()
    assert np.array_equal(fused, unfused)
    assert np.array_equal(fused, orc.quantize_act(t, y.cpu().numpy()))
    assert np.array_equal(be.rms_norm_quantize(t, x, w, 1e-5, mem=B.MEM_HOST), fused)
    # against the oracle's own (sequential) normalization
    ref = orc.quantize_act(t, orc.rms_norm(x, w, 1e-5))
    dq = orc.dequantize(t, fused, rows * n)
    dr = orc.dequantize(t, ref, rows * n)
    assert np.linalg.norm(dq - dr) / np.linalg.norm(dr) <= 1e-3


def test_zero_row_and_eps_floor(be, orc):
    x = np.zeros((2, 1024), np.float32)
    x[1] = 1e-30
    w = np.ones(1024, np.float32)
    got = be.rms_norm(dev(x), dev(w), 0.0).cpu().numpy()
    assert np.array_equal(got, orc.rms_norm(x, w, 0.0))
    q = be.rms_norm_quantize(B.Q8_K, dev(x), dev(w), 0.0).cpu().numpy()
    assert np.array_equal(q, orc.quantize_q8_k(orc.rms_norm(x, w, 0.0)))


@pytest.mark.parametrize("out", ["F32", "Q8_K", "Q8_0"])
@pytest.mark.parametrize("rows,n", [(1, 4096), (3, 5120), (2, 16384)])
def test_residual_add_fused_with_norm(be, orc, out, rows, n):
    """add_vectors (transformer.rs:505-510) fused into the next RMSNorm: the
    stored sum is x + d bit for bit, and the output is exactly what the
    unfused norm (or fused norm + quantizer) gives on that sum."""
    import torch
    t = {"F32": B.F32, "Q8_K": B.Q8_K, "Q8_0": B.Q8_0}[out]
    x, w = inputs(rows, n, 300 + n + rows)
    d = (synth.gen_f32(rows * n, 400 + n) * 3.0).reshape(rows, n)
    xd, dd, wd = dev(x), dev(d), dev(w)
    s = torch.empty_like(xd)
    got = be.add_rms_norm_quantize(t, xd, dd, wd, 1e-5, sum_out=s).cpu().numpy()
    assert np.array_equal(s.cpu().numpy(), x + d)
    if t == B.F32:
        assert np.array_equal(got, be.rms_norm(s, wd, 1e-5).cpu().numpy())
    else:
        assert np.array_equal(got, be.rms_norm_quantize(t, s, wd, 1e-5).cpu().numpy())
    # without d it is the plain (fused) norm; host buffers give the same bytes
    plain = be.add_rms_norm_quantize(t, xd, None, wd, 1e-5).cpu().numpy()
    ref_plain = be.rms_norm(xd, wd, 1e-5).cpu().numpy() if t == B.F32 else be.rms_norm_quantize(t, xd, wd, 1e-5).cpu().numpy()
    assert np.array_equal(plain, ref_plain)
    s_h = np.empty((rows, n), np.float32)
    got_h = be.add_rms_norm_quantize(t, x, d, w, 1e-5, sum_out=s_h, mem=B.MEM_HOST)
    assert np.array_equal(s_h, x + d) and np.array_equal(np.asarray(got_h).reshape(got.shape), got)
    with pytest.raises(B.BarqError):
        be.add_rms_norm_quantize(t, xd, None, wd, 1e-5, sum_out=s)   # a sum needs d
