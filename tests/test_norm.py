"""RMSNorm (models/src/transformer.rs:148-172): the oracle pinned on the CPU,
and the boundary's argument checks.  GPU parity is in test_gpu_norm.py."""
import numpy as np
import pytest

import barq_rocm._lib as L


def test_reference_known_answer_rms_of_output_is_one(orc):
    # barq_core/src/normalization.rs:115-124 and tests/integration_test.rs:167-186:
    # input [1, 2, 3, 4], unit weight, eps 1e-5 -> the output's RMS is 1 within 1e-4
    y = orc.rms_norm(np.float32([1, 2, 3, 4]), np.ones(4, np.float32), 1e-5)[0]
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-4


def test_matches_the_closed_form_in_double(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 4096)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    y = orc.rms_norm(x, w, 1e-5).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w.astype(np.float64)
    assert np.max(np.abs(y - ref) / np.max(np.abs(ref))) < 1e-6


def test_sum_of_squares_is_sequential_and_products_left_to_right(orc):
    # transformer.rs:162 sums with Iterator::sum (a left fold); a pairwise sum
    # rounds differently on this input, and x * rms_inv * w is (x * rms_inv) * w
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-6, 6, 4096))).astype(np.float32)
    w = rng.uniform(0.1, 3.0, 4096).astype(np.float32)
    sq = x * x
    seq = np.cumsum(sq, dtype=np.float32)[-1]
    assert seq != np.float32(np.sum(sq, dtype=np.float32))   # the input separates the two orders
    rms_inv = np.float32(1.0) / np.sqrt(np.float32(seq / np.float32(4096)) + np.float32(1e-5))
    want = (x * rms_inv) * w
    got = orc.rms_norm(x, w, 1e-5)[0]
    assert np.array_equal(got, want)
    assert not np.array_equal(x * (rms_inv * w), want)   # the other association is distinguishable


def test_eps_is_floored_at_f32_epsilon(orc):
    # transformer.rs:158: eps.max(f32::EPSILON); an all-zero row stays zero
    x = np.zeros((1, 256), np.float32)
    assert np.array_equal(orc.rms_norm(x, np.ones(256, np.float32), 0.0), x)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256) * 1e-4).astype(np.float32)
    a = orc.rms_norm(x, np.ones(256, np.float32), 1e-12)
    b = orc.rms_norm(x, np.ones(256, np.float32), float(np.finfo(np.float32).eps))
    assert np.array_equal(a, b)


def test_argument_errors():
    lib = L.lib()
    x = np.zeros(512, np.float32)
    w = np.ones(512, np.float32)
    out = np.zeros(2 * 292, np.uint8)
    # n not a multiple of 256 for the fused quantizer -> DimensionMismatch
    rc = lib.barq_rocm_rms_norm_quantize(None, L.Q8_K, x.ctypes.data, w.ctypes.data, 1, 260, 1e-5, out.ctypes.data,
                                         L.MEM_HOST)
    assert rc == L.E_DIM
    # unsupported output type
    rc = lib.barq_rocm_rms_norm_quantize(None, L.Q4_K, x.ctypes.data, w.ctypes.data, 1, 512, 1e-5, out.ctypes.data,
                                         L.MEM_HOST)
    assert rc == L.E_UNSUPPORTED
    # rows longer than the register-resident kernel takes
    rc = lib.barq_rocm_rms_norm(None, x.ctypes.data, w.ctypes.data, 1, 16388, 1e-5, x.ctypes.data, L.MEM_HOST)
    assert rc == L.E_DIM
    # valid arguments, no handle
    rc = lib.barq_rocm_rms_norm(None, x.ctypes.data, w.ctypes.data, 1, 512, 1e-5, x.ctypes.data, L.MEM_HOST)
    assert rc == L.E_INVALID
    # empty problems succeed
    assert lib.barq_rocm_rms_norm(None, None, None, 0, 512, 1e-5, None, L.MEM_HOST) == L.OK
