"""The synthetic-input generator is deterministic and produces the block
statistics the benchmark configurations describe."""
import numpy as np

import barq_rocm as B
from barq_rocm import synth


def test_splitmix64_published_vector():
    # SplitMix64 with state 0: first outputs (Steele et al.; java.util.SplittableRandom)
    w = synth.splitmix64(0, 3)
    assert [int(v) for v in w] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_stream_offsets_and_determinism():
    a = synth.splitmix64(1234, 100)
    b = synth.splitmix64(1234, 60, start=40)
    assert np.array_equal(a[40:], b)
    assert np.array_equal(synth.gen_q4_k(8, 512, 9), synth.gen_q4_k(8, 512, 9))
    assert not np.array_equal(synth.gen_q4_k(8, 512, 9), synth.gen_q4_k(8, 512, 10))


def test_normals_moments():
    z = synth.normals(42, 200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


def test_q4_k_fields(orc):
    w = synth.gen_q4_k(64, 4096, 3).reshape(-1, 144)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float64)
    assert np.all(d >= 0) and 0.005 < d.mean() < 0.011   # E|N(0,0.01)| = 0.008
    sc = [orc.get_scale_min_k4(j, w[0, 4:16]) for j in range(8)]
    assert all(0 <= s < 64 and 0 <= m < 64 for s, m in sc)


def test_q6_k_fields():
    w = synth.gen_q6_k(64, 4096, 3).reshape(-1, 210)
    sc = w[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31


def test_sizes_match_baseline_configs():
    # packed weight bytes of the five configs' matrices (C1-C3 and C5's down projection)
    assert B.row_bytes(B.Q4_0, 4096) * 4096 == 9437184
    assert B.row_bytes(B.Q4_K, 4096) * 14336 == 33030144
    assert B.row_bytes(B.Q6_K, 4096) * 128256 == 430940160
    assert B.row_bytes(B.Q6_K, 14336) * 4096 == 48168960
