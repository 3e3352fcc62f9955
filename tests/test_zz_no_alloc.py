"""barq_rocm_matmul_noalloc (fixed per-GPU scratch, no allocation) against
barq_rocm_matmul on the same inputs, through the C ABI: bit-identical
outputs, on two calls in a row (the second with a smaller input), for the
paths that use scratch (activations quantized in the call, K slices, the
32-element-block GEMM's repacked rows, the literal f32 matmul) and for one
that uses none; a call needing more scratch than the array holds fails
before anything is enqueued."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_both(be, t, wd, n, k, act, xd, m):
    import torch
    y_ref = torch.empty((m, n), dtype=torch.float32, device="cuda")
    y_na = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    be.matmul_raw(t, wd, n, k, act, xd, m, y_ref, B.MEM_DEVICE)
    be.matmul_noalloc_raw(t, wd, n, k, act, xd, m, y_na)
    be.sync()
    return y_ref.cpu().numpy(), y_na.cpu().numpy()


# (weight type, n_rows, k, activation mode, [m of the first call, m of the second])
CASES = [
    ("Q4_K_f32q8_kslices", B.Q4_K, 1000, 4096, B.ACT_F32_Q8, [16, 5]),
    ("Q6_K_q8k_kslices", B.Q6_K, 1100, 2048, B.Q8_K, [40, 17]),
    ("Q4_0_b32_repack", B.Q4_0, 300, 1024, B.ACT_F32_Q8, [64, 9]),
    ("Q8_0_b32_repack", B.Q8_0, 257, 512, B.Q8_0, [33, 4]),
    ("Q4_K_gemv_f32q8", B.Q4_K, 700, 4096, B.ACT_F32_Q8, [1, 1]),
    ("Q4_K_literal_f32", B.Q4_K, 96, 512, B.ACT_F32, [7, 3]),
    ("Q4_K_c4_shape", B.Q4_K, 4096, 4096, B.ACT_F32_Q8, [512, 100]),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_matmul(be, orc, case):
    name, t, n, k, act, ms = case
    w = synth.gen_weights(t, n, k, 4242 + n)
    wd = dev(w)
    for call, m in enumerate(ms):
        x = synth.gen_f32(m * k, 4343 + 7 * call + m).reshape(m, k)
        if act in (B.Q8_0, B.Q8_K):
            xd = dev(orc.quantize_act(act, x))
        else:
            xd = dev(x)
        print(f"noalloc {name} call {call} m={m}", flush=True)
        y_ref, y_na = run_both(be, t, wd, n, k, act, xd, m)
        assert np.array_equal(y_ref.view(np.uint32), y_na.view(np.uint32)), f"{name} call {call}: outputs differ"


def test_noalloc_rejects_oversized_scratch(be):
    import torch
    # literal f32 matmul dequantizes W into scratch: 4096 x 4096 x 4 B = 64 MiB > 32 MiB
    n = k = 4096
    assert n * k * 4 > B.NOALLOC_SCRATCH_BYTES
    w = dev(synth.gen_weights(B.Q4_K, n, k, 1))
    x = dev(synth.gen_f32(2 * k, 2))
    y = torch.full((2, n), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(B.BarqError) as e:
        be.matmul_noalloc_raw(B.Q4_K, w, n, k, B.ACT_F32, x, 2, y)
    assert e.value.code == B.E_UNSUPPORTED and "scratch" in str(e.value)
    be.sync()
    assert bool(torch.all(y == 7.0))   # nothing was enqueued
