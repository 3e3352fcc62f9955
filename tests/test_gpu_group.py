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
