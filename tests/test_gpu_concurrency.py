"""Distinct handles used from concurrent threads (the reference calls its
BLAS from rayon workers, models/src/transformer.rs:315-331): four threads,
each with its own handle and stream, run matvec / matmul / attention calls
repeatedly; every result must equal the single-threaded one bit for bit.
ctypes releases the GIL around each library call, so the calls overlap."""
import threading

import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import attention as A
from barq_rocm import synth

pytestmark = pytest.mark.gpu


def test_distinct_handles_from_threads():
    import torch
    n, k, m = 2048, 4096, 40
    w4 = torch.from_numpy(synth.gen_q4_k(n, k, 5)).cuda()
    w6 = torch.from_numpy(synth.gen_q6_k(n, k, 6)).cuda()
    w0 = torch.from_numpy(synth.gen_q4_0(n, k, 7)).cuda()
    x = torch.from_numpy(synth.gen_f32(m * k, 8).reshape(m, k)).cuda()
    rng = np.random.default_rng(9)
    kv = rng.standard_normal((4, 700, 128)).astype(np.float32)
    vv = rng.standard_normal((4, 700, 128)).astype(np.float32)
    q = rng.standard_normal((16, 1, 128)).astype(np.float32)

    def work(be, cache):
        xk = be.quantize_act(B.Q8_K, x)
        x0 = be.quantize_act(B.Q8_0, x)
        return [be.matvec(B.Q4_K, w4, n, k, B.Q8_K, xk).cpu(),
                be.matvec(B.Q4_0, w0, n, k, B.Q8_0, x0).cpu(),
                be.matmul(B.Q4_K, w4, n, k, B.Q8_K, xk, m).cpu(),
                be.matmul(B.Q6_K, w6, n, k, B.Q8_K, xk, m).cpu(),
                torch.from_numpy(A.compute_attention(be, q, cache, 0, 16, 4, 128, 1, 700, 699, mem=B.MEM_HOST))]

    def setup():
        be = B.Backend(0)
        cache = A.KVCache(be, 700, 1, 4, 128)
        cache.append(0, kv, vv, 700, 128, mem=B.MEM_HOST)
        return be, cache

    be0, c0 = setup()
    ref = work(be0, c0)
    c0.close()
    be0.close()

    errors, results = [], {}

    def run(tid):
        try:
            be, cache = setup()
            for it in range(6):
                results[(tid, it)] = work(be, cache)
            cache.close()
            be.close()
        except Exception as e:   # reported below
            errors.append(f"thread {tid}: {e!r}")

    threads = [threading.Thread(target=run, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
    assert len(results) == 24
    for key, got in results.items():
        for a, b in zip(got, ref):
            assert torch.equal(a, b), key


def test_stream_switch_orders_workspace_users():
    """barq_rocm_set_stream between two calls that use the handle's one
    workspace (f32 activations quantized into it, then a GEMM reading them):
    the second call, on the new stream, must not overwrite the first call's
    quantized rows while the first GEMM, on the old stream, still reads them.
    The first call is made long (a large matmul) so an unordered second call
    would land inside it."""
    import torch
    n, k, m = 14336, 4096, 256
    w = torch.from_numpy(synth.gen_q4_k(n, k, 21)).cuda()
    xa = torch.from_numpy(synth.gen_f32(m * k, 22).reshape(m, k)).cuda()
    xb = torch.from_numpy(synth.gen_f32(m * k, 23).reshape(m, k) * 3.0).cuda()
    be = B.Backend(0)
    try:
        ref_a = be.matmul(B.Q4_K, w, n, k, B.ACT_F32_Q8, xa, m)
        ref_b = be.matmul(B.Q4_K, w, n, k, B.ACT_F32_Q8, xb, m)
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        for it in range(3):
            ya = torch.full((m, n), float("nan"), device="cuda")
            yb = torch.full((m, n), float("nan"), device="cuda")
            torch.cuda.synchronize()
            be.set_stream(s1.cuda_stream)
            be.matmul_raw(B.Q4_K, w, n, k, B.ACT_F32_Q8, xa, m, ya, B.MEM_DEVICE)
            be.set_stream(s2.cuda_stream)
            be.matmul_raw(B.Q4_K, w, n, k, B.ACT_F32_Q8, xb, m, yb, B.MEM_DEVICE)
            torch.cuda.synchronize()
            assert torch.equal(ya, ref_a), f"iteration {it}: first call's result changed"
            assert torch.equal(yb, ref_b), f"iteration {it}: second call's result changed"
        be.set_stream(None)
    finally:
        be.close()
