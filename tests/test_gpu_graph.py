"""Entry points captured in a HIP graph (torch.cuda.CUDAGraph on the handle's
stream) and replayed several times, with eager work of the program and
synchronisations between the replays: every replay must equal the eager
result bit for bit (the kernels are deterministic).  This is how bench.py
times them, and how a caller that cannot launch per call would use them."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import attention as A
from barq_rocm import synth

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def replays_match(be, launch, out, eager_noise):
    """Eager result, then a captured graph replayed 3 times with unrelated
    eager work in between; every replay must reproduce the eager bits."""
    import torch
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    try:
        launch()
        torch.cuda.synchronize()
        ref = out.clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            launch()
        for _ in range(3):
            out.fill_(float("nan"))
            eager_noise()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
    finally:
        torch.cuda.set_stream(torch.cuda.default_stream())
        be.set_stream(None)


def test_matvec_and_matmul_graph_replays(be):
    import torch
    n, k, m = 1024, 4096, 64
    w = dev(synth.gen_q4_k(n, k, 11))
    x = dev(synth.gen_f32(m * k, 12).reshape(m, k))
    xq = be.quantize_act(B.Q8_K, x)
    y1 = torch.empty(n, dtype=torch.float32, device="cuda")
    ym = torch.empty((m, n), dtype=torch.float32, device="cuda")
    other = torch.randn(1 << 20, device="cuda")

    def noise():
        be.matvec_raw(B.Q4_K, w, n, k, B.Q8_K, xq[-(k // 256) * 292:], y1, B.MEM_DEVICE)
        other.mul_(1.0001)
    replays_match(be, lambda: be.matvec_raw(B.Q4_K, w, n, k, B.Q8_K, xq, y1, B.MEM_DEVICE), y1, noise)
    replays_match(be, lambda: be.matmul_raw(B.Q4_K, w, n, k, B.Q8_K, xq, m, ym, B.MEM_DEVICE), ym, noise)


@pytest.mark.parametrize("w_type,m", [(B.Q4_0, 16), (B.Q8_0, 40), (B.Q6_K, 24)])
def test_small_m_matmul_graph_replays(be, w_type, m):
    """Few tiles: K split across workgroups (partial products in the
    workspace, then the ordered slice sum), and for the 32-element formats the
    activation repack, all inside the captured graph."""
    import torch
    n, k = 1000, 4096
    w = dev(synth.gen_weights(w_type, n, k, 13))
    x = dev(synth.gen_f32(m * k, 14).reshape(m, k))
    at = B.Q8_PARTNER[w_type]
    xq = be.quantize_act(at, x)
    ym = torch.empty((m, n), dtype=torch.float32, device="cuda")
    other = torch.randn(1 << 20, device="cuda")

    def noise():
        be.matmul_raw(w_type, w, n, k, at, xq, m, torch.empty_like(ym), B.MEM_DEVICE)   # same workspace
        other.mul_(1.0001)
    replays_match(be, lambda: be.matmul_raw(w_type, w, n, k, at, xq, m, ym, B.MEM_DEVICE), ym, noise)


def test_moe_step_graph_replays(be, orc):
    import torch
    ne, hid, nff, rows, k = 4, 512, 1024, 24, 2
    gates = [synth.gen_q4_k(nff, hid, 40 + e) for e in range(ne)]
    ups = [synth.gen_q4_k(nff, hid, 50 + e) for e in range(ne)]
    downs = [synth.gen_q6_k(hid, nff, 60 + e) for e in range(ne)]
    x = synth.gen_f32(rows * hid, 70).reshape(rows, hid)
    ids, w = orc.moe_select_top_k(synth.gen_f32(rows * ne, 71).reshape(rows, ne), k)
    gd, ud, dd = [dev(a) for a in gates], [dev(a) for a in ups], [dev(a) for a in downs]
    xd, idd, wd = dev(x), dev(np.ascontiguousarray(ids, np.int32)), dev(np.ascontiguousarray(w, np.float32))
    out = torch.empty((rows, hid), dtype=torch.float32, device="cuda")
    x2 = dev(synth.gen_f32(rows * hid, 72).reshape(rows, hid))
    out2 = torch.empty_like(out)

    def step():
        be.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hid, nff, xd, rows, idd, wd, k, B.ACT_F32_Q8, sync=False,
                   out=out)

    def noise():   # the same workspace, other inputs
        be.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hid, nff, x2, rows, idd, wd, k, B.ACT_F32_Q8, sync=False,
                   out=out2)
    replays_match(be, step, out, noise)


def test_attention_graph_replays(be):
    import torch
    n_head, n_kv, hd, kv = 32, 8, 128, 3000
    c = A.KVCache(be, kv, 2, n_kv, hd)
    rng = np.random.default_rng(5)
    for layer in range(2):
        c.append(layer, dev(rng.standard_normal((n_kv, kv, hd)).astype(np.float32)),
                 dev(rng.standard_normal((n_kv, kv, hd)).astype(np.float32)), kv, hd)
    q = dev(rng.standard_normal((n_head, 1, hd)).astype(np.float32))
    out = torch.empty((1, n_head, hd), dtype=torch.float32, device="cuda")
    out2 = torch.empty_like(out)

    def call(layer, o):
        B._lib.check(be._lib.barq_rocm_attention(be.h, q.data_ptr(), c.c, layer, n_head, n_kv, hd, 1, kv, kv - 1,
                                                 o.data_ptr(), B.MEM_DEVICE))
    replays_match(be, lambda: call(1, out), out, lambda: call(0, out2))
    c.close()


@pytest.mark.parametrize("q_len", [512, 100])
def test_prompt_attention_graph_replays(be, q_len):
    """The MFMA prompt kernel captured: 512 tokens (position splits, the
    one-thread merge) and a ragged 100-token chunk after a prefix."""
    import torch
    n_head, n_kv, hd = 32, 8, 128
    kv = q_len + 40
    c = A.KVCache(be, kv, 2, n_kv, hd)
    rng = np.random.default_rng(9)
    for layer in range(2):
        c.append(layer, dev(rng.standard_normal((n_kv, kv, hd)).astype(np.float32)),
                 dev(rng.standard_normal((n_kv, kv, hd)).astype(np.float32)), kv, hd)
    q = dev(rng.standard_normal((n_head, q_len, hd)).astype(np.float32))
    out = torch.empty((q_len, n_head, hd), dtype=torch.float32, device="cuda")
    out2 = torch.empty_like(out)

    def call(layer, o):
        B._lib.check(be._lib.barq_rocm_attention(be.h, q.data_ptr(), c.c, layer, n_head, n_kv, hd, q_len, kv, 40,
                                                 o.data_ptr(), B.MEM_DEVICE))
    replays_match(be, lambda: call(1, out), out, lambda: call(0, out2))
    c.close()


def test_ffn_graph_replays(be):
    """The one-token FFN (fused gate/up launch, h's quantizer, down GEMV):
    every replay equals the eager call, with FFN calls of another shape
    between the replays."""
    import torch
    n_embd, n_ff = 1024, 2304
    w = [dev(synth.gen_q4_k(n_ff, n_embd, 41)), dev(synth.gen_q4_k(n_ff, n_embd, 42)),
         dev(synth.gen_weights(B.Q6_K, n_embd, n_ff, 43))]
    xq = be.quantize_act(B.Q8_K, dev(synth.gen_f32(n_embd, 44)))
    y = torch.empty((1, n_embd), dtype=torch.float32, device="cuda")
    w2 = [dev(synth.gen_q4_k(512, 768, 45)), dev(synth.gen_q4_k(512, 768, 46)), dev(synth.gen_weights(B.Q6_K, 768, 512, 47))]
    x2 = be.quantize_act(B.Q8_K, dev(synth.gen_f32(768, 48)))

    def noise():
        be.ffn(B.Q4_K, w2[0], B.Q4_K, w2[1], B.Q6_K, w2[2], 768, 512, B.Q8_K, x2, 1, sync=False)
    replays_match(be, lambda: be.ffn(B.Q4_K, w[0], B.Q4_K, w[1], B.Q6_K, w[2], n_embd, n_ff, B.Q8_K, xq, 1,
                                     sync=False, out=y), y, noise)


def test_graph_replay_after_workspace_growth(be):
    """A graph captured around a call that uses the workspace keeps working
    after a later, larger call grows the workspace: the old buffer is
    retired, not freed, so the captured kernels still address valid memory."""
    import torch
    be2 = B.Backend(0)   # a fresh handle: its workspace starts at the 16 MiB minimum
    try:
        n, k, m = 1152, 4096, 16
        w = dev(synth.gen_q4_k(n, k, 31))
        x = dev(synth.gen_f32(m * k, 32).reshape(m, k))
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        y2 = torch.empty((2, n), dtype=torch.float32, device="cuda")
        # the literal f32 matmul dequantizes W into the workspace: n * k * 4 B
        # = 18.9 MB, more than the first allocation
        assert n * k * 4 > 16 * 1024 * 1024
        grown = []

        def grow_once():
            if not grown:
                be2.matmul_raw(B.Q4_K, w, n, k, B.ACT_F32, x, 2, y2, B.MEM_DEVICE)
                grown.append(1)
            else:
                be2.matmul_raw(B.Q4_K, w, n, k, B.ACT_F32_Q8, x, 1, y2, B.MEM_DEVICE)
        replays_match(be2, lambda: be2.matmul_raw(B.Q4_K, w, n, k, B.ACT_F32_Q8, x, m, y, B.MEM_DEVICE), y, grow_once)
        assert grown
    finally:
        be2.close()
