"""GPU parity: libbarq_rocm (through the C ABI) against the CPU oracle.

Bars: dequantized weights and quantized activations bit-exact; matvec and
matmul outputs within 1e-3 (relative L2 and max-abs relative to max |y|),
the tolerance the north star states.  The oracle for the Q8 paths runs on
the same quantized activations the GPU produced (after checking those are
bit-exact with the oracle's own quantization)."""
import contextlib
import os

import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth
from conftest import assert_bits_equal, assert_close_1e3

pytestmark = pytest.mark.gpu

TYPES = {"Q4_0": B.Q4_0, "Q4_0_BARQ": B.Q4_0_BARQ, "Q8_0": B.Q8_0, "Q4_K": B.Q4_K, "Q6_K": B.Q6_K}


@contextlib.contextmanager
def tuned(**kv):
    """A handle created with tuning variables kv set (read at creation)."""
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


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def special_blocks(t, nb, seed):
    """Random blocks with edge values mixed in: f16 subnormal / zero / max
    scales, all-0x00 and all-0xFF payloads."""
    bb = B.BLOCK_BYTES[t]
    w = synth.gen_weights(t, nb, B.BLOCK_ELEMS[t], seed).reshape(nb, bb).copy()
    rng = np.random.default_rng(seed)
    f16s = np.float16([0.0, 2.0 ** -24, 6.1e-5, 65504.0, -1.5, 1.0]).view(np.uint8).reshape(-1, 2)
    for i in range(0, nb, 7):
        if t in (B.Q4_0, B.Q8_0):
            w[i, 0:2] = f16s[i % 6]
        elif t == B.Q4_K:
            w[i, 0:2] = f16s[i % 6]
            w[i, 2:4] = f16s[(i + 1) % 6]
        elif t == B.Q6_K:
            w[i, 208:210] = f16s[i % 6]
        elif t == B.Q4_0_BARQ:
            w[i, 0:4] = np.float32([0.0, 1e-40, 3.4e38, -2.0, 1.0, 0.125])[i % 6:i % 6 + 1].view(np.uint8)
        if i % 3 == 0:
            off = 4 if t == B.Q4_0_BARQ else (0 if t == B.Q6_K else 2 if t != B.Q4_K else 16)
            end = 208 if t == B.Q6_K else bb
            w[i, off:end] = 0xFF if i % 2 else 0x00
    return w.reshape(-1)


# ---- dequantize: bit-exact -------------------------------------------------

@pytest.mark.parametrize("name", list(TYPES))
def test_dequantize_bit_exact(be, orc, name):
    t = TYPES[name]
    nb = 3001
    w = special_blocks(t, nb, 11)
    n = nb * B.BLOCK_ELEMS[t]
    print(f"dequantize {name} n={n}", flush=True)
    got = host(be.dequantize(t, dev(w), n))
    ref = orc.dequantize(t, w, n)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    assert_bits_equal(got[fin], ref[fin])


def test_dequantize_f16_all_patterns(be, orc):
    bits = np.arange(65536, dtype=np.uint16).view(np.uint8)
    got = host(be.dequantize(B.F16, dev(bits), 65536))
    ref = orc.dequantize(orc.F16, bits, 65536)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_bits_equal(got[~nan], ref[~nan])


def test_dequantize_host_memory(be, orc):
    w = synth.gen_q4_k(33, 512, 5)
    out = np.empty(33 * 512, np.float32)
    be.dequantize_raw(B.Q4_K, w, out.size, out, B.MEM_HOST)
    assert_bits_equal(out, orc.dequantize(orc.Q4_K, w, out.size))


# ---- activation quantizers: bit-exact --------------------------------------

def act_rows(k, rows, seed):
    x = synth.gen_f32(rows * k, seed).reshape(rows, k)
    x[1 % rows, :] = 0.0                                   # zero rows / blocks
    x[2 % rows, 7] = 1e4                                   # one huge value
    x[3 % rows, :] *= 1e-6                                 # tiny values
    if rows > 4:
        x[4, :64] = np.float32(np.arange(64) - 31.5)        # many ties after scaling
        x[4, 100], x[4, 200] = 9.0, -9.0                    # |max| tie: first wins
    return x


@pytest.mark.parametrize("act", ["Q8_0", "Q8_K"])
def test_quantize_act_bit_exact(be, orc, act):
    at = getattr(B, act)
    for k, rows in [(256, 8), (4096, 5), (14336, 3)]:
        x = act_rows(k, rows, 21 + k)
        print(f"quantize {act} k={k} rows={rows}", flush=True)
        got = host(be.quantize_act(at, dev(x)))
        ref = np.concatenate([orc.quantize_act(at, x[r]) for r in range(rows)])
        assert np.array_equal(got, ref)


def test_quantize_q8_k_first_largest_magnitude(be, orc):
    """Q8_K's scale comes from the signed value of the FIRST element with the
    largest |x|; the device finds it by a wave maximum and a ballot (lane l
    holds elements 4l .. 4l + 3), so place ties inside one lane, across
    lanes with the later lane's element first in its lane, at the block's
    last element, and over a whole block."""
    k = 256
    rows = []
    b = synth.gen_f32(k, 31) * np.float32(0.5)
    b[8], b[11] = -5.0, 5.0            # one lane (2): element 0 of it wins
    rows.append(b)
    b = synth.gen_f32(k, 32) * np.float32(0.5)
    b[11], b[12] = 7.0, -7.0           # lanes 2 (last element) and 3 (first): index 11 wins
    rows.append(b)
    b = synth.gen_f32(k, 33) * np.float32(0.5)
    b[255] = -6.0                      # the very last element
    rows.append(b)
    b = np.where(np.arange(k) % 3 == 0, 1.0, -1.0).astype(np.float32)   # every |x| equal
    rows.append(b)
    b = synth.gen_f32(k, 34) * np.float32(0.5)
    b[200], b[17] = 3.0, -3.0          # the earlier index is in the lower lane
    rows.append(b)
    x = np.stack(rows).astype(np.float32)
    got = host(be.quantize_act(B.Q8_K, dev(x)))
    ref = np.concatenate([orc.quantize_act(B.Q8_K, r) for r in x])
    assert np.array_equal(got, ref)
    # the scale's sign follows the chosen element: d = 1 / (-127 / max)
    d = got.reshape(len(rows), 292)[:, :4].copy().view(np.float32)[:, 0]
    assert np.all(np.sign(d) == -np.sign(np.float32([-5.0, 7.0, -6.0, 1.0, -3.0])))


def test_quantize_q4_0_barq_bit_exact(be, orc):
    x = act_rows(4096, 6, 31).reshape(-1)
    got = host(be.quantize_q4_0_barq(dev(x)))
    assert np.array_equal(got, orc.q4_0_quantize_barq(x))


# ---- matvec ----------------------------------------------------------------

SHAPES_K = [(1, 256), (5, 512), (67, 4096), (33, 4352), (129, 14336), (1023, 768)]
SHAPES_32 = [(1, 32), (7, 96), (5, 64), (67, 4096), (33, 4128), (70, 4160), (130, 4064), (33, 14336)]


def shapes_for(t):
    return SHAPES_K if B.BLOCK_ELEMS[t] == 256 else SHAPES_32


@pytest.mark.parametrize("name", list(TYPES))
def test_matvec_q8_activations(be, orc, name):
    t = TYPES[name]
    at = B.Q8_PARTNER[t]
    for n, k in shapes_for(t):
        w = synth.gen_weights(t, n, k, 100 + n)
        x = synth.gen_f32(k, 200 + k)
        print(f"matvec {name} x {at} n={n} k={k}", flush=True)
        xq = be.quantize_act(at, dev(x))
        assert np.array_equal(host(xq), orc.quantize_act(at, x))
        y = host(be.matvec(t, dev(w), n, k, at, xq))
        ref = orc.matvec(t, w, n, k, at, host(xq))
        assert_close_1e3(y, ref)
        # library-side quantization gives the same result
        y2 = host(be.matvec(t, dev(w), n, k, B.ACT_F32_Q8, dev(x)))
        assert np.array_equal(y, y2)


@pytest.mark.parametrize("name", list(TYPES))
def test_matvec_f32_activations_literal(be, orc, name):
    # the literal reference path: gemv_f32(dequant(W), x)
    t = TYPES[name]
    for n, k in shapes_for(t):
        w = synth.gen_weights(t, n, k, 300 + n)
        x = synth.gen_f32(k, 400 + k)
        print(f"matvec {name} x f32 n={n} k={k}", flush=True)
        y = host(be.matvec(t, dev(w), n, k, B.ACT_F32, dev(x)))
        ref = orc.matvec(t, w, n, k, orc.F32, x)
        assert_close_1e3(y, ref, tol=1e-5)


def test_matvec_host_memory(be, orc):
    n, k = 100, 4096
    w = synth.gen_q4_k(n, k, 7)
    x = synth.gen_f32(k, 8)
    y = np.empty(n, np.float32)
    be.matvec_raw(B.Q4_K, w, n, k, B.ACT_F32_Q8, x, y, B.MEM_HOST)
    ref = orc.matvec(B.Q4_K, w, n, k, B.Q8_K, orc.quantize_q8_k(x))
    assert_close_1e3(y, ref)


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_matvec_full_baseline_configs(be, orc, cfg):
    """C1 Q4_0 4096x4096, C2 Q4_K 14336x4096, C3 Q6_K 128256x4096 at full size."""
    t, w, x = synth.linear_inputs(cfg)
    c = synth.CONFIGS[cfg]
    n, k = c["n_rows"], c["k"]
    at = B.Q8_PARTNER[t]
    print(f"full config C{cfg}", flush=True)
    xq = be.quantize_act(at, dev(x[0]))
    assert np.array_equal(host(xq), orc.quantize_act(at, x[0]))
    y = host(be.matvec(t, dev(w), n, k, at, xq))
    ref = orc.matvec(t, w, n, k, at, host(xq))
    assert_close_1e3(y, ref)
    # gap to the literal f32-activation reference, information only
    lit = orc.matvec(t, w, n, k, orc.F32, x[0])
    rel = float(np.linalg.norm(y.astype(np.float64) - lit) / np.linalg.norm(lit))
    print(f"C{cfg}: Q8-activation gap to literal f32 reference {rel:.2e}")
    assert rel < 2e-2


# ---- matmul ----------------------------------------------------------------

@pytest.mark.parametrize("name", list(TYPES))
def test_matmul_q8(be, orc, name):
    t = TYPES[name]
    at = B.Q8_PARTNER[t]
    k = 512 if B.BLOCK_ELEMS[t] == 256 else 256
    for n, m in [(40, 3), (96, 17), (257, 33)]:
        w = synth.gen_weights(t, n, k, 500 + n)
        x = synth.gen_f32(m * k, 600 + m).reshape(m, k)
        print(f"matmul {name} n={n} k={k} m={m}", flush=True)
        xq = be.quantize_act(at, dev(x))
        y = host(be.matmul(t, dev(w), n, k, at, xq, m))
        ref = orc.matmul(t, w, n, k, at, host(xq), m)
        assert_close_1e3(y, ref)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q4_0"])
def test_matmul_f32_literal_bit_exact(be, orc, name):
    # dequantize (bit-exact) + sequential unfused f32 GEMM == the reference's
    # gemm_f32(X, W^T) bit for bit
    t = TYPES[name]
    n, k, m = 70, 512, 5
    w = synth.gen_weights(t, n, k, 700)
    x = synth.gen_f32(m * k, 701).reshape(m, k)
    y = host(be.matmul(t, dev(w), n, k, B.ACT_F32, dev(x), m))
    assert_bits_equal(y, orc.matmul(t, w, n, k, orc.F32, x, m))


# ---- f32 BLAS and the split-scale API: bit-exact ------------------------------

def test_gemm_gemv_f32_reference_known_answers(be):
    a = np.float32([1, 2, 3, 4]); b = np.float32([5, 6, 7, 8])
    assert be.gemm_f32(a, b, 2, 2, 2, B.MEM_HOST).reshape(-1).tolist() == [19, 22, 43, 50]
    a = np.float32([1, 2, 3, 4, 5, 6]); b = np.float32([7, 8, 9, 10, 11, 12])
    assert be.gemm_f32(a, b, 2, 3, 2, B.MEM_HOST).reshape(-1).tolist() == [58, 64, 139, 154]
    assert be.gemv_f32(np.float32([1, 2, 3, 4]), np.float32([5, 6]), 2, 2, B.MEM_HOST).tolist() == [17, 39]
    assert be.gemv_f32(np.float32([1e8, 1, -1e8]), np.float32([1, 1, 1]), 1, 3, B.MEM_HOST)[0] == 0.0


def test_gemm_gemv_f32_bit_exact(be, orc):
    rng = np.random.default_rng(9)
    for m, k, n in [(1, 4096, 300), (67, 129, 65), (128, 256, 192)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        assert_bits_equal(host(be.gemm_f32(dev(a), dev(b), m, k, n)), orc.gemm_f32(a, b, m, k, n))
    a = rng.standard_normal((1000, 4099)).astype(np.float32)
    x = rng.standard_normal(4099).astype(np.float32)
    assert_bits_equal(host(be.gemv_f32(dev(a), dev(x), 1000, 4099)), orc.gemv_f32(a, x, 1000, 4099))


def test_split_api_bit_exact(be, orc):
    rng = np.random.default_rng(10)
    for bs in (32, 256, 5):
        nsc = 40
        q = rng.integers(0, 256, nsc * ((bs + 1) // 2) - 3).astype(np.uint8)
        s = rng.standard_normal(nsc).astype(np.float32)
        for kind_q8 in (False, True):
            qq = rng.integers(0, 256, nsc * bs - 3).astype(np.uint8) if kind_q8 else q
            got = be.dequantize_split(B.Q8_0 if kind_q8 else B.Q4_K, qq, s, bs, nsc * bs + 7)
            assert_bits_equal(got, orc.dequantize_split(kind_q8, qq, s, bs, nsc * bs + 7))
    # the reference's own tests (cuda_quant.rs:345-373)
    assert be.dequantize_split(B.Q4_K, np.uint8([0x88, 0x88]), np.float32([1.0]), 4, 4).tolist() == [-8.0] * 4
    c = be.quantized_matmul_split(np.float32([1, 2, 3, 4]), np.uint8([0x11, 0x11]), np.float32([1.0]), 2, 2, 2, B.Q4_K, 4)
    assert c.reshape(-1).tolist() == [3.0, 3.0, 7.0, 7.0]
    m, n, k = 9, 40, 96
    a = rng.standard_normal((m, k)).astype(np.float32)
    bq = rng.integers(0, 256, k * n // 2).astype(np.uint8)
    bsc = rng.standard_normal(k * n // 32).astype(np.float32)
    got = be.quantized_matmul_split(a, bq, bsc, m, n, k, B.Q4_K, 32)
    assert_bits_equal(got, orc.quantized_matmul_split(a, bq, bsc, m, n, k, False, 32))


# ---- MoE -------------------------------------------------------------------

def test_moe_route(be, orc):
    logits = synth.gen_f32(64 * 8, 5).reshape(64, 8)
    logits[3, :] = np.float32([1, 3, 3, 0, 0, 0, 0, 0])      # tie: lower index first
    ids, w = be.moe_route(dev(logits), 64, 8, 2)
    rid, rw = orc.moe_select_top_k(logits, 2)
    assert np.array_equal(host(ids), rid)
    assert np.allclose(host(w), rw, rtol=1e-6, atol=1e-7)
    ids, _ = be.moe_route(np.float32([[0.1, 2.0, 1.0, -1.0], [3.0, 0.0, 1.5, 1.0]]), 2, 4, 2, B.MEM_HOST)
    assert ids.tolist() == [[1, 2], [0, 2]]


def test_moe_route_reduce_and_reduce(be, orc):
    """Smart expert reduction (reduce_expert_assignments, moe_fused.rs:147-194)
    after top-k routing, fused into the routing launch and on its own:
    tokens with a wide logit gap lose their second expert at the default
    threshold 0.05 (advanced/src/moe.rs:24-31)."""
    rows, ne, k = 96, 8, 3
    logits = synth.gen_f32(rows * ne, 77).reshape(rows, ne)
    logits[::3, 5] += 4.0                      # a dominant expert: the others fall below 0.05
    logits[1::7, :] = 0.0                      # all equal: ties, nothing dropped at k = 3
    rid, rw = orc.moe_select_top_k(logits, k)
    ref_i, ref_w = orc.moe_reduce_experts(rid, rw, 2, 0.05)
    assert (ref_i[:, 1] < 0).sum() > 10 and (ref_i[:, 1] >= 0).sum() > 10
    # standalone reduce on the oracle's routing: bit-exact
    gi, gw = be.moe_reduce(dev(rid), dev(rw), 2, 0.05)
    assert np.array_equal(host(gi), ref_i)
    assert_bits_equal(host(gw), ref_w)
    gi, gw = be.moe_reduce(rid, rw, 2, 0.05, mem=B.MEM_HOST)
    assert np.array_equal(gi, ref_i)
    # in place
    ti, tw = dev(rid), dev(rw)
    be.moe_reduce(ti, tw, 2, 0.05, out=(ti, tw))
    assert np.array_equal(host(ti), ref_i)
    # fused with the routing (device expf: weights within float rounding)
    fi, fw = be.moe_route_reduce(dev(logits), rows, ne, k, 2, 0.05)
    assert np.array_equal(host(fi), ref_i)
    assert np.allclose(host(fw), ref_w, rtol=1e-6, atol=1e-7)
    # the reference's own test (moe_fused.rs:338-350)
    gi, gw = be.moe_reduce(np.int32([[0, 1, 2], [2, 1, 0]]), np.float32([[0.7, 0.2, 0.1], [0.4, 0.35, 0.25]]), 2, 0.15,
                           mem=B.MEM_HOST)
    assert gi.tolist() == [[0, 1, -1], [2, 1, -1]]
    assert np.all(np.abs(gw.sum(1) - 1.0) < 1e-6)
    # "no cap" (usize::MAX, or anything >= 2^31): every slot above the
    # threshold is kept and renormalised, as in the oracle
    for cap in (2**64 - 1, 2**31, k + 1):
        ref_i, ref_w = orc.moe_reduce_experts(rid, rw, cap, 0.05)
        assert (ref_i[:, 2] >= 0).sum() > 10
        gi, gw = be.moe_reduce(dev(rid), dev(rw), cap, 0.05)
        assert np.array_equal(host(gi), ref_i)
        assert_bits_equal(host(gw), ref_w)
        fi, fw = be.moe_route_reduce(dev(logits), rows, ne, k, cap, 0.05)
        assert np.array_equal(host(fi), ref_i)
        assert np.allclose(host(fw), ref_w, rtol=1e-6, atol=1e-7)


def test_moe_ffn_after_reduction(be, orc):
    """The MoE step on reduced assignments (dropped slots are id -1): the
    experts each token keeps, weighted by the renormalised weights."""
    ne, hid, nff, rows, k = 6, 512, 1024, 40, 2
    gates, ups, downs, x, _, _ = _moe_case(orc, ne, hid, nff, rows, k, 880)
    logits = synth.gen_f32(rows * ne, 881).reshape(rows, ne)
    logits[::2, 3] += 5.0
    ids, w = orc.moe_select_top_k(logits, k)
    ids, w = orc.moe_reduce_experts(ids, w, k, 0.05)
    assert (ids[:, 1] < 0).sum() >= 10
    out = be.moe_ffn(B.Q4_K, [dev(g) for g in gates], B.Q4_K, [dev(u) for u in ups], B.Q6_K, [dev(d) for d in downs],
                     hid, nff, dev(x), rows, dev(ids), dev(w), k, B.ACT_F32_Q8)
    ref = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x, ids, w, orc.Q8_K)
    assert_close_1e3(host(out), ref)


@pytest.mark.parametrize("act", ["q8", "f32"])
def test_moe_ffn_small(be, orc, act):
    ne, hid, nff, rows, k = 4, 512, 1024, 24, 2
    gates = [synth.gen_q4_k(nff, hid, 10 + e) for e in range(ne)]
    ups = [synth.gen_q4_k(nff, hid, 20 + e) for e in range(ne)]
    downs = [synth.gen_q6_k(hid, nff, 30 + e) for e in range(ne)]
    x = synth.gen_f32(rows * hid, 40).reshape(rows, hid)
    ids, w = orc.moe_select_top_k(synth.gen_f32(rows * ne, 41).reshape(rows, ne), k)
    a = B.ACT_F32_Q8 if act == "q8" else B.ACT_F32
    out = be.moe_ffn(B.Q4_K, [dev(g) for g in gates], B.Q4_K, [dev(u) for u in ups], B.Q6_K,
                     [dev(d) for d in downs], hid, nff, dev(x), rows, dev(ids), dev(w), k, a)
    ref = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x, ids, w,
                      orc.Q8_K if act == "q8" else orc.F32)
    assert_close_1e3(host(out), ref)
    # host-memory entry point gives the same result
    out_h = be.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x, rows, ids, w, k, a, mem=B.MEM_HOST)
    assert np.array_equal(out_h, host(out))


def _moe_case(orc, ne, hid, nff, rows, k, seed, gt=B.Q4_K, ut=B.Q4_K, dt=B.Q6_K):
    gen = {B.Q4_K: synth.gen_q4_k, B.Q6_K: synth.gen_q6_k}
    gates = [gen[gt](nff, hid, seed + e) for e in range(ne)]
    ups = [gen[ut](nff, hid, seed + 100 + e) for e in range(ne)]
    downs = [gen[dt](hid, nff, seed + 200 + e) for e in range(ne)]
    x = synth.gen_f32(rows * hid, seed + 300).reshape(rows, hid)
    ids, w = orc.moe_select_top_k(synth.gen_f32(rows * ne, seed + 301).reshape(rows, ne), k)
    return gates, ups, downs, x, np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(w, np.float32)


# Expert-grouped integer path (one launch per weight set, row ranges read on
# the device): skewed and empty experts, skipped and repeated ids, more
# experts than one launch carries, mixed gate/up types, 64-row tiles, and the
# per-expert fallback for Q6_K with an odd number of super-blocks.
MOE_CASES = {
    "skew": dict(ne=5, hid=512, nff=1024, rows=40, k=2),
    "many_experts": dict(ne=40, hid=256, nff=512, rows=24, k=3),
    "mixed_types": dict(ne=3, hid=512, nff=512, rows=20, k=2, gt=B.Q6_K, ut=B.Q4_K),
    "wide_tiles": dict(ne=2, hid=256, nff=512, rows=80, k=2),
    "odd_q6k_fallback": dict(ne=3, hid=256, nff=768, rows=12, k=2),
    # more tiles than workgroups, so each workgroup streams several tiles
    # through one pipeline: gate/up 8 x 2 x 64 tiles; down 24 x 32 tiles
    "multi_tile_gate_up": dict(ne=8, hid=512, nff=8192, rows=16, k=2),
    "multi_tile_down": dict(ne=24, hid=4096, nff=512, rows=24, k=2),
    # five super-blocks per row (an odd count for the Q4_K tiles), experts
    # of up to ~40 rows
    "nsb5": dict(ne=5, hid=1280, nff=512, rows=70, k=2),
    # grouping fused with the gather-quantize over several 256-assignment
    # chunks (with skipped ids)
    "many_chunks": dict(ne=6, hid=256, nff=256, rows=700, k=2),
    # decode-size steps (at most 4 assignments): expert-grouped GEMVs
    "decode_1": dict(ne=8, hid=512, nff=1024, rows=1, k=2),
    "decode_1_repeat": dict(ne=4, hid=256, nff=512, rows=1, k=2),
    "decode_2_repeat": dict(ne=4, hid=256, nff=512, rows=2, k=2),
    "decode_top1": dict(ne=3, hid=512, nff=512, rows=4, k=1),
    "decode_mixed": dict(ne=3, hid=512, nff=512, rows=2, k=2, gt=B.Q6_K, ut=B.Q4_K),
    # decode with a down projection over several 4096-element chunks, the
    # last one partial (k = 5120 and 14336, Mixtral's n_ff)
    "decode_long_k": dict(ne=4, hid=256, nff=5120, rows=1, k=2),
    "decode_mixtral_nff": dict(ne=2, hid=512, nff=14336, rows=1, k=2),
}


@pytest.mark.parametrize("name", list(MOE_CASES))
def test_moe_ffn_grouped_cases(be, orc, name):
    c = dict(MOE_CASES[name])
    ne, hid, nff, rows, k = c.pop("ne"), c.pop("hid"), c.pop("nff"), c.pop("rows"), c.pop("k")
    gt, ut, dt = c.get("gt", B.Q4_K), c.get("ut", B.Q4_K), B.Q6_K
    gates, ups, downs, x, ids, w = _moe_case(orc, ne, hid, nff, rows, k, 500 + len(name), gt, ut, dt)
    if name == "skew":
        ids[:, 0] = 0           # expert 0: 40 rows (two 32-row tiles); expert 3 stays empty
        ids[:, 1] = np.where(ids[:, 1] == 3, 1, ids[:, 1])
        ids[ids[:, 1] == 0, 1] = 2
        ids[5, 1] = -1          # skipped ids
        ids[6, 1] = ne
        ids[7, :] = [2, 2]      # a repeated expert
    if name == "many_chunks":
        ids[::37, 1] = -1       # skipped ids spread over the chunks
        ids[300, :] = [5, 5]
    if name == "decode_1_repeat":
        ids[:] = [[2, 2]]           # one token, the same expert twice: two passes
    if name == "decode_2_repeat":
        ids[:] = [[3, 3], [3, 1]]   # three rows on one expert
    if name == "decode_top1":
        ids[:, 0] = 1               # four rows on one expert
    out = be.moe_ffn(gt, [dev(g) for g in gates], ut, [dev(u) for u in ups], dt, [dev(d) for d in downs], hid, nff,
                     dev(x), rows, dev(ids), dev(w), k, B.ACT_F32_Q8)
    ref = orc.moe_ffn(gt, gates, ut, ups, dt, downs, hid, nff, x, ids, w, orc.Q8_K)
    assert_close_1e3(host(out), ref)
    if name.startswith("decode"):
        # the same step on the grouped MFMA GEMM (0) and on the grouped GEMVs
        # (2: also for more than one token, several rows per expert)
        for mode in ("0", "2"):
            with tuned(BARQ_MOE_GEMV=mode) as b:
                out2 = b.moe_ffn(gt, [dev(g) for g in gates], ut, [dev(u) for u in ups], dt, [dev(d) for d in downs],
                                 hid, nff, dev(x), rows, dev(ids), dev(w), k, B.ACT_F32_Q8)
            assert_close_1e3(host(out2), ref)
    if name == "many_chunks":
        # grouping in its own launch (the path above 2048 assignments, or with
        # BARQ_MOE_FUSED_GROUP=0) gives the same rows in the same order
        with tuned(BARQ_MOE_FUSED_GROUP=0) as b:
            out2 = b.moe_ffn(gt, [dev(g) for g in gates], ut, [dev(u) for u in ups], dt, [dev(d) for d in downs], hid,
                             nff, dev(x), rows, dev(ids), dev(w), k, B.ACT_F32_Q8)
        assert np.array_equal(host(out2), host(out))


# ---- the quant crate's own Q4_K (quant/src/q4_k.rs): encode and decode bit-exact ----
@pytest.mark.parametrize("n", [256, 256 * 37, 256 * 5 + 37, 100, 1])
def test_q4_k_barq_quantize_and_dequantize_bit_exact(be, orc, n):
    x = synth.gen_f32(n, 600 + n)
    x[::97] *= 40.0
    ref = orc.q4_k_barq_quantize(x)
    got = be.quantize_q4_k_barq(dev(x)).cpu().numpy()
    assert np.array_equal(got, ref)
    assert np.array_equal(be.quantize_q4_k_barq(x, mem=B.MEM_HOST), ref)
    whole = n // 256 * 256
    if whole:
        deq = be.dequantize(B.Q4_K_BARQ, dev(ref[:whole // 256 * 136]), whole).cpu().numpy()
        assert_bits_equal(deq, orc.q4_k_barq_dequantize(ref, whole))
