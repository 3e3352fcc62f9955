"""Every launch-shape override the kernels accept (the BARQ_GEMM_*,
BARQ_GEMV_*, BARQ_MOE_* and BARQ_ATTN_* tuning variables, read when a handle
is created) against the oracle, in one process: each variant runs on a
fresh handle created under its settings.  The variants that measured slower
stay off by default but must still compute the same product.  Bars as in
test_gpu_parity.py / test_gpu_attention.py."""
import contextlib
import os

import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import attention as A
from barq_rocm import synth
from conftest import assert_close_1e3

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@contextlib.contextmanager
def env(**kv):
    """A handle created with the tuning variables kv set (the library reads
    them at handle creation); the environment is restored before the body."""
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


def matmul_case(orc, w_type, n, k, m, seed):
    w = synth.gen_weights(w_type, n, k, seed)
    x = synth.gen_f32(m * k, seed + 1).reshape(m, k)
    xq = orc.quantize_act(B.Q8_PARTNER[w_type], x)
    return w, xq, orc.matmul(w_type, w, n, k, B.Q8_PARTNER[w_type], xq, m)


GEMM_VARIANTS = [
    dict(BARQ_GEMM_KG=1), dict(BARQ_GEMM_KG=2), dict(BARQ_GEMM_BM=32), dict(BARQ_GEMM_BM=64),
    dict(BARQ_GEMM_BM=65), dict(BARQ_GEMM_BM=65, BARQ_GEMM_KG=1), dict(BARQ_GEMM_BM=64, BARQ_GEMM_KG=1), dict(BARQ_GEMM_BM=16), dict(BARQ_GEMM_BM=16, BARQ_GEMM_NS=2),
    dict(BARQ_GEMM_BM=16, BARQ_GEMM_NS=4), dict(BARQ_GEMM_BM=32, BARQ_GEMM_KG=1, BARQ_GEMM_NS=2),
    dict(BARQ_GEMM_BM=32, BARQ_GEMM_KG=1, BARQ_GEMM_NS=3), dict(BARQ_GEMM_BM=32, BARQ_GEMM_KG=1, BARQ_GEMM_NS=4),
    dict(BARQ_GEMM_BM=32, BARQ_GEMM_KG=1), dict(BARQ_GEMM_XCD=0), dict(BARQ_GEMM_IMPL=0),
    dict(BARQ_GEMM_KS=1), dict(BARQ_GEMM_KS=2), dict(BARQ_GEMM_KS=4, BARQ_GEMM_KG=1),
    dict(BARQ_GEMM_KS=2, BARQ_GEMM_BM=16), dict(BARQ_GEMM_KS=2, BARQ_GEMM_BM=65), dict(BARQ_GEMM_KS=4, BARQ_GEMM_BM=32),
    dict(BARQ_GEMM_DEFER=1), dict(BARQ_GEMM_DEFER=0), dict(BARQ_GEMM_DEFER=1, BARQ_GEMM_KS=2),
    dict(BARQ_GEMM_DEFER=2), dict(BARQ_GEMM_DEFER=3), dict(BARQ_GEMM_DEFER=3, BARQ_GEMM_KS=2), dict(BARQ_GEMM_DEFER=2, BARQ_GEMM_KS=4),
    dict(BARQ_GEMM_BM=66), dict(BARQ_GEMM_BM=66, BARQ_GEMM_KS=2), dict(BARQ_GEMM_BM=67), dict(BARQ_GEMM_BM=67, BARQ_GEMM_KS=2),
]


@pytest.mark.parametrize("name", ["Q4_0", "Q8_0", "Q4_0_BARQ"])
def test_gemm_32_element_blocks(be, orc, name):
    """Batched GEMM for the 32-element block formats (int8 MFMA, one block per
    MFMA): ragged tiles in M and N, 32- and 64-row tiles, K split across
    workgroups (the default for few tiles, and each override), the
    host-buffer path, and k not a multiple of 256 (per-row GEMV fallback)."""
    import torch
    t = getattr(B, name)
    at = B.Q8_PARTNER[t]
    for n, k, m, env_v in [(300, 512, 16, {}), (128, 1024, 40, {}), (257, 768, 97, {}), (64, 256, 33, dict(BARQ_GEMM_BM=32)),
                           (200, 512, 70, dict(BARQ_GEMM_BM=64)), (130, 512, 18, dict(BARQ_GEMM_XCD=0)), (96, 288, 20, {}),
                           (160, 1024, 50, dict(BARQ_GEMM_KG=1)), (160, 1024, 50, dict(BARQ_GEMM_KG=2)),
                           (160, 1024, 50, dict(BARQ_GEMM_KG=4)), (160, 768, 20, dict(BARQ_GEMM_KG=4, BARQ_GEMM_BM=32)),
                           (257, 2048, 17, {}), (160, 1024, 50, dict(BARQ_GEMM_KS=1)), (160, 1024, 50, dict(BARQ_GEMM_KS=4)),
                           (160, 1024, 50, dict(BARQ_GEMM_KS=2, BARQ_GEMM_KG=4)), (131, 1024, 19, dict(BARQ_GEMM_KS=4, BARQ_GEMM_KG=1)),
                           (1100, 512, 33, dict(BARQ_GEMM_KS=2)), (500, 4096, 16, {})]:   # the last: 16 K slices
        w = synth.gen_weights(t, n, k, 900 + n + k)
        x = synth.gen_f32(m * k, 901 + m).reshape(m, k)
        xq = orc.quantize_act(at, x)
        ref = orc.matmul(t, w, n, k, at, xq, m)
        print(f"gemm {name} n={n} k={k} m={m} {env_v}", flush=True)
        with env(**env_v) as b:
            got = b.matmul(t, dev(w), n, k, at, dev(xq), m).cpu().numpy()
            assert_close_1e3(got, ref)
            y = np.empty((m, n), np.float32)
            b.matmul_raw(t, w, n, k, at, xq, m, y, B.MEM_HOST)
            assert_close_1e3(y, ref)
            # f32 activations quantized inside the call
            got_f = b.matmul(t, dev(w), n, k, B.ACT_F32_Q8, dev(x), m).cpu().numpy()
            assert_close_1e3(got_f, ref)


@pytest.mark.parametrize("w_type", [B.Q4_K, B.Q6_K])
def test_gemm_variants(be, orc, w_type):
    n, k, m = 384, 2048, 72
    w, xq, ref = matmul_case(orc, w_type, n, k, m, 900 + w_type)
    wd, xd = dev(w), dev(xq)
    for v in GEMM_VARIANTS:
        print("gemm variant", w_type, v, flush=True)
        with env(**v) as b:
            got = b.matmul(w_type, wd, n, k, B.Q8_PARTNER[w_type], xd, m).cpu().numpy()
        assert_close_1e3(got, ref)


@pytest.mark.parametrize("w_type", [B.Q4_K, B.Q6_K])
def test_gemm_k_slices(be, orc, w_type):
    """Few tiles split K across workgroups (the slices' partial products are
    added in order): ragged M and N at the slice counts the automatic choice
    makes (one to eight), device and host buffers, and f32 activations
    quantized in the call (the quantized rows and the partials share the
    workspace)."""
    for n, k, m in [(1000, 4096, 16), (130, 2048, 17), (300, 1024, 40), (4100, 512, 33), (129, 4096, 100),
                    (256, 8192, 128)]:   # the last: Q6_K's 64-row four-wave tiles by default (long K)
        w, xq, ref = matmul_case(orc, w_type, n, k, m, 700 + n + m)
        print(f"k slices {w_type} n={n} k={k} m={m}", flush=True)
        got = be.matmul(w_type, dev(w), n, k, B.Q8_PARTNER[w_type], dev(xq), m).cpu().numpy()
        assert_close_1e3(got, ref)
        y = np.empty((m, n), np.float32)
        be.matmul_raw(w_type, w, n, k, B.Q8_PARTNER[w_type], xq, m, y, B.MEM_HOST)
        assert_close_1e3(y, ref)
        x = synth.gen_f32(m * k, 700 + n + m + 1).reshape(m, k)   # the rows matmul_case quantized
        got_f = be.matmul(w_type, dev(w), n, k, B.ACT_F32_Q8, dev(x), m).cpu().numpy()
        assert_close_1e3(got_f, ref)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q4_0", "Q8_0", "Q4_0_BARQ"])
def test_matmul_small_m(be, orc, name):
    """A few activation rows: 2-4 rows run one GEMV over all of them (for
    Q4_K the LDS-staged GEMV up to k = 4096 and the register GEMV above, the
    LDS-streamed one for the other formats; k = 5120 adds a second, partial
    4096-element chunk), 5 and more the MFMA
    GEMMs; each M also with the GEMM and the per-row GEMVs forced
    (BARQ_GEMM_MIN_M=2 or 16 with the multi-row GEMV off), device and host
    buffers."""
    t = getattr(B, name)
    at = B.Q8_PARTNER[t]
    # above 8192 rows the 32-element formats take another multi-token launch shape
    shapes = [(300, 1024), (77, 5120), (8200, 512)]
    variants = [{}, dict(BARQ_GEMM_MIN_M=2, BARQ_GEMV_MULTI_MAX=0), dict(BARQ_GEMM_MIN_M=16, BARQ_GEMV_MULTI_MAX=0)]
    for n, k in shapes:
        w = synth.gen_weights(t, n, k, 820)
        wd = dev(w)
        for m in (2, 3, 4, 7, 15):
            x = synth.gen_f32(m * k, 821 + m).reshape(m, k)
            xq = orc.quantize_act(at, x)
            ref = orc.matmul(t, w, n, k, at, xq, m)
            for env_v in variants:
                print(f"small m {name} n={n} k={k} m={m} {env_v}", flush=True)
                with env(**env_v) as b:
                    assert_close_1e3(b.matmul(t, wd, n, k, at, dev(xq), m).cpu().numpy(), ref)
                    y = np.empty((m, n), np.float32)
                    b.matmul_raw(t, w, n, k, at, xq, m, y, B.MEM_HOST)
                    assert_close_1e3(y, ref)


GEMV_VARIANTS = [dict(BARQ_GEMV_DMA=c) for c in (-1, 422, 444, 482, 822, 842, 222, 242, 411, 811)] + [
    dict(BARQ_GEMV_DMA_TYPES=0), dict(BARQ_GEMV_DMA_TYPES=31), dict(BARQ_GEMV_LDS=0)] + [
    dict(BARQ_GEMV_DMA_TYPES=0, BARQ_GEMV_CFG=c) for c in ("1,4", "2,4", "4,4", "8,4", "1,8", "2,8", "4,8", "2,2",
                                                          "4,2", "8,2", "4,1")]


@pytest.mark.parametrize("w_type", [B.Q4_K, B.Q6_K, B.Q4_0, B.Q8_0])
def test_gemv_variants(be, orc, w_type):
    # one 4096-element slice, and a down-projection-like shape of 3.5 slices
    for n, k in [(517, 4096), (203, 14336)]:
        w, xq, ref = matmul_case(orc, w_type, n, k, 1, 950 + w_type + k)
        wd, xd = dev(w), dev(xq)
        for v in GEMV_VARIANTS:
            print("gemv variant", w_type, n, k, v, flush=True)
            with env(**v) as b:
                got = b.matvec(w_type, wd, n, k, B.Q8_PARTNER[w_type], xd).cpu().numpy()
            assert_close_1e3(got, ref.ravel())


def test_gemv_q4k_lds_equals_register_gemv(be, orc):
    """The LDS-staged Q4_K GEMV (k <= 4096, the default there: one row per
    wave up to 4096 rows, two above) against the register GEMV
    (BARQ_GEMV_LDS=0), with one, two and four rows per wave forced
    (BARQ_GEMV_LDS=3, 2, 4): bit-identical outputs (same lane slices,
    arithmetic and reduction), all within the bar of the oracle.  Row counts
    that are not a multiple of the rows per wave leave the last wave short;
    short k leaves lanes idle and changes how many copies each row's wait
    skips; 4096 and 4097 rows sit either side of the default's switch."""
    from conftest import assert_bits_equal
    for n, k in [(1, 256), (5, 512), (67, 4096), (129, 3840), (1023, 768), (14336, 4096), (3, 4096), (30, 2304),
                 (4096, 4096), (4097, 4096)]:
        print("q4k lds gemv", n, k, flush=True)
        w, xq, ref = matmul_case(orc, B.Q4_K, n, k, 1, 1300 + n + k)
        wd, xd = dev(w), dev(xq)
        got = be.matvec(B.Q4_K, wd, n, k, B.Q8_K, xd).cpu().numpy()
        with env(BARQ_GEMV_LDS=0) as b:
            reg = b.matvec(B.Q4_K, wd, n, k, B.Q8_K, xd).cpu().numpy()
        # one, two and four rows per wave: the same per-row arithmetic and reduction
        forced = {}
        for mode in (3, 2, 4):
            with env(BARQ_GEMV_LDS=mode) as b:
                forced[mode] = b.matvec(B.Q4_K, wd, n, k, B.Q8_K, xd).cpu().numpy()
        assert_bits_equal(got, reg)
        for mode, y in forced.items():
            assert_bits_equal(y, reg)
        assert_close_1e3(got, ref.ravel())


def test_gemv_q4k_lds_multi_equals_one_token_gemv(be, orc):
    """2-4 activation rows on the LDS-staged Q4_K GEMV (the default for k <=
    4096; four or, with BARQ_GEMV_LDS=2, two weight rows per wave): row j of
    the result equals the one-token GEMV of activation row j bit for bit, and
    the oracle within its bar.  Ragged row counts, short k."""
    from conftest import assert_bits_equal
    for n, k in [(300, 4096), (14336, 4096), (37, 512), (1, 256), (8203, 1024)]:
        for m in (2, 3, 4):
            print("q4_k lds multi", n, k, m, flush=True)
            w, xq, ref = matmul_case(orc, B.Q4_K, n, k, m, 2500 + n + k + m)
            wd, xd = dev(w), dev(xq)
            rb = B.row_bytes(B.Q8_K, k)
            one = [be.matvec(B.Q4_K, wd, n, k, B.Q8_K, xd[j * rb:(j + 1) * rb]).cpu().numpy() for j in range(m)]
            got = be.matmul(B.Q4_K, wd, n, k, B.Q8_K, xd, m).cpu().numpy().reshape(m, n)
            with env(BARQ_GEMV_LDS=2) as b:
                pair = b.matmul(B.Q4_K, wd, n, k, B.Q8_K, xd, m).cpu().numpy().reshape(m, n)
            with env(BARQ_GEMV_LDS=0) as b:   # the register multi-row GEMV
                reg = b.matmul(B.Q4_K, wd, n, k, B.Q8_K, xd, m).cpu().numpy().reshape(m, n)
            for j in range(m):
                assert_bits_equal(got[j], one[j])
                assert_bits_equal(pair[j], one[j])
            assert_close_1e3(got, ref)
            assert_close_1e3(reg, ref)


def test_gemv_q6_k_pairs_equal_dma_gemv(be, orc):
    """The two-row LDS-staged Q6_K GEMV (the default for k <= 4096) against
    the LDS-streamed GEMV (BARQ_GEMV_LDS=0): bit-identical outputs, both
    within the bar of the oracle (both default launch shapes of the streamed
    GEMV: one row per wave up to 8192 rows, four above)."""
    from conftest import assert_bits_equal
    for n, k in [(1, 512), (7, 1024), (300, 4096), (4096, 4096), (129, 3584), (8201, 4096)]:
        print("q6_k pair gemv", n, k, flush=True)
        w, xq, ref = matmul_case(orc, B.Q6_K, n, k, 1, 2100 + n + k)
        wd, xd = dev(w), dev(xq)
        got = be.matvec(B.Q6_K, wd, n, k, B.Q8_K, xd).cpu().numpy()
        with env(BARQ_GEMV_LDS=0) as b:
            base = b.matvec(B.Q6_K, wd, n, k, B.Q8_K, xd).cpu().numpy()
        assert_bits_equal(got, base)
        assert_close_1e3(got, ref.ravel())


def test_gemv_q6_k_pairs_multi_equal_one_token_gemv(be, orc):
    """2-4 activation rows on the two-row Q6_K GEMV (the default for k <=
    4096): row j of the result equals the one-token GEMV of activation row j
    bit for bit, the LDS-streamed multi-token GEMV (BARQ_GEMV_LDS=0) and the
    oracle within the bar.  Odd row counts, short k, more than 8192 rows."""
    from conftest import assert_bits_equal
    for n, k in [(300, 4096), (129, 3584), (1, 512), (8201, 1024)]:
        for m in (2, 3, 4):
            print("q6_k pair multi", n, k, m, flush=True)
            w, xq, ref = matmul_case(orc, B.Q6_K, n, k, m, 2700 + n + k + m)
            wd, xd = dev(w), dev(xq)
            rb = B.row_bytes(B.Q8_K, k)
            one = [be.matvec(B.Q6_K, wd, n, k, B.Q8_K, xd[j * rb:(j + 1) * rb]).cpu().numpy() for j in range(m)]
            got = be.matmul(B.Q6_K, wd, n, k, B.Q8_K, xd, m).cpu().numpy().reshape(m, n)
            with env(BARQ_GEMV_LDS=0) as b:
                base = b.matmul(B.Q6_K, wd, n, k, B.Q8_K, xd, m).cpu().numpy().reshape(m, n)
            for j in range(m):
                assert_bits_equal(got[j], one[j])
            assert_close_1e3(got, ref)
            assert_close_1e3(base, ref)


@pytest.mark.parametrize("name", ["Q4_0", "Q8_0", "Q4_0_BARQ"])
def test_gemv_32_element_pairs_multi_equal_one_token_gemv(be, orc, name):
    """2-4 activation rows on the two-row GEMV of the 32-element formats (the
    default for k <= 4096): row j equals the one-token GEMV of activation
    row j bit for bit; the LDS-streamed multi-token GEMV (BARQ_GEMV_LDS=0)
    and the oracle within the bar."""
    from conftest import assert_bits_equal
    t = getattr(B, name)
    at = B.Q8_PARTNER[t]
    for n, k in [(300, 4096), (129, 2048), (1, 256), (8201, 1024)]:
        for m in (2, 3, 4):
            print(name, "pair multi", n, k, m, flush=True)
            w, xq, ref = matmul_case(orc, t, n, k, m, 2900 + n + k + m)
            wd, xd = dev(w), dev(xq)
            rb = B.row_bytes(at, k)
            one = [be.matvec(t, wd, n, k, at, xd[j * rb:(j + 1) * rb]).cpu().numpy() for j in range(m)]
            got = be.matmul(t, wd, n, k, at, xd, m).cpu().numpy().reshape(m, n)
            with env(BARQ_GEMV_LDS=0) as b:
                base = b.matmul(t, wd, n, k, at, xd, m).cpu().numpy().reshape(m, n)
            for j in range(m):
                assert_bits_equal(got[j], one[j])
            assert_close_1e3(got, ref)
            assert_close_1e3(base, ref)


@pytest.mark.parametrize("name", ["Q4_0", "Q8_0", "Q4_0_BARQ"])
def test_gemv_32_element_pairs_equal_dma_gemv(be, orc, name):
    """The LDS-staged GEMV of the 32-element formats (the default for k <=
    4096: one weight row per wave up to 1024 rows, two above; BARQ_GEMV_LDS
    = 3 / 2 force one / two) against the LDS-streamed one-row-per-wave GEMV
    (BARQ_GEMV_LDS=0): bit-identical outputs (same lane slicing, arithmetic
    and reduction), all within the bar of the oracle; odd row counts leave
    the last wave one row, short k leaves lanes idle; 1024 and 1025 rows sit
    either side of the default's switch."""
    from conftest import assert_bits_equal
    t = getattr(B, name)
    for n, k in [(1, 256), (7, 512), (300, 4096), (4096, 4096), (129, 1280), (64, 3840), (1024, 4096),
                 (1025, 2048)]:
        print(f"{name} pair gemv", n, k, flush=True)
        w, xq, ref = matmul_case(orc, t, n, k, 1, 1900 + n + k)
        wd, xd = dev(w), dev(xq)
        got = be.matvec(t, wd, n, k, B.Q8_PARTNER[t], xd).cpu().numpy()
        with env(BARQ_GEMV_LDS=0) as b:
            base = b.matvec(t, wd, n, k, B.Q8_PARTNER[t], xd).cpu().numpy()
        assert_bits_equal(got, base)
        for mode in (3, 2):
            with env(BARQ_GEMV_LDS=mode) as b:
                assert_bits_equal(b.matvec(t, wd, n, k, B.Q8_PARTNER[t], xd).cpu().numpy(), base)
        assert_close_1e3(got, ref.ravel())


MOE_VARIANTS = [dict(BARQ_GEMM_BM=16), dict(BARQ_GEMM_BM=16, BARQ_GEMM_NS=4), dict(BARQ_GEMM_NS=3),
                dict(BARQ_GEMM_NS=4), dict(BARQ_GEMM_KS=1), dict(BARQ_GEMM_KS=2), dict(BARQ_GEMM_KS=4)]


def test_moe_variants(be, orc):
    ne, hid, nff, rows, k = 6, 512, 2048, 40, 2
    gates = [synth.gen_q4_k(nff, hid, 70 + e) for e in range(ne)]
    ups = [synth.gen_q4_k(nff, hid, 80 + e) for e in range(ne)]
    downs = [synth.gen_q6_k(hid, nff, 90 + e) for e in range(ne)]
    x = synth.gen_f32(rows * hid, 99).reshape(rows, hid)
    ids, w = orc.moe_select_top_k(synth.gen_f32(rows * ne, 98).reshape(rows, ne), k)
    ids, w = np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(w, np.float32)
    ref = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x, ids, w, orc.Q8_K)
    gd, ud, dd = [dev(a) for a in gates], [dev(a) for a in ups], [dev(a) for a in downs]
    for v in MOE_VARIANTS:
        print("moe variant", v, flush=True)
        with env(**v) as b:
            got = b.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hid, nff, dev(x), rows, dev(ids), dev(w), k,
                            B.ACT_F32_Q8).cpu().numpy()
        assert_close_1e3(got, ref)


def test_attention_split_variants(be, orc):
    n_head, n_kv, hd, kv = 16, 4, 128, 1500
    rng = np.random.default_rng(17)
    k = rng.standard_normal((n_kv, kv, hd)).astype(np.float32)
    v = rng.standard_normal((n_kv, kv, hd)).astype(np.float32)
    c = A.KVCache(be, kv, 1, n_kv, hd)
    c.append(0, k, v, kv, hd, mem=B.MEM_HOST)
    q = rng.standard_normal((n_head, 2, hd)).astype(np.float32)
    ref = orc.attention(q, k, v, n_head, 2, kv, kv - 2)
    for wg in (1, 8, 64, 256, 4096):
        print("attention workgroup target", wg, flush=True)
        with env(BARQ_ATTN_WG=wg) as b:
            got = A.compute_attention(b, q, c, 0, n_head, n_kv, hd, 2, kv, kv - 2, mem=B.MEM_HOST)
        assert np.max(np.abs(got - ref)) <= 2e-5 * np.max(np.abs(v))
    c.close()
