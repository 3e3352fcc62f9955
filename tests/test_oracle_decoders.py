"""Pins the CPU oracle's block decoders (oracle/barq_oracle.c).

Each decoder is checked against the reference's own tests where they exist
and otherwise against closed forms, library routines and brute force chosen
so that a plausible slip (wrong nibble half, wrong index, unsigned instead of
signed, fused multiply-subtract) fails a test.
"""
import numpy as np
import pytest

from conftest import assert_bits_equal

F16_ONE = np.array([1.0], dtype=np.float16).view(np.uint8)


def f16b(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


# ---- f16 -> f32 (half 2.7.1 to_f32; gguf.rs:661,763,768,869) -------------

def test_f16_to_f32_all_patterns_match_numpy(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = orc.dequantize(orc.F16, bits.view(np.uint8), 65536)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_bits_equal(got[~nan], ref[~nan])
    # NaNs come back quiet
    assert np.all(got[nan].view(np.uint32) & 0x00400000)


def test_f32_to_f16_round_to_nearest_even_matches_numpy(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.float32([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                    2.9802326e-08, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf]),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---- Q8_0 (gguf.rs:634-681) ---------------------------------------------

def test_q8_0_zero_block_reference_test(orc):
    # gguf.rs:1288-1300: d = 1.0, qs = 0 -> all 0.0
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = F16_ONE
    assert np.all(orc.dequantize(orc.Q8_0, blk, 32) == 0.0)


def test_q8_0_every_byte_is_signed(orc):
    # d = 1: output is the byte reinterpreted as i8 (0x80 -> -128, 0xFF -> -1)
    blocks = np.zeros((8, 34), dtype=np.uint8)
    blocks[:, 0:2] = F16_ONE
    blocks[:, 2:] = np.arange(256, dtype=np.uint8).reshape(8, 32)
    got = orc.dequantize(orc.Q8_0, blocks.reshape(-1), 256)
    assert np.array_equal(got, np.arange(256, dtype=np.uint8).view(np.int8).astype(np.float32))


def test_q8_0_scale_applies_per_block(orc):
    blocks = np.zeros((3, 34), dtype=np.uint8)
    for i, d in enumerate([0.5, -2.0, 2.0 ** -24]):  # includes the smallest f16 subnormal
        blocks[i, 0:2] = f16b(d)
        blocks[i, 2:] = 3
    got = orc.dequantize(orc.Q8_0, blocks.reshape(-1), 96)
    assert np.all(got[:32] == 1.5) and np.all(got[32:64] == -6.0) and np.all(got[64:] == np.float32(3 * 2.0 ** -24))


# ---- Q4_0: the reference's 20-byte layout (gguf.rs:521-578) ---------------

def test_q4_0_barq_0x88_reference_test(orc):
    # quant/src/simd_quant.rs:323-353: nibble 8 -> -8 * scale, scales 1, 0.5, 2
    blocks = np.zeros((3, 20), dtype=np.uint8)
    for i, s in enumerate([1.0, 0.5, 2.0]):
        blocks[i, 0:4] = np.array([s], dtype=np.float32).view(np.uint8)
        blocks[i, 4:] = 0x88
    got = orc.dequantize(orc.Q4_0_BARQ, blocks.reshape(-1), 96)
    assert np.all(got[:32] == -8.0) and np.all(got[32:64] == -4.0) and np.all(got[64:] == -16.0)


def test_q4_0_barq_every_nibble_both_halves(orc):
    # byte i holds element 2i (low nibble) and 2i+1 (high), sign-extended
    blk = np.zeros(20, dtype=np.uint8)
    blk[0:4] = np.array([1.0], dtype=np.float32).view(np.uint8)
    for lo in range(16):
        hi = 15 - lo
        b = blk.copy()
        b[4 + 3] = (hi << 4) | lo
        got = orc.dequantize(orc.Q4_0_BARQ, b, 32)
        sext = lambda n: n - 16 if n >= 8 else n
        exp = np.zeros(32, dtype=np.float32)
        exp[6], exp[7] = sext(lo), sext(hi)
        assert np.array_equal(got, exp), (lo, hi)


def test_q4_0_barq_quantize_roundtrip_reference_test(orc):
    # quant/src/q4_0.rs:128-149: 1..8 then zeros, |error| < 1.5
    x = np.zeros(32, dtype=np.float32)
    x[:8] = np.arange(1, 9)
    q = orc.q4_0_quantize_barq(x)
    assert q.size == 20
    y = orc.dequantize(orc.Q4_0_BARQ, q, 32)
    assert np.all(np.abs(x - y) < 1.5)
    # scale = max_abs / 8 = 1.0 exactly; 8 saturates to 7
    assert q[:4].view(np.float32)[0] == 1.0
    assert y[7] == 7.0 and y[0] == 1.0


def test_q4_0_barq_quantize_rounding_and_zero_block(orc):
    # Rust f32::round is half away from zero: x/scale = 2.5 -> 3, -2.5 -> -3
    x = np.zeros(64, dtype=np.float32)
    x[0], x[1], x[2] = 8.0, 2.5, -2.5   # scale = 1
    q = orc.q4_0_quantize_barq(x)
    y = orc.dequantize(orc.Q4_0_BARQ, q, 64)
    assert y[1] == 3.0 and y[2] == -3.0 and y[0] == 7.0
    assert q[20:24].view(np.float32)[0] == 0.0 and np.all(y[32:] == 0.0)


# ---- Q4_0 GGUF layout through the byte adapter ----------------------------

def test_q4_0_gguf_adapter_every_nibble_every_position(orc):
    # llama.cpp dequantize_row_q4_0: y[j] = ((qs[j] & 15) - 8) d,
    # y[j+16] = ((qs[j] >> 4) - 8) d.  The adapter must give exactly this via
    # the reference's 20-byte decoder, for every (position, nibble).
    d = 0.375
    for pos in range(32):
        for nib in range(16):
            blk = np.zeros(18, dtype=np.uint8)
            blk[0:2] = f16b(d)
            blk[2:] = 0x88            # every other element decodes to 0
            j = pos % 16
            if pos < 16:
                blk[2 + j] = (blk[2 + j] & 0xF0) | nib
            else:
                blk[2 + j] = (blk[2 + j] & 0x0F) | (nib << 4)
            got = orc.dequantize(orc.Q4_0, blk, 32)
            exp = np.zeros(32, dtype=np.float32)
            exp[pos] = np.float32(nib - 8) * np.float32(d)
            assert np.array_equal(got, exp), (pos, nib)


def test_q4_0_gguf_adapter_bytes(orc):
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = f16b(1.0)
    blk[2:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    barq = orc.q4_0_gguf_to_barq(blk)
    assert barq.size == 20 and barq[:4].view(np.float32)[0] == 1.0
    # element 0 (gguf low nibble of byte 0 = 0) -> reference nibble 0^8 = 8 in the low half of byte 0
    assert barq[4] & 0x0F == 8


# ---- Q4_K (gguf.rs:730-837) ------------------------------------------------

def test_get_scale_min_k4_inverts_the_packing_exhaustively(orc):
    # quant/src/q5_k.rs:175-182 packs 8 (scale, min) 6-bit pairs into 12
    # bytes; gguf.rs:825-837 must return every pair, for every j and value.
    rng = np.random.default_rng(2)
    for j in range(8):
        for v in range(64):
            ls = rng.integers(0, 64, 8).astype(np.uint8)
            lm = rng.integers(0, 64, 8).astype(np.uint8)
            ls[j], lm[j] = v, 63 - v
            q = orc.pack_scale_min_k4(ls, lm)
            for jj in range(8):
                assert orc.get_scale_min_k4(jj, q) == (ls[jj], lm[jj])


def test_get_scale_min_k4_bit_level_spec(orc):
    # brute force over single set bits of the 12 bytes: each bit maps to
    # exactly one (j, field, bit) per the GGUF layout
    for byte in range(12):
        for bit in range(8):
            q = np.zeros(12, dtype=np.uint8)
            q[byte] = 1 << bit
            hits = []
            for j in range(8):
                sc, m = orc.get_scale_min_k4(j, q)
                if sc: hits.append(("sc", j, sc))
                if m: hits.append(("m", j, m))
            if byte < 4:
                exp = [("sc", byte, 1 << bit)] if bit < 6 else [("sc", byte + 4, 1 << (bit - 2))]
            elif byte < 8:
                exp = [("m", byte - 4, 1 << bit)] if bit < 6 else [("m", byte, 1 << (bit - 2))]
            else:
                j = byte - 4
                exp = [("sc", j, 1 << bit)] if bit < 4 else [("m", j, 1 << (bit - 4))]
            assert hits == exp, (byte, bit, hits)


def q4k_block(d, dmin, scales12, qs128):
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = f16b(d)
    b[2:4] = f16b(dmin)
    b[4:16] = scales12
    b[16:] = qs128
    return b


def test_q4_k_constant_block(orc):
    # the q5_k.rs:542-555 pattern: scale bytes all 1, nibbles 1, d = 1 -> 1.0
    b = q4k_block(1.0, 0.0, np.ones(12, np.uint8), np.full(128, 0x11, np.uint8))
    assert np.all(orc.dequantize(orc.Q4_K, b, 256) == 1.0)


def test_q4_k_mins_subtract(orc):
    ls = np.zeros(8, np.uint8)
    lm = np.arange(1, 9, dtype=np.uint8) * 7
    b = q4k_block(0.0, 1.0, orc.pack_scale_min_k4(ls, lm), np.zeros(128, np.uint8))
    got = orc.dequantize(orc.Q4_K, b, 256)
    assert np.array_equal(got, np.repeat(-lm.astype(np.float32), 32))


def test_q4_k_element_positions(orc):
    # llama.cpp dequantize_row_q4_K: qs[32c + l] low nibble -> element 64c + l,
    # high nibble -> 64c + 32 + l
    ls = np.arange(1, 9, dtype=np.uint8)
    b0 = q4k_block(1.0, 0.0, orc.pack_scale_min_k4(ls, np.zeros(8, np.uint8)), np.zeros(128, np.uint8))
    for c in range(4):
        for l in (0, 5, 31):
            for half in (0, 1):
                b = b0.copy()
                b[16 + 32 * c + l] = 3 << (4 * half)
                got = orc.dequantize(orc.Q4_K, b, 256)
                e = 64 * c + 32 * half + l
                nz = np.nonzero(got)[0]
                assert list(nz) == [e] and got[e] == 3.0 * ls[2 * c + half]


def test_q4_k_value_is_one_rounding_of_the_exact_value(orc):
    # d (f16, 11 significant bits) * sc (6 bits) and then * q (4 bits) are
    # exact in f32, so d1*q - m1 (gguf.rs:804) rounds once: the decoded value
    # is the exact d*sc*q - dmin*m rounded to f32, whether or not an
    # implementation fuses the multiply and the subtract.
    rng = np.random.default_rng(3)
    for _ in range(200):
        d = np.float16(rng.uniform(1e-4, 0.05))
        dmin = np.float16(rng.uniform(1e-4, 0.05))
        ls = rng.integers(0, 64, 8).astype(np.uint8)
        lm = rng.integers(0, 64, 8).astype(np.uint8)
        qs = rng.integers(0, 256, 128).astype(np.uint8)
        b = q4k_block(d, dmin, orc.pack_scale_min_k4(ls, lm), qs)
        got = orc.dequantize(orc.Q4_K, b, 256)
        for j in range(8):
            c, half = divmod(j, 2)
            q = ((qs[32 * c: 32 * c + 32] >> (4 * half)) & 15).astype(np.float64)
            exact = float(d) * int(ls[j]) * q - float(dmin) * int(lm[j])
            assert np.array_equal(got[32 * j: 32 * j + 32], exact.astype(np.float32))


# ---- Q6_K (gguf.rs:839-914) -------------------------------------------------

def q6k_block(d, ql, qh, sc):
    b = np.zeros(210, dtype=np.uint8)
    b[0:128] = ql
    b[128:192] = qh
    b[192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    b[208:210] = f16b(d)
    return b


def test_q6_k_extremes(orc):
    z = q6k_block(1.0, np.zeros(128, np.uint8), np.zeros(64, np.uint8), np.ones(16))
    assert np.all(orc.dequantize(orc.Q6_K, z, 256) == -32.0)
    f = q6k_block(1.0, np.full(128, 0xFF, np.uint8), np.full(64, 0xFF, np.uint8), np.ones(16))
    assert np.all(orc.dequantize(orc.Q6_K, f, 256) == 31.0)
    n = q6k_block(0.5, np.full(128, 0xFF, np.uint8), np.full(64, 0xFF, np.uint8), -np.ones(16) * 3)
    assert np.all(orc.dequantize(orc.Q6_K, n, 256) == -46.5)


def test_q6_k_element_positions(orc):
    # llama.cpp dequantize_row_q6_K: for half h, l < 32:
    #   y[128h+l]    = ql[64h+l] low  | qh[32h+l] bits 0-1, scale sc[8h + l/16]
    #   y[128h+l+32] = ql[64h+l+32] low | bits 2-3, sc + 2
    #   y[128h+l+64] = ql[64h+l] high | bits 4-5, sc + 4
    #   y[128h+l+96] = ql[64h+l+32] high | bits 6-7, sc + 6
    sc = np.arange(1, 17)
    base_ql = np.full(128, 0x00, np.uint8)
    base_qh = np.full(64, 0xAA, np.uint8)   # high bits 2 everywhere -> q = 32 -> value 0
    for h in (0, 1):
        for l in (0, 17, 31):
            for qd in range(4):
                ql, qh = base_ql.copy(), base_qh.copy()
                idx = 64 * h + l + (32 if qd in (1, 3) else 0)
                ql[idx] = 5 << (4 if qd >= 2 else 0)
                got = orc.dequantize(orc.Q6_K, q6k_block(1.0, ql, qh, sc), 256)
                e = 128 * h + l + 32 * qd
                nz = np.nonzero(got)[0]
                assert list(nz) == [e], (h, l, qd, nz)
                assert got[e] == 5.0 * sc[8 * h + l // 16 + 2 * qd]
            # the two qh bits of one lane position
            for qd in range(4):
                ql, qh = base_ql.copy(), base_qh.copy()
                qh[32 * h + l] = (0xAA & ~(3 << (2 * qd))) | (3 << (2 * qd)) & 0xFF
                got = orc.dequantize(orc.Q6_K, q6k_block(1.0, ql, qh, sc), 256)
                e = 128 * h + l + 32 * qd
                assert list(np.nonzero(got)[0]) == [e]
                assert got[e] == 16.0 * sc[8 * h + l // 16 + 2 * qd]


def test_dequantize_truncates_to_total_elements(orc):
    # load_* truncate to total_elements (gguf.rs:576,679,821,912)
    b = q4k_block(1.0, 0.0, np.ones(12, np.uint8), np.full(128, 0x11, np.uint8))
    assert orc.dequantize(orc.Q4_K, b, 100).size == 100


def test_block_geometry(orc):
    # gguf.rs:168-186 block sizes and the per-type byte counts
    for t, e, nb in [(orc.Q4_0, 32, 18), (orc.Q4_0_BARQ, 32, 20), (orc.Q8_0, 32, 34), (orc.Q4_K, 256, 144),
                     (orc.Q6_K, 256, 210), (orc.Q8_K, 256, 292)]:
        assert orc.block_elems(t) == e and orc.block_bytes(t) == nb


# ---- the quant crate's own Q4_K (quant/src/q4_k.rs; not the GGUF format) --------------
def test_q4_k_barq_reference_roundtrip(orc):
    # quant/src/q4_k.rs:166-180: 0..256 round trip keeps the length, no NaN
    x = np.arange(256, dtype=np.float32)
    q = orc.q4_k_barq_quantize(x)
    assert q.size == 136
    y = orc.q4_k_barq_dequantize(q, 256)
    assert y.size == 256 and not np.isnan(y).any()
    # and for 0..255 every value is within half a step (255/15/2) of its input
    assert np.max(np.abs(y - x)) <= 255.0 / 30.0 + 1e-4


def test_q4_k_barq_layout_and_closed_forms(orc):
    x = np.array([3.0, -1.0, 7.0, 1.0] * 64, dtype=np.float32)
    q = orc.q4_k_barq_quantize(x)
    smin, srange = np.frombuffer(q[:8].tobytes(), dtype=np.float32)
    assert smin == -1.0 and srange == 8.0
    # (x - min) / range * 15: 3 -> 7.5 -> 8 (half away from zero), -1 -> 0, 7 -> 15, 1 -> 3.75 -> 4
    assert q[8] == (8 | (0 << 4)) and q[9] == (15 | (4 << 4))
    y = orc.q4_k_barq_dequantize(q, 256)
    assert y[1] == -1.0 and y[2] == np.float32(-1.0) + np.float32(np.float32(15) / np.float32(15)) * np.float32(8.0)
    # a constant block: range 0, every q = round(7.5) = 8, decodes to the constant
    c = orc.q4_k_barq_quantize(np.full(256, 2.5, dtype=np.float32))
    assert np.all(c[8:] == 0x88) and np.all(orc.q4_k_barq_dequantize(c, 256) == 2.5)


def test_q4_k_barq_partial_block_and_truncation(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256 + 37).astype(np.float32)
    q = orc.q4_k_barq_quantize(x)
    assert q.size == 136 + 8 + 19          # the last block: 8 + ceil(37 / 2) bytes, odd length -> high nibble 0
    assert q[-1] >> 4 == 0
    # the reference's dequantize reads whole 136-byte blocks only: the short block is dropped
    y = orc.q4_k_barq_dequantize(q, x.size)
    assert y.size == 256
    step = (x[:256].max() - x[:256].min()) / 15.0
    assert np.max(np.abs(y - x[:256])) <= step / 2 * (1 + 1e-5)
    # a decoder that read the short block's nibbles anyway would return 293 values
    assert orc.q4_k_barq_dequantize(q, x.size + 1000).size == 256
