"""The CPU oracle against the committed golden fixtures: the reference's own
known-answer tests (tests/golden/reference_kat.json) and the build's
regression fixtures and input hashes (tests/golden/make_golden.py)."""
import hashlib
import json
import os

import numpy as np
import pytest

from barq_rocm import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def kat():
    with open(os.path.join(GOLD, "reference_kat.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "blocks.npz"))


def test_kat_gemm_gemv(orc):
    k = kat()
    for c in k["gemm_f32"]:
        got = orc.gemm_f32(np.float32(c["a"]), np.float32(c["b"]), c["m"], c["k"], c["n"])
        assert np.array_equal(got.reshape(-1), np.float32(c["c"])), c["src"]
    for c in k["gemv_f32"]:
        got = orc.gemv_f32(np.float32(c["a"]), np.float32(c["x"]), c["m"], c["n"])
        assert np.array_equal(got, np.float32(c["y"])), c["src"]


def test_kat_split_decoders(orc):
    k = kat()
    c = k["dequantize_q4_0_split"][0]
    nb, bs = len(c["scales"]), c["block_size"]
    q = np.full(nb * bs // 2, c["quant_byte"], np.uint8)
    out = orc.dequantize_split(False, q, np.float32(c["scales"]), bs, nb * bs)
    assert np.array_equal(out, np.repeat(np.float32(c["expect_per_block"]), bs)), c["src"]
    c = k["dequantize_q4_0_split"][1]
    out = orc.dequantize_split(False, np.uint8(c["quants"]), np.float32(c["scales"]), c["block_size"], len(c["out"]))
    assert np.array_equal(out, np.float32(c["out"])), c["src"]
    c = k["quantized_matmul_split"][0]
    out = orc.quantized_matmul_split(np.float32(c["a"]), np.uint8(c["bq"]), np.float32(c["bs"]), c["m"], c["n"], c["k"],
                                     False, c["block_size"])
    assert out.size == c["out_len"], c["src"]
    # beyond the reference's length check: B decodes to all ones, so C = row sums of A
    assert np.array_equal(out, np.float32([[3, 3], [7, 7]]))


def test_kat_block_decoders(orc):
    k = kat()
    c = k["q8_0_block"][0]
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([c["d_f16"]], np.uint16).view(np.uint8)
    assert np.array_equal(orc.dequantize(orc.Q8_0, blk, 32), np.zeros(32, np.float32)), c["src"]
    c = k["k_quant_constant_block"][0]
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([c["d_f16"]], np.uint16).view(np.uint8)
    blk[2:4] = np.array([c["dmin_f16"]], np.uint16).view(np.uint8)
    blk[4:16] = 1
    blk[16:] = c["qs_byte"]
    assert np.array_equal(orc.dequantize(orc.Q4_K, blk, 256), np.ones(256, np.float32)), c["src"]
    c = k["q4_0_barq_roundtrip"][0]
    x = np.zeros(c["pad_to"], np.float32)
    x[:len(c["x"])] = c["x"]
    back = orc.dequantize(orc.Q4_0_BARQ, orc.q4_0_quantize_barq(x), x.size)
    assert np.max(np.abs(back - x)) < c["max_abs_err"], c["src"]


def test_kat_moe(orc):
    k = kat()
    c = k["moe_select_top_k"][0]
    ids, w = orc.moe_select_top_k(np.float32(c["logits"]).reshape(c["rows"], c["n_experts"]), c["top_k"])
    assert ids.tolist() == c["ids"], c["src"]
    assert np.all(np.abs(w.sum(1) - c["weight_row_sum"]) < c["tol"])
    c = k["moe_reduce_experts"][0]
    ids, w = orc.moe_reduce_experts(np.int32(c["ids"]), np.float32(c["weights"]), c["max_active"], c["min_weight"])
    kept = [[int(e) for e in row if e >= 0] for row in ids]
    assert kept == c["reduced_ids"], c["src"]
    assert np.all(np.abs(w.sum(1) - c["weight_row_sum"]) < c["tol"]), c["src"]
    c = k["moe_dispatch"][0]
    fns = [lambda a, s=s: a * s for s in c["expert_scale"]]
    out = orc.moe_dispatch(np.float32(c["input"]).reshape(c["rows"], c["hidden"]), len(fns), np.int32(c["ids"]),
                           np.float32(c["weights"]), fns)
    assert np.array_equal(out.reshape(-1), np.float32(c["out"])), c["src"]


def test_oracle_matches_committed_blocks(orc, gold):
    names = {"Q4_0": orc.Q4_0, "Q4_0_BARQ": orc.Q4_0_BARQ, "Q8_0": orc.Q8_0, "Q4_K": orc.Q4_K, "Q6_K": orc.Q6_K}
    for name, t in names.items():
        w = gold[f"{name}_blocks"]
        ref = gold[f"{name}_deq"]
        got = orc.dequantize(t, w, ref.size)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
    x = gold["act_x"]
    assert np.array_equal(orc.quantize_act(orc.Q8_0, x), gold["act_q8_0"])
    assert np.array_equal(orc.quantize_act(orc.Q8_K, x), gold["act_q8_k"])
    for name, t in names.items():
        w = gold[f"{name}_mv_w"]
        at = orc.Q8_K if t in (orc.Q4_K, orc.Q6_K) else orc.Q8_0
        y = orc.matvec(t, w, 8, 512, at, orc.quantize_act(at, x[0]))
        assert np.array_equal(y, gold[f"{name}_mv_y_q8"]), name
        assert np.array_equal(orc.matvec(t, w, 8, 512, orc.F32, x[0]), gold[f"{name}_mv_y_f32"]), name


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_synthetic_inputs_match_committed_hashes():
    with open(os.path.join(GOLD, "synth_sha256.json")) as f:
        h = json.load(f)
    for c in (1, 2, 3, 4):
        _, w, x = synth.linear_inputs(c)
        assert _sha(w) == h[f"C{c}_w"], c
        assert _sha(x) == h[f"C{c}_x"], c
    g, u, d, x, logits = synth.moe_inputs()
    assert hashlib.sha256(b"".join(_sha(a).encode() for a in g)).hexdigest() == h["C5_gate"]
    assert hashlib.sha256(b"".join(_sha(a).encode() for a in d)).hexdigest() == h["C5_down"]
    assert _sha(logits) == h["C5_logits"]
