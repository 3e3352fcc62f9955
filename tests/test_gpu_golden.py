"""libbarq_rocm (through the C ABI) against the committed golden fixtures:
bit-exact for decoders, activation blocks and the reference's f32 known
answers; 1e-3 for the small matvecs."""
import json
import os

import numpy as np
import pytest

import barq_rocm as B
from conftest import assert_bits_equal, assert_close_1e3

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = {"Q4_0": B.Q4_0, "Q4_0_BARQ": B.Q4_0_BARQ, "Q8_0": B.Q8_0, "Q4_K": B.Q4_K, "Q6_K": B.Q6_K}


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLD, "blocks.npz"))


def test_golden_dequantize(be, gold):
    for name, t in NAMES.items():
        ref = gold[f"{name}_deq"]
        print(f"golden dequantize {name}", flush=True)
        got = be.dequantize(t, dev(gold[f"{name}_blocks"]), ref.size).cpu().numpy()
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), fin), name
        assert_bits_equal(got[fin], ref[fin])


def test_golden_quantize_act(be, gold):
    x = gold["act_x"]
    assert np.array_equal(be.quantize_act(B.Q8_0, dev(x)).cpu().numpy(), gold["act_q8_0"])
    assert np.array_equal(be.quantize_act(B.Q8_K, dev(x)).cpu().numpy(), gold["act_q8_k"])


def test_golden_matvec(be, gold):
    x = gold["act_x"][0]
    for name, t in NAMES.items():
        at = B.Q8_PARTNER[t]
        w = dev(gold[f"{name}_mv_w"])
        xq = be.quantize_act(at, dev(x))
        y = be.matvec(t, w, 8, 512, at, xq).cpu().numpy()
        assert_close_1e3(y, gold[f"{name}_mv_y_q8"])
        y = be.matvec(t, w, 8, 512, B.ACT_F32, dev(x)).cpu().numpy()
        assert_close_1e3(y, gold[f"{name}_mv_y_f32"], tol=1e-5)


def test_golden_reference_kats(be):
    with open(os.path.join(GOLD, "reference_kat.json")) as f:
        k = json.load(f)
    for c in k["gemm_f32"]:
        got = be.gemm_f32(np.float32(c["a"]), np.float32(c["b"]), c["m"], c["k"], c["n"], mem=B.MEM_HOST)
        assert np.array_equal(got.reshape(-1), np.float32(c["c"])), c["src"]
    for c in k["gemv_f32"]:
        got = be.gemv_f32(np.float32(c["a"]), np.float32(c["x"]), c["m"], c["n"], mem=B.MEM_HOST)
        assert np.array_equal(got, np.float32(c["y"])), c["src"]
    c = k["dequantize_q4_0_split"][0]
    nb, bs = len(c["scales"]), c["block_size"]
    out = be.dequantize_split(B.Q4_K, np.full(nb * bs // 2, c["quant_byte"], np.uint8), np.float32(c["scales"]), bs,
                              nb * bs)
    assert np.array_equal(out, np.repeat(np.float32(c["expect_per_block"]), bs)), c["src"]
    c = k["moe_select_top_k"][0]
    ids, w = be.moe_route(np.float32(c["logits"]), c["rows"], c["n_experts"], c["top_k"], mem=B.MEM_HOST)
    assert ids.tolist() == c["ids"], c["src"]
    assert np.all(np.abs(w.sum(1) - c["weight_row_sum"]) < c["tol"])
