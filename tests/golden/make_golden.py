"""Writes the build's own golden fixtures (run from the repo root:
``python tests/golden/make_golden.py``).

blocks.npz   small seeded and edge-case blocks of every weight type with their
             dequantized f32 values, Q8_0/Q8_K activation blocks of fixed
             vectors, and small matvec outputs, all computed by the CPU
             oracle (oracle/barq_oracle.c) — regression fixtures for the
             oracle and fixed data the GPU tests check against.
synth_sha256.json  SHA-256 of every full-size BASELINE config buffer the
             SplitMix64 generators produce, so a box that regenerates them is
             known to time and check exactly the same inputs.
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "barq-inference_amd"))
HERE = os.path.dirname(os.path.abspath(__file__))

from barq_rocm import synth  # noqa: E402
from oracle import oracle as orc  # noqa: E402

TYPES = {"Q4_0": orc.Q4_0, "Q4_0_BARQ": orc.Q4_0_BARQ, "Q8_0": orc.Q8_0, "Q4_K": orc.Q4_K, "Q6_K": orc.Q6_K}
BYTES = {orc.Q4_0: 18, orc.Q4_0_BARQ: 20, orc.Q8_0: 34, orc.Q4_K: 144, orc.Q6_K: 210}
ELEMS = {orc.Q4_0: 32, orc.Q4_0_BARQ: 32, orc.Q8_0: 32, orc.Q4_K: 256, orc.Q6_K: 256}


def edge_blocks(t, nb, seed):
    """Seeded blocks with f16/f32 scale extremes and all-0x00 / all-0xFF payloads."""
    bb = BYTES[t]
    w = synth.gen_weights(t, nb, ELEMS[t], seed).reshape(nb, bb).copy()
    f16s = np.float16([0.0, 2.0 ** -24, 6.1e-5, 65504.0, -1.5, 1.0]).view(np.uint8).reshape(-1, 2)
    for i in range(nb):
        if i % 4 == 0:
            if t == orc.Q6_K:
                w[i, 208:210] = f16s[i % 6]
            elif t == orc.Q4_0_BARQ:
                w[i, 0:4] = np.float32([0.0, 1e-40, 3.0e38, -2.0, 1.0, 0.125])[i % 6:i % 6 + 1].view(np.uint8)
            else:
                w[i, 0:2] = f16s[i % 6]
                if t == orc.Q4_K:
                    w[i, 2:4] = f16s[(i + 1) % 6]
        if i % 3 == 1:
            lo = {orc.Q4_0: 2, orc.Q8_0: 2, orc.Q4_0_BARQ: 4, orc.Q4_K: 4, orc.Q6_K: 0}[t]
            hi = 208 if t == orc.Q6_K else bb
            w[i, lo:hi] = 0xFF if i % 2 else 0x00
    return w.reshape(-1)


def blocks():
    out = {}
    for name, t in TYPES.items():
        nb = 24
        w = edge_blocks(t, nb, 4242 + t)
        out[f"{name}_blocks"] = w
        out[f"{name}_deq"] = orc.dequantize(t, w, nb * ELEMS[t])
    x = synth.gen_f32(4 * 512, 77).reshape(4, 512)
    x[1, :256] = 0.0                      # an all-zero Q8_K block and Q8_0 blocks
    x[2, 0] = 300.0                       # one large element per block
    x[2, 300] = -250.0
    x[3] = np.round(x[3] * 4) / 4         # many exact ties
    out["act_x"] = x
    out["act_q8_0"] = orc.quantize_act(orc.Q8_0, x)
    out["act_q8_k"] = orc.quantize_act(orc.Q8_K, x)
    # small matvecs (n=8 rows, k=512) on Q8 and f32 activations
    for name, t in TYPES.items():
        k = 512
        w = synth.gen_weights(t, 8, k, 99 + t)
        at = orc.Q8_K if ELEMS[t] == 256 else orc.Q8_0
        xq = orc.quantize_act(at, x[0])
        out[f"{name}_mv_w"] = w
        out[f"{name}_mv_y_q8"] = orc.matvec(t, w, 8, k, at, xq)
        out[f"{name}_mv_y_f32"] = orc.matvec(t, w, 8, k, orc.F32, x[0])
    np.savez_compressed(os.path.join(HERE, "blocks.npz"), **out)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def synth_hashes():
    h = {}
    for c in (1, 2, 3, 4):
        _, w, x = synth.linear_inputs(c)
        h[f"C{c}_w"] = sha(w)
        h[f"C{c}_x"] = sha(x)
    g, u, d, x, logits = synth.moe_inputs()
    h["C5_gate"] = hashlib.sha256(b"".join(sha(a).encode() for a in g)).hexdigest()
    h["C5_up"] = hashlib.sha256(b"".join(sha(a).encode() for a in u)).hexdigest()
    h["C5_down"] = hashlib.sha256(b"".join(sha(a).encode() for a in d)).hexdigest()
    h["C5_x"] = sha(x)
    h["C5_logits"] = sha(logits)
    with open(os.path.join(HERE, "synth_sha256.json"), "w") as f:
        json.dump(h, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    orc.lib()
    blocks()
    synth_hashes()
    print("wrote", os.listdir(HERE))
