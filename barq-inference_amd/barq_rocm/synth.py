"""Deterministic synthetic inputs for the five benchmark configurations.

Generator: counter-based SplitMix64 (Steele, Lea & Flood 2014) seeded with
0xBA590000 + config, one sub-stream per field; normals by Box-Muller in f64;
f16 fields rounded to nearest-even from f64.  Block layouts are the GGUF /
llama.cpp ones the kernels and the reference decoders read
(barq_core/src/gguf.rs:521-914).
"""
from __future__ import annotations

import numpy as np

from . import _lib as L

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Words start..start+n-1 of the SplitMix64 stream of `seed`."""
    out = np.empty(n, dtype=np.uint64)
    s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        for c0 in range(0, n, _CHUNK):
            c1 = min(n, c0 + _CHUNK)
            idx = np.arange(start + c0 + 1, start + c1 + 1, dtype=np.uint64)
            out[c0:c1] = _mix(s + idx * _GOLDEN)
    return out


def sub_seed(base: int, field: int) -> int:
    with np.errstate(over="ignore"):
        return int(_mix(np.array([np.uint64(base) * np.uint64(0x100000001B3) + np.uint64(field)]))[0])


def uniform_bytes(seed: int, n: int) -> np.ndarray:
    w = splitmix64(seed, (n + 7) // 8)
    return w.view(np.uint8)[:n].copy()


def normals(seed: int, n: int) -> np.ndarray:
    """n standard normals (f64), Box-Muller on pairs of 53-bit uniforms."""
    m = (n + 1) // 2
    w = splitmix64(seed, 2 * m)
    u1 = (w[0::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log1p(-u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n]


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def gen_q4_0(n_rows: int, k: int, seed: int) -> np.ndarray:
    """GGUF Q4_0 (18 B / 32): d = f16(|N(0,0.02)|/8), 16 uniform bytes."""
    nb = n_rows * k // 32
    out = np.empty((nb, 18), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(normals(sub_seed(seed, 1), nb)) * 0.02 / 8.0)
    out[:, 2:] = uniform_bytes(sub_seed(seed, 2), nb * 16).reshape(nb, 16)
    return out.reshape(-1)


def gen_q4_0_barq(n_rows: int, k: int, seed: int) -> np.ndarray:
    """The reference's 20-byte Q4_0: f32 scale = |N(0,0.02)|/8, 16 uniform bytes."""
    nb = n_rows * k // 32
    out = np.empty((nb, 20), dtype=np.uint8)
    out[:, 0:4] = (np.abs(normals(sub_seed(seed, 1), nb)) * 0.02 / 8.0).astype(np.float32).view(np.uint8).reshape(nb, 4)
    out[:, 4:] = uniform_bytes(sub_seed(seed, 2), nb * 16).reshape(nb, 16)
    return out.reshape(-1)


def gen_q8_0(n_rows: int, k: int, seed: int) -> np.ndarray:
    """Q8_0 weights (34 B / 32): d = f16(|N(0,0.02)|/127), uniform i8 in [-127, 127]."""
    nb = n_rows * k // 32
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(normals(sub_seed(seed, 1), nb)) * 0.02 / 127.0)
    b = uniform_bytes(sub_seed(seed, 2), nb * 32).astype(np.int32)
    out[:, 2:] = ((b % 255) - 127).astype(np.int8).view(np.uint8).reshape(nb, 32)
    return out.reshape(-1)


def gen_q4_k(n_rows: int, k: int, seed: int) -> np.ndarray:
    """Q4_K (144 B / 256): d, dmin = f16(|N(0,0.01)|), 12 uniform scale bytes
    (uniform 6-bit scales and mins), 128 uniform nibble bytes."""
    nb = n_rows * k // 256
    out = np.empty((nb, 144), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(np.abs(normals(sub_seed(seed, 1), nb)) * 0.01)
    out[:, 2:4] = _f16_bytes(np.abs(normals(sub_seed(seed, 2), nb)) * 0.01)
    out[:, 4:16] = uniform_bytes(sub_seed(seed, 3), nb * 12).reshape(nb, 12)
    out[:, 16:] = uniform_bytes(sub_seed(seed, 4), nb * 128).reshape(nb, 128)
    return out.reshape(-1)


def gen_q6_k(n_rows: int, k: int, seed: int) -> np.ndarray:
    """Q6_K (210 B / 256): uniform ql/qh bit planes, i8 scales uniform in
    [-32, 31], d = f16(|N(0,0.01)|)."""
    nb = n_rows * k // 256
    out = np.empty((nb, 210), dtype=np.uint8)
    out[:, 0:192] = uniform_bytes(sub_seed(seed, 1), nb * 192).reshape(nb, 192)
    sc = (uniform_bytes(sub_seed(seed, 2), nb * 16).astype(np.int32) % 64) - 32
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8).reshape(nb, 16)
    out[:, 208:210] = _f16_bytes(np.abs(normals(sub_seed(seed, 3), nb)) * 0.01)
    return out.reshape(-1)


GENERATORS = {L.Q4_0: gen_q4_0, L.Q4_0_BARQ: gen_q4_0_barq, L.Q8_0: gen_q8_0, L.Q4_K: gen_q4_k, L.Q6_K: gen_q6_k}


def gen_weights(type_: int, n_rows: int, k: int, seed: int) -> np.ndarray:
    return GENERATORS[type_](n_rows, k, seed)


def gen_f32(n: int, seed: int, scale: float = 1.0) -> np.ndarray:
    return (normals(seed, n) * scale).astype(np.float32)


def config_seed(cfg: int) -> int:
    return 0xBA590000 + cfg


# (weight type, n_rows, k, batch)
CONFIGS = {
    1: dict(w_type=L.Q4_0, n_rows=4096, k=4096, m=1, name="C1 Q4_0 matvec 4096x4096, x->Q8_0"),
    2: dict(w_type=L.Q4_K, n_rows=14336, k=4096, m=1, name="C2 Q4_K matvec 14336x4096, x->Q8_K"),
    3: dict(w_type=L.Q6_K, n_rows=128256, k=4096, m=1, name="C3 Q6_K matvec 128256x4096, x->Q8_K"),
    4: dict(w_type=L.Q4_K, n_rows=4096, k=4096, m=512, name="C4 Q4_K GEMM 4096x4096, M=512, X->Q8_K"),
}
MOE_CONFIG = dict(n_experts=8, hidden=4096, n_ff=14336, tokens=64, top_k=2,
                  name="C5 MoE 8 experts, Q4_K gate/up 14336x4096, Q6_K down 4096x14336, 64 tokens top-2")


def linear_inputs(cfg: int, n_rows: int | None = None, k: int | None = None, m: int | None = None):
    """Weights and f32 activations of config 1-4 (optionally at reduced size)."""
    c = CONFIGS[cfg]
    n_rows = n_rows or c["n_rows"]
    k = k or c["k"]
    m = m or c["m"]
    s = config_seed(cfg)
    w = gen_weights(c["w_type"], n_rows, k, sub_seed(s, 10))
    x = gen_f32(m * k, sub_seed(s, 20)).reshape(m, k)
    return c["w_type"], w, x


def moe_inputs(n_experts=8, hidden=4096, n_ff=14336, tokens=64, top_k=2):
    s = config_seed(5)
    gates = [gen_q4_k(n_ff, hidden, sub_seed(s, 100 + e)) for e in range(n_experts)]
    ups = [gen_q4_k(n_ff, hidden, sub_seed(s, 200 + e)) for e in range(n_experts)]
    downs = [gen_q6_k(hidden, n_ff, sub_seed(s, 300 + e)) for e in range(n_experts)]
    x = gen_f32(tokens * hidden, sub_seed(s, 20)).reshape(tokens, hidden)
    logits = gen_f32(tokens * n_experts, sub_seed(s, 30)).reshape(tokens, n_experts)
    return gates, ups, downs, x, logits
