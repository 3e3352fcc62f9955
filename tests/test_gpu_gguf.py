"""Device weight cache (barq_rocm_cache_*): the packed tensors of a GGUF file
copied once to HBM and used directly by the kernels."""
import ctypes

import numpy as np
import pytest

import barq_rocm as B
import barq_rocm._lib as L
from barq_rocm import synth
from barq_rocm.gguf import GgufFile, WeightCache
import gguf_writer as W
from conftest import assert_close_1e3

pytestmark = pytest.mark.gpu


def test_cached_projections_match_host_calls(be, orc, tmp_path):
    p = str(tmp_path / "m.gguf")
    k = 4096
    ts = [
        ("blk.0.ffn_up.weight", [k, 96], 12, synth.gen_q4_k(96, k, 21)),
        ("blk.0.ffn_down.weight", [k, 80], 14, synth.gen_q6_k(80, k, 22)),
        ("blk.0.attn_q.weight", [k, 70], 2, synth.gen_weights(B.Q4_0, 70 * k // 32, 32, 23)),
        ("blk.0.attn_v.weight", [k, 33], 8, synth.gen_weights(B.Q8_0, 33 * k // 32, 32, 24)),
        ("output_norm.weight", [k], 0, synth.gen_f32(k, 25)),
    ]
    W.write(p, [("general.architecture", W.STRING, "llama")], [(n, d, t, np.asarray(r).tobytes()) for n, d, t, r in ts])
    x = synth.gen_f32(k, 26)
    with GgufFile(p) as g:
        cache = WeightCache(be, g)
        want_bytes = sum((len(np.asarray(r).tobytes()) + 255) // 256 * 256 for *_, r in ts)
        assert cache.nbytes() == want_bytes
        for name, dims, tid, raw in ts[:4]:
            t, n_rows, kk, ptr = cache.get(name)
            assert (t, n_rows, kk) == (tid, dims[1], dims[0]) and ptr % 256 == 0
            at = B.Q8_PARTNER[t]
            import torch
            xq = be.quantize_act(at, torch.from_numpy(x).cuda())
            y = torch.empty(n_rows, dtype=torch.float32, device="cuda")
            be.matvec_raw(t, ptr, n_rows, kk, at, xq, y, B.MEM_DEVICE)
            be.sync()
            # the same call on the file's bytes from host memory
            host = g.tensor(g.find(name))["data"]
            y_host = np.empty(n_rows, np.float32)
            be.matvec_raw(t, host, n_rows, kk, at, xq.cpu().numpy(), y_host, B.MEM_HOST)
            assert np.array_equal(y.cpu().numpy(), y_host)
            ref = orc.matvec(t, np.asarray(raw), n_rows, kk, at, xq.cpu().numpy())
            assert_close_1e3(y.cpu().numpy(), ref)
        # the f32 norm weight is cached as is
        t, n_rows, kk, ptr = cache.get("output_norm.weight")
        assert (t, n_rows, kk) == (0, 1, k)
        with pytest.raises(L.BarqError):
            cache.get("missing.weight")
        cache.close()
