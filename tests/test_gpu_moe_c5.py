"""Config C5 at its BASELINE shape (Mixtral-8x7B experts: 8 experts, Q4_K
gate/up 14336 x 4096, Q6_K down 4096 x 14336, 64 tokens routed top-2 by
softmax over seeded N(0,1) logits): the whole 64-token step runs on the
device, and a spread of tokens, covering the most- and the least-loaded
expert, is checked against the oracle's dispatch_experts
(moe_fused.rs:226-308) at the 1e-3 bar, on the integer path and on the f32
path.  The oracle runs only on the chosen tokens (each token's output
depends on its own row alone: activations are quantized per row)."""
import numpy as np
import pytest

import barq_rocm as B
from barq_rocm import synth
from conftest import assert_close_1e3

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def c5():
    c = synth.MOE_CONFIG
    print("C5: generating the Mixtral-shape experts", flush=True)
    gates, ups, downs, x, logits = synth.moe_inputs()
    return c, gates, ups, downs, x, logits


def pick_tokens(ids, n_experts, n_pick):
    """Tokens routed to the most-loaded and the least-loaded expert first,
    then spread over the rest."""
    counts = np.bincount(ids.ravel(), minlength=n_experts)
    most, least = int(np.argmax(counts)), int(np.argmin(np.where(counts > 0, counts, 1 << 30)))
    chosen = []
    for e in (most, least):
        for t in np.nonzero((ids == e).any(axis=1))[0][:2]:
            if int(t) not in chosen:
                chosen.append(int(t))
    for t in np.linspace(0, ids.shape[0] - 1, n_pick).astype(int):
        if len(chosen) >= n_pick:
            break
        if int(t) not in chosen:
            chosen.append(int(t))
    return sorted(chosen), counts, most, least


def test_moe_c5_integer_path(be, orc, c5):
    import torch
    c, gates, ups, downs, x, logits = c5
    ne, hid, nff, T, k = c["n_experts"], c["hidden"], c["n_ff"], c["tokens"], c["top_k"]
    ids_d, w_d = be.moe_route(dev(logits), T, ne, k)
    ids, w = ids_d.cpu().numpy(), w_d.cpu().numpy()
    rid, rw = orc.moe_select_top_k(logits, k)
    assert np.array_equal(ids, rid)
    gd, ud, dd = [dev(a) for a in gates], [dev(a) for a in ups], [dev(a) for a in downs]
    print("C5: 64-token step on the device", flush=True)
    out = be.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hid, nff, dev(x), T, ids_d, w_d, k, B.ACT_F32_Q8)
    out = out.cpu().numpy()
    assert np.all(np.isfinite(out))
    sel, counts, most, least = pick_tokens(ids, ne, 8)
    print(f"C5: expert loads {counts.tolist()}, checking tokens {sel} (most {most}, least {least})", flush=True)
    assert counts.max() > counts.min()          # the routing is uneven, as the config says
    ref = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x[sel], ids[sel], w[sel], orc.Q8_K)
    assert_close_1e3(out[sel], ref)
    # the same tokens as a step of their own give the same rows bit for bit
    out_sub = be.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hid, nff, dev(x[sel]), len(sel), dev(ids[sel]),
                         dev(w[sel]), k, B.ACT_F32_Q8).cpu().numpy()
    assert np.array_equal(out_sub, out[sel])
    del gd, ud, dd
    torch.cuda.empty_cache()


def test_moe_c5_f32_path(be, orc, c5):
    import torch
    c, gates, ups, downs, x, logits = c5
    ne, hid, nff, T, k = c["n_experts"], c["hidden"], c["n_ff"], c["tokens"], c["top_k"]
    ids, w = orc.moe_select_top_k(logits, k)
    sel = [0, T - 1]
    gd, ud, dd = [dev(a) for a in gates], [dev(a) for a in ups], [dev(a) for a in downs]
    print(f"C5: f32-activation step on tokens {sel}", flush=True)
    out = be.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hid, nff, dev(x[sel]), len(sel), dev(ids[sel]),
                     dev(w[sel]), k, B.ACT_F32).cpu().numpy()
    ref = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hid, nff, x[sel], ids[sel], w[sel], orc.F32)
    assert_close_1e3(out, ref)
    del gd, ud, dd
    torch.cuda.empty_cache()
