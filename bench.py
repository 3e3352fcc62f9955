#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Headline (BASELINE.json metric): Q4_K x Q8_K batch-1 GEMV at the Llama-3-8B
FFN up/gate shape (config 2: 14336 x 4096), achieved HBM GB/s against the
8 TB/s peak and us/call.  A step is one GEMV call.  Weights rotate over
enough distinct copies (>= 1 GiB) that the 256 MB Infinity Cache cannot
hold them, activations are quantized once beforehand (their kernel is timed
on its own line) and all inputs are resident in HBM before timing starts.

The K timed launches are captured into a HIP graph and replayed five
times, so the per-launch time measured with HIP events on the launch stream
(the median of the five replays) is the kernel's own duration rather than
host launch overhead; the eager back-to-back rate is reported beside it.

The CPU baseline times the reference's per-call CPU arithmetic (an f32
GEMV over weights dequantized at load, barq_core/src/blas.rs) as restated in
oracle/, on a bounded sample of the same workload.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "barq-inference_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
F32_MFMA_PEAK_TFLOPS = 157.3   # dense f32 matrix peak
METRIC = "Q4_K GEMV achieved HBM GB/s (% of peak) + µs/call at Llama-3-8B shapes, 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    # untimed launches before the timed ones: enough (< 1 s) for the GPU's clocks to settle
    p.add_argument("--warmup", type=int, default=2000)
    p.add_argument("--config", type=int, default=2, help="BASELINE.json config: 1-4 linear, 5 MoE")
    p.add_argument("--w-type", default=None, choices=["Q4_0", "Q8_0", "Q4_0_BARQ", "Q4_K", "Q6_K"],
                   help="configs 1-4: another weight format at the same shape (e.g. --config 4 --w-type Q4_0)")
    p.add_argument("--copies", type=int, default=0, help="distinct weight copies (default: >= 1 GiB of them)")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline sample budget")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of a graph")
    p.add_argument("--no-traffic", action="store_true",
                   help="skip the two rocprofv3 --pmc child runs that measure HBM traffic per launch")
    p.add_argument("--norm", action="store_true",
                   help="time the fused RMSNorm -> Q8_K quantizer (the step before each projection) instead of a config")
    p.add_argument("--attn", action="store_true",
                   help="time decode attention over the device KV cache (Llama-3-8B heads) instead of a config")
    p.add_argument("--kv-len", type=int, default=4096, help="--attn: cached positions per query")
    p.add_argument("--q-len", type=int, default=1, help="--attn: new tokens per call (1 = decode; > 1 = a prompt chunk)")
    p.add_argument("--ffn", action="store_true",
                   help="time the dense FFN (feed_forward: gate/up Q4_K, SwiGLU, down Q6_K) at Llama-3-8B shapes")
    p.add_argument("--m", type=int, default=1,
                   help="--ffn: tokens per call; --prefill: prompt tokens (default 512); "
                        "configs 1-3: 2-4 activation rows on the same weights (a small decode batch)")
    p.add_argument("--decode", action="store_true",
                   help="a whole Llama-3-8B decode token (32 layers, output norm, LM head) over --kv-len cached positions")
    p.add_argument("--prefill", action="store_true",
                   help="one Llama-3-8B layer over a --m token prompt (GEMMs, MFMA attention): tokens/s")
    p.add_argument("--layer", action="store_true",
                   help="time one Llama-3-8B decode layer (norm, q/k/v, RoPE + KV append, attention, o, norm, FFN)")
    p.add_argument("--no-fixed", action="store_true",
                   help="one-token configs: skip timing the per-launch floor and the GEMV over twice the rows "
                        "(kernel traces and counter runs then hold only the measured launches)")
    p.add_argument("--probe-copy", action="store_true",
                   help="also run 5 device copies of 256 MiB (reference for rocprofv3 FETCH_SIZE/WRITE_SIZE scaling)")
    return p.parse_args()


def algorithmic_bytes(w_type, n, k, m):
    import barq_rocm as B
    at = B.Q8_PARTNER[w_type]
    return n * B.row_bytes(w_type, k) + m * B.row_bytes(at, k) + m * n * 4


def time_launches(launch, K, eager):
    """Average per-launch ms over K launches on the backend stream."""
    import torch
    s = torch.cuda.current_stream()
    if not eager:
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for i in range(K):
                    launch(i)
            # untimed replays first: the first replays of a graph of long
            # kernels ran slower in kernel traces (the MoE step: 263, 255, then
            # 229-236 us a step) than the later ones
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            # the median of five timed replays (a single replay varies by a few %)
            times = []
            for _ in range(5):
                t0 = torch.cuda.Event(enable_timing=True)
                t1 = torch.cuda.Event(enable_timing=True)
                t0.record(s)
                g.replay()
                t1.record(s)
                t1.synchronize()
                times.append(t0.elapsed_time(t1) / K)
            return sorted(times)[2], "hip-graph replay (median of 5)"
        except Exception as e:  # graph capture unavailable: eager launches
            log(f"graph capture failed ({e}); timing eager launches")
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(s)
    for i in range(K):
        launch(i)
    t1.record(s)
    t1.synchronize()
    return t0.elapsed_time(t1) / K, "eager"


# Timed calls rotate over distinct copies of their weights (and KV caches)
# totalling at least this many bytes.  The 256 MB Infinity Cache must not
# serve them: with 363 MB of C2 copies the GEMV measured ~1.7 % faster than
# with 1-2 GB, and a decode layer ~4.5 % faster with 2 copies than with 6.
ROTATE_BYTES = 1 << 30

# dominant kernel of each config (config 5: every kernel of the MoE step)
# (GEMVs with k <= 4096 run the LDS-staged two-row kernels unless
# BARQ_GEMV_LDS=0)
_LDS_OFF = os.environ.get("BARQ_GEMV_LDS") == "0"
Q4K_GEMV = "gemv_q8_kernel<barq::FmtQ4K" if _LDS_OFF else "gemv_q4k_lds_kernel"
Q40_GEMV = "gemv_dma_kernel<barq::DQ40," if _LDS_OFF else "gemv_pair32_kernel<barq::DQ40,"
Q6K_GEMV = "gemv_dma_kernel<barq::DQ6K" if _LDS_OFF else "gemv_q6k_pair_kernel"
KERNEL_OF_CONFIG = {1: Q40_GEMV, 2: Q4K_GEMV,
                    3: Q6K_GEMV, 4: "kq_kernel<barq::KQ4, 64", 5: "barq::"}
# with --w-type: (GEMV, GEMM) kernel of each format
KERNEL_OF_TYPE = {"Q4_0": (Q40_GEMV, "b32_gemm_kernel<barq::B40,"),
                  "Q8_0": ("gemv_dma_kernel<barq::DQ80" if _LDS_OFF else "gemv_pair32_kernel<barq::DQ80",
                           "b32_gemm_kernel<barq::B80,"),
                  "Q4_0_BARQ": ("gemv_dma_kernel<barq::DQ40B" if _LDS_OFF else "gemv_pair32_kernel<barq::DQ40B",
                                "b32_gemm_kernel<barq::B40Barq"),
                  "Q4_K": (Q4K_GEMV, "kq_kernel<barq::KQ4, 64"),
                  "Q6_K": (Q6K_GEMV, "kq_kernel<barq::KQ6")}


def measure_traffic(config, w_type_name=None):
    """HBM bytes per launch of the config's dominant kernel: two rocprofv3
    child runs of this script (FETCH_SIZE, then WRITE_SIZE, in KiB per
    dispatch), each scaled by what the same counter reads for a 256 MiB
    device copy (--probe-copy).  Returns (bytes, detail) or (None, reason)."""
    import csv
    import shutil
    import statistics as st
    import subprocess
    import tempfile

    if not shutil.which("rocprofv3"):
        return None, "rocprofv3 not found"
    name = KERNEL_OF_CONFIG[config]
    extra = []
    if w_type_name:
        name = KERNEL_OF_TYPE[w_type_name][1 if config == 4 else 0]
        extra = ["--w-type", w_type_name]
    vals = {}
    tmp = tempfile.mkdtemp(prefix="barq_pmc_")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = os.path.join(tmp, counter)
        cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "t", "--",
               sys.executable, os.path.abspath(__file__), "--config", str(config), "--steps", "10", "--warmup", "2",
               "--no-cpu", "--no-traffic", "--no-fixed", "--probe-copy"] + extra
        try:
            r = subprocess.run(cmd, cwd=tmp, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, timeout=180)
        except subprocess.TimeoutExpired:
            return None, f"{counter} run timed out"
        files = [os.path.join(dp, f) for dp, _, fs in os.walk(out) for f in fs if f.endswith("counter_collection.csv")]
        if r.returncode != 0 and not files:
            return None, f"{counter} run failed: {r.stderr.decode(errors='replace')[-300:]}"
        rows = [row for f in files for row in csv.DictReader(open(f))]
        copies = [float(row["Counter_Value"]) for row in rows if "copyBuffer" in row["Kernel_Name"]][-5:]
        if config == 5:
            # per step: the median of every kernel of the step, summed
            by = {}
            for row in rows:
                kn = row["Kernel_Name"]
                if name in kn and "moe_route" not in kn:
                    by.setdefault(kn.split("(")[0], []).append(float(row["Counter_Value"]))
            kern = [sum(st.median(v) for v in by.values())] if by else []
        else:
            kern = [float(row["Counter_Value"]) for row in rows if name in row["Kernel_Name"]]
        if not kern or len(copies) < 5:
            return None, f"{counter}: kernel or copy-probe dispatches missing"
        vals[counter] = (st.median(kern), 262144.0 / st.median(copies))
    shutil.rmtree(tmp, ignore_errors=True)
    fk, fs = vals["FETCH_SIZE"]
    wk, wsc = vals["WRITE_SIZE"]
    traffic = (fk * fs + wk * wsc) * 1024.0
    return traffic, dict(fetch_kib=round(fk, 1), fetch_scale=round(fs, 4), write_kib=round(wk, 1),
                         write_scale=round(wsc, 4))


def host_cpu():
    """CPU model as /proc/cpuinfo names it, with family/model/stepping (a
    virtualised host may report only the vendor's brand)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if info:
                        break
                    continue
                key, val = (p.strip() for p in line.split(":", 1))
                info.setdefault(key, val)
    except OSError:
        pass
    name = info.get("model name") or platform.processor() or "unknown CPU"
    fam = [f"{k_} {info[k_]}" for k_ in ("cpu family", "model", "stepping") if k_ in info]
    sockets = "?"
    try:
        with open("/proc/cpuinfo") as f:
            sockets = str(len({ln.split(":", 1)[1].strip() for ln in f if ln.startswith("physical id")}) or "?")
    except OSError:
        pass
    return f"{name} ({', '.join(fam)}; {sockets} socket(s))"


def cpu_baseline(w_type, w, x, n, k, budget_s, alg_bytes):
    """The reference's per-call CPU path on a bounded sample (oracle restatement)."""
    import numpy as np
    from oracle import oracle as orc

    wf = orc.dequantize(w_type, w, n * k)                  # load-time dequant (not timed)
    out = {}
    nproc = os.cpu_count() or 1
    # variant (iii) runs on every host core this process may be scheduled on
    # (nproc unless an affinity mask narrows it)
    threads = max(1, len(os.sched_getaffinity(0)))
    # (i) literal: gemm_f32(x[1 x k], W^T[k x n]) column by column (blas.rs:199-210)
    w_t = np.ascontiguousarray(wf.reshape(n, k).T)          # weight_cache.rs:196-201
    y = np.zeros(n, np.float32)
    # whole passes over the output columns, repeated until the budget is spent
    done, t_used = 0, 0.0
    chunk = 256
    while t_used < budget_s * 0.5:
        j = done % n
        j1 = min(n, j + chunk)
        t0 = time.perf_counter()
        orc.cpub_gemm_literal_m1(x, w_t, k, n, j, j1, y)
        t_used += time.perf_counter() - t0
        done += j1 - j
    lit_s = t_used * n / done
    out["literal_1core"] = dict(us_per_call=lit_s * 1e6, cols_sampled=done, sample_s=round(t_used, 3))
    del w_t
    # (ii) reference SIMD dot per row (simd.rs:115-138), one thread
    a = wf
    done, t_used = 0, 0.0
    while t_used < budget_s * 0.25:
        r = done % n
        r1 = min(n, r + 512)
        t0 = time.perf_counter()
        orc.cpub_gemv_simd(a, x, k, r, r1, y)
        t_used += time.perf_counter() - t0
        done += r1 - r
    simd_s = t_used * n / done
    out["simd_1core"] = dict(us_per_call=simd_s * 1e6, rows_sampled=done, sample_s=round(t_used, 3))
    # (iii) the same dot over all host threads, full calls
    reps, t_used = 0, 0.0
    while t_used < budget_s * 0.25:
        t0 = time.perf_counter()
        used = orc.cpub_gemv_simd_threaded(a, x, k, 0, n, y, threads)
        t_used += time.perf_counter() - t0
        reps += 1
    thr_s = t_used / reps
    out["simd_threads"] = dict(us_per_call=thr_s * 1e6, threads=used, calls=reps, sample_s=round(t_used, 3))
    simd = {2: "avx512", 1: "avx2", 0: "scalar"}[orc.cpub_simd_level()]
    cpu_model = host_cpu()
    for v in out.values():
        v["gbs_alg"] = alg_bytes / (v["us_per_call"] * 1e-6) / 1e9
    return {
        "value": round(out["literal_1core"]["gbs_alg"], 4),
        "unit": "GB/s (algorithmic Q4_K call bytes / CPU time)",
        "cores": 1,
        "kind": "port",
        "sample": (f"reference per-call path (blas.rs:199-210 gemm_f32 at M=1 over f32 W^T dequantized at load, "
                   f"not timed), {out['literal_1core']['cols_sampled']} output columns timed "
                   f"({out['literal_1core']['cols_sampled'] / n:.1f} calls' worth) in "
                   f"{out['literal_1core']['sample_s']} s; {cpu_model}, {simd}; nproc {nproc}, "
                   f"variant (iii) on {out['simd_threads']['threads']} threads"),
        "host_cpu": cpu_model,
        "nproc": nproc,
        "us_per_call": round(out["literal_1core"]["us_per_call"], 1),
        "variants": {k_: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                     for k_, v in out.items()},
    }


def cpu_baseline_gemm(w_type, w, x, n, k, m, budget_s):
    """C4: the reference's per-call CPU path at M = m, blas::gemm_f32
    (blas.rs:193-212) over f32 W^T dequantized and transposed at load (not
    timed): output rows split over every host core (rayon par_chunks_mut),
    each element a sequential sum over the column-strided W^T.  A bounded
    sample of rows (each thread one row per round) is timed and scaled to the
    m-row call."""
    import numpy as np
    from oracle import oracle as orc

    wf = orc.dequantize(w_type, w, n * k)
    w_t = np.ascontiguousarray(wf.reshape(n, k).T)
    del wf
    threads = max(1, len(os.sched_getaffinity(0)))
    c = np.empty((threads, n), np.float32)
    rows, t_used, used = 0, 0.0, 0
    while t_used < budget_s and rows < m:
        i0 = rows % m
        xs = np.ascontiguousarray(x[i0:i0 + threads], dtype=np.float32)
        t0 = time.perf_counter()
        used = orc.cpub_gemm_rows_threaded(xs, w_t, k, n, 0, xs.shape[0], c, threads)
        t_used += time.perf_counter() - t0
        rows += xs.shape[0]
    per_call = t_used * m / rows
    ops = 2.0 * m * n * k
    cpu_model = host_cpu()
    return {
        "value": round(ops / per_call / 1e12, 6), "unit": "TOP/s (2 M N K / CPU time)", "cores": used,
        "kind": "port",
        "sample": (f"reference per-call path (blas.rs:193-212 gemm_f32 at M={m} over f32 W^T dequantized at load, "
                   f"not timed), rows over {used} threads; {rows} of {m} rows timed in {t_used:.2f} s and scaled "
                   f"to the call; {cpu_model}; nproc {os.cpu_count()}"),
        "host_cpu": cpu_model, "nproc": os.cpu_count(), "us_per_call": round(per_call * 1e6, 1),
    }


def cpu_baseline_moe(gates, ups, downs, x, ids, hidden, n_ff, budget_s, alg_bytes):
    """C5: the reference's MoE step on the CPU, MoEFusedOps::dispatch_experts
    (moe_fused.rs:226-308): for each expert its batch of token rows through
    fused_ffn (:84-92) = ops::MatMul (ops.rs:68-128, one thread) with G and U,
    ops::Silu times x U, MatMul with D, over f32 weights transposed at load
    (not timed), then the weighted scatter.  Every assignment costs the same
    three products, so a bounded sample of rows of one expert is timed and
    scaled to the step's assignments (the scatter and routing are <0.01 %)."""
    import numpy as np

    import barq_rocm as B
    from oracle import oracle as orc

    ids = np.asarray(ids)
    n_assign = int((ids >= 0).sum())
    e0 = int(ids.reshape(-1)[0])
    toks = [t for t in range(ids.shape[0]) if e0 in ids[t].tolist()]
    gt = np.ascontiguousarray(orc.dequantize(B.Q4_K, gates[e0], n_ff * hidden).reshape(n_ff, hidden).T)
    ut = np.ascontiguousarray(orc.dequantize(B.Q4_K, ups[e0], n_ff * hidden).reshape(n_ff, hidden).T)
    dt = np.ascontiguousarray(orc.dequantize(B.Q6_K, downs[e0], hidden * n_ff).reshape(hidden, n_ff).T)
    g = np.empty((1, n_ff), np.float32)
    u = np.empty_like(g)
    out = np.empty((1, hidden), np.float32)
    rows, t_used = 0, 0.0
    while t_used < budget_s and rows < len(toks):
        xr = np.ascontiguousarray(x[toks[rows]:toks[rows] + 1], dtype=np.float32)
        t0 = time.perf_counter()
        orc.cpub_moe_expert_ffn(xr, 1, hidden, n_ff, gt, ut, dt, g, u, out)
        t_used += time.perf_counter() - t0
        rows += 1
    per_step = t_used / rows * n_assign
    cpu_model = host_cpu()
    return {
        "value": round(alg_bytes / per_step / 1e9, 6), "unit": "GB/s (algorithmic step bytes / CPU time)",
        "cores": 1, "kind": "port",
        "sample": (f"reference MoE step (moe_fused.rs:226-308 dispatch_experts, fused_ffn over ops::MatMul, one "
                   f"thread, f32 weights transposed at load, not timed); {rows} token rows of expert {e0} timed in "
                   f"{t_used:.2f} s and scaled to the step's {n_assign} assignments; {cpu_model}"),
        "host_cpu": cpu_model, "nproc": os.cpu_count(), "us_per_step": round(per_step * 1e6, 1),
    }


def bench_moe(args):
    """Config 5: the Mixtral-shaped MoE FFN step (barq_rocm_moe_ffn, integer path)
    on 64 tokens routed top-2 over 8 experts by the device router.  A step is
    one full expert FFN: gate/up (Q4_K), SwiGLU, down (Q6_K) and the weighted
    scatter; weights are 914 MB, beyond the 256 MB MALL, so no copies rotate."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import synth

    c = synth.MOE_CONFIG
    ne, hidden, n_ff, tokens, top_k = c["n_experts"], c["hidden"], c["n_ff"], c["tokens"], c["top_k"]
    log(f"generating {c['name']}")
    gates, ups, downs, x, logits = synth.moe_inputs(ne, hidden, n_ff, tokens, top_k)
    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    gd = [torch.from_numpy(g).cuda() for g in gates]
    ud = [torch.from_numpy(u).cuda() for u in ups]
    dd = [torch.from_numpy(d).cuda() for d in downs]
    xd = torch.from_numpy(x).cuda()
    ld = torch.from_numpy(logits).cuda()
    ids, wts = be.moe_route(ld, tokens, ne, top_k)
    torch.cuda.synchronize()

    out = torch.empty((tokens, hidden), dtype=torch.float32, device="cuda")

    def launch(i):
        be.moe_ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, hidden, n_ff, xd, tokens, ids, wts, top_k, B.ACT_F32_Q8,
                   sync=False, out=out)

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    # the whole step (five kernels, no host synchronisation) as one HIP graph
    ms, method = time_launches(launch, args.steps, args.eager)
    ms_eager, _ = time_launches(launch, args.steps, True)
    ids_h = ids.cpu().numpy()
    used = sorted(set(ids_h.reshape(-1).tolist()))
    wbytes = sum(gates[e].nbytes + ups[e].nbytes + downs[e].nbytes for e in used)
    alg = wbytes + tokens * hidden * 4 * 2 + tokens * top_k * (hidden + n_ff) * 292 // 256
    gbs = alg / (ms * 1e-3) / 1e9
    counts = np.bincount(ids_h.reshape(-1), minlength=ne).tolist()
    rel = None
    try:
        from oracle import oracle as orc
        sub = [0, 21, 42, 63]   # four tokens: the oracle restates the whole FFN per token in sequential f32
        ref = orc.moe_ffn(B.Q4_K, gates, B.Q4_K, ups, B.Q6_K, downs, hidden, n_ff, x[sub], ids_h[sub],
                          wts.cpu().numpy()[sub], orc.Q8_K)
        got = out.cpu().numpy()[sub]
        rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    except Exception as e:
        log(f"parity check skipped: {e}")
    result = {
        "metric": "MoE FFN step (Mixtral-8x7B shapes, 64 tokens top-2) achieved HBM GB/s + us/step, 1 GPU",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": c["name"], "experts_used": len(used), "tokens_per_expert": counts, "timing": method},
        "us_per_step": round(ms * 1e3, 2), "us_per_step_eager": round(ms_eager * 1e3, 2),
        "parity_rel_err_4_tokens": rel,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "alg_bytes_per_launch": alg,
                     "scope": "the whole step (grouping, quantizers, grouped GEMMs, scatter)"},
    }
    if args.probe_copy:
        src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    if not args.no_traffic:
        log("measuring HBM traffic per step (rocprofv3 --pmc child runs)")
        traffic, detail = measure_traffic(5)
        result["roofline"]["traffic"] = round(traffic) if traffic else None
        result["roofline"]["traffic_detail"] = detail
    if not args.no_cpu:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline_moe(gates, ups, downs, x, ids_h, hidden, n_ff, args.cpu_seconds, alg)
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def bench_norm(args):
    """RMSNorm fused with the Q8_K quantizer of the next projection
    (transformer.rs:148-172 then the activation quantize), Llama-3-8B hidden
    4096, at 1 and 512 rows, beside the unfused pair (rms_norm then
    quantize_act).  HBM-bound: x and the norm weight read, Q8_K written."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import synth

    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    n = 4096
    lines = {}
    for rows in (1, 512):
        x = torch.from_numpy(synth.gen_f32(rows * n, 7).reshape(rows, n)).cuda()
        w = torch.from_numpy((1.0 + 0.25 * synth.gen_f32(n, 8)).astype(np.float32)).cuda()
        q = torch.empty(rows * (n // 256) * 292, dtype=torch.uint8, device="cuda")
        y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()

        def fused(i):
            be.rms_norm_quantize_raw(B.Q8_K, x, w, rows, n, 1e-5, q, B.MEM_DEVICE)

        def unfused(i):
            be.rms_norm_raw(x, w, rows, n, 1e-5, y, B.MEM_DEVICE)
            be.quantize_act_raw(B.Q8_K, y, rows, n, q, B.MEM_DEVICE)
        for i in range(args.warmup):
            fused(i)
            unfused(i)
        ms_f, method = time_launches(fused, args.steps, args.eager)
        ms_u, _ = time_launches(unfused, args.steps, args.eager)
        alg = rows * n * 4 + n * 4 + rows * (n // 256) * 292
        lines[rows] = dict(us_fused=round(ms_f * 1e3, 3), us_unfused=round(ms_u * 1e3, 3),
                           gbs_fused=round(alg / (ms_f * 1e-3) / 1e9, 2), alg_bytes=alg, timing=method)
    big = lines[512]
    result = {
        "metric": "RMSNorm -> Q8_K fused achieved HBM GB/s (512 x 4096 rows) + us/call, 1 GPU",
        "value": big["gbs_fused"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(big["us_fused"] / 1e3, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "RMSNorm(4096) -> Q8_K, 1 and 512 rows", "rows": lines},
        "roofline": {"bound": "hbm", "achieved": big["gbs_fused"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(big["gbs_fused"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "alg_bytes_per_launch": big["alg_bytes"]},
    }
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def bench_ffn(args):
    """The dense FFN of one Llama-3-8B layer (LlamaTransformer::feed_forward,
    transformer.rs:378-408): Q4_K gate and up 14336 x 4096, SwiGLU, Q6_K down
    4096 x 14336 (the Q4_K_M mix), on m rows already quantized to Q8_K (the
    fused RMSNorm -> Q8_K of the layer writes them).  One token runs gate and
    up in one launch with the SwiGLU in its epilogue; beside it the same work
    as two separate GEMVs and the SwiGLU quantizer.  Layers rotate over
    enough weight copies (>= 1 GiB) that the Infinity Cache cannot hold them."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import synth

    n_embd, n_ff, m = 4096, 14336, args.m
    s0 = synth.config_seed(2)
    gate = synth.gen_q4_k(n_ff, n_embd, synth.sub_seed(s0, 40))
    up = synth.gen_q4_k(n_ff, n_embd, synth.sub_seed(s0, 41))
    down = synth.gen_q6_k(n_embd, n_ff, synth.sub_seed(s0, 42))
    x = synth.gen_f32(m * n_embd, synth.sub_seed(s0, 43)).reshape(m, n_embd)
    wbytes = gate.nbytes + up.nbytes + down.nbytes
    copies = args.copies or max(2, -(-ROTATE_BYTES // wbytes))
    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    layers = [tuple(torch.from_numpy(a).cuda() for a in (gate, up, down)) for _ in range(copies)]
    xq = be.quantize_act(B.Q8_K, torch.from_numpy(x).cuda(), sync=False)
    out = torch.empty((m, n_embd), dtype=torch.float32, device="cuda")
    g = torch.empty((m, n_ff), dtype=torch.float32, device="cuda")
    u = torch.empty((m, n_ff), dtype=torch.float32, device="cuda")
    hq = torch.empty(m * (n_ff // 256) * 292, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    def fused(i):
        gd, ud, dd = layers[i % copies]
        be.ffn(B.Q4_K, gd, B.Q4_K, ud, B.Q6_K, dd, n_embd, n_ff, B.Q8_K, xq, m, sync=False, out=out)

    def separate(i):
        gd, ud, dd = layers[i % copies]
        be.matmul_raw(B.Q4_K, gd, n_ff, n_embd, B.Q8_K, xq, m, g, B.MEM_DEVICE)
        be.matmul_raw(B.Q4_K, ud, n_ff, n_embd, B.Q8_K, xq, m, u, B.MEM_DEVICE)
        L = B._lib
        L.check(be._lib.barq_rocm_swiglu(be.h, B.Q8_K, g.data_ptr(), u.data_ptr(), m, n_ff, hq.data_ptr(),
                                         B.MEM_DEVICE))
        be.matmul_raw(B.Q6_K, dd, n_embd, n_ff, B.Q8_K, hq, m, out, B.MEM_DEVICE)

    for i in range(args.warmup):
        fused(i)
        separate(i)
    torch.cuda.synchronize()
    log(f"timing {args.steps} FFN calls over {copies} layer copies ({copies * wbytes / 2**20:.0f} MiB)")
    ms, method = time_launches(fused, args.steps, args.eager)
    ms_sep, _ = time_launches(separate, args.steps, args.eager)
    fused(0)
    torch.cuda.synchronize()
    alg = wbytes + m * (n_embd // 256) * 292 + m * (n_ff // 256) * 292 + m * n_ff * 4 * 2 + m * n_embd * 4
    gbs = alg / (ms * 1e-3) / 1e9
    rel = None
    try:
        from oracle import oracle as orc
        ref = orc.ffn(B.Q4_K, gate, B.Q4_K, up, B.Q6_K, down, n_embd, n_ff, orc.Q8_K, xq.cpu().numpy(), m)
        got = out.cpu().numpy()
        rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    except Exception as e:
        log(f"parity check skipped: {e}")
    result = {
        "metric": "dense FFN (Llama-3-8B, gate/up Q4_K + down Q6_K) achieved HBM GB/s + us/call, 1 GPU",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"feed_forward 4096 -> 14336 -> 4096, {m} token(s), x as Q8_K",
                   "layer_copies": copies, "timing": method},
        "us_per_call": round(ms * 1e3, 3), "us_per_call_separate_launches": round(ms_sep * 1e3, 3),
        "parity_rel_err": rel,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "alg_bytes_per_launch": alg,
                     "scope": "the whole FFN call (gate/up, SwiGLU + Q8_K, down)"},
    }
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def bench_decode(args):
    """One decode token of a Llama-3-8B-shaped model (LlamaTransformer::forward
    for one token, transformer.rs:81-94: get_embeddings, 32 x forward_layer
    :123-144, final_output :468-498) on the integer path through
    barq_rocm.llama.DeviceLlama (the chain tests/test_gpu_token.py checks
    against the oracle), every launch of a token captured in one HIP graph.
    Each layer has its own KV cache of --kv-len cached positions and its own
    copy of a Q4_K_M layer's weights (32 copies of the same synthetic contents
    at distinct addresses, 4.4 GB: no cache holds them across layers);
    token_embd Q4_K and the LM head Q6_K are 128256 x 4096.  Synthetic
    weights and activations."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import attention as A
    from barq_rocm import synth
    from barq_rocm.llama import DeviceLlama, LlamaConfig

    cfg = LlamaConfig(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128, n_ff=14336)
    n_vocab = 128256
    kv_len = args.kv_len
    tokens = args.steps if args.steps <= 16 else 4
    mats = [("attn_q", B.Q4_K, cfg.n_head * cfg.head_dim, cfg.n_embd), ("attn_k", B.Q4_K, cfg.n_head_kv * cfg.head_dim, cfg.n_embd),
            ("attn_v", B.Q6_K, cfg.n_head_kv * cfg.head_dim, cfg.n_embd), ("attn_output", B.Q4_K, cfg.n_embd, cfg.n_head * cfg.head_dim),
            ("ffn_gate", B.Q4_K, cfg.n_ff, cfg.n_embd), ("ffn_up", B.Q4_K, cfg.n_ff, cfg.n_embd),
            ("ffn_down", B.Q6_K, cfg.n_embd, cfg.n_ff)]
    log("generating the synthetic layer, embedding and LM-head weights")
    host = {nm: synth.gen_weights(t, n, k, 800 + i) for i, (nm, t, n, k) in enumerate(mats)}
    types = {nm: (t, n, k) for nm, t, n, k in mats}
    head_h = synth.gen_weights(B.Q6_K, n_vocab, cfg.n_embd, 880)
    emb_h = synth.gen_weights(B.Q4_K, n_vocab, cfg.n_embd, 881)
    wbytes = sum(a.nbytes for a in host.values())
    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    tensors, keep = {}, []
    norm_w = torch.from_numpy((0.01 * (1.0 + 0.1 * synth.gen_f32(cfg.n_embd, 820))).astype(np.float32)).cuda()
    keep.append(norm_w)
    for il in range(cfg.n_layer):
        for nm, a in host.items():
            d = torch.from_numpy(a).cuda()
            keep.append(d)
            tensors[f"blk.{il}.{nm}.weight"] = (*types[nm], d.data_ptr())
        for nm in ("attn_norm", "ffn_norm"):
            tensors[f"blk.{il}.{nm}.weight"] = (0, 1, cfg.n_embd, norm_w.data_ptr())
    for nm, t, a in (("output.weight", B.Q6_K, head_h), ("token_embd.weight", B.Q4_K, emb_h)):
        d = torch.from_numpy(a).cuda()
        keep.append(d)
        tensors[nm] = (t, n_vocab, cfg.n_embd, d.data_ptr())
    tensors["output_norm.weight"] = (0, 1, cfg.n_embd, norm_w.data_ptr())
    head_bytes = head_h.nbytes
    del host, head_h, emb_h
    kv = A.KVCache(be, kv_len + 3 * tokens + 8, cfg.n_layer, cfg.n_head_kv, cfg.head_dim)
    rng = np.random.default_rng(5)
    kk = rng.standard_normal((cfg.n_head_kv, kv_len - 1, cfg.head_dim)).astype(np.float32)
    kkd = torch.from_numpy(kk).cuda()
    for layer in range(cfg.n_layer):   # kv_len - 1 cached positions per layer
        kv.append(layer, kkd, kkd * 0.5, kv_len - 1, cfg.head_dim)
    del kkd
    llama = DeviceLlama(be, cfg, tensors.get, kv)
    tok = torch.tensor([1234], dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    pos = [kv_len - 1]

    def token(i):
        llama.forward(tok, pos[0])
        pos[0] += 1

    token(0)   # warm-up outside the graph (workspace, kernel attributes, activation buffers)
    torch.cuda.synchronize()
    log(f"timing {tokens} decode tokens ({cfg.n_layer} layers, kv_len {kv_len})")
    ms, method = time_launches(token, tokens, args.eager)
    kv_bytes = 2 * cfg.n_head_kv * kv_len * cfg.head_dim * 4
    alg = cfg.n_layer * (wbytes + kv_bytes) + head_bytes
    gbs = alg / (ms * 1e-3) / 1e9
    result = {
        "metric": f"Llama-3-8B-shaped decode (batch 1, kv_len {kv_len}) tokens/s, 1 GPU",
        "value": round(1e3 / ms, 2), "unit": "tokens/s", "n_gpus": 1, "steps": tokens, "warmup": 1,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"LlamaTransformer forward, 1 token, {cfg.n_layer} layers (Q4_K_M mix, one weight copy "
                               f"per layer), kv_len {kv_len}, token_embd Q4_K + LM head Q6_K {n_vocab} x {cfg.n_embd}",
                   "timing": method},
        "ms_per_token": round(ms, 4),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "alg_bytes_per_launch": alg,
                     "scope": "one token: 32 layers' weights and K/V rows, the LM head, activations not counted"},
    }
    kv.close()
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def bench_prefill(args):
    """One Llama-3-8B layer over an M-token prompt from position 0
    (forward_layer, transformer.rs:123-144, with seq_len = M) on the integer
    path: residual add + attn_norm -> Q8_K rows, q / k / v GEMMs (int8 MFMA),
    RoPE of q and k with the cache append, causal attention (f32 MFMA) with
    its rows quantized for the o GEMM, residual add + ffn_norm -> Q8_K, the
    dense FFN (gate/up GEMMs, SwiGLU -> Q8_K, down GEMM).  Steps rotate over
    layer copies of >= 1 GiB.  Throughput: prompt tokens per second through
    one layer; the op count is 2 M N K over the seven projections plus the
    attention's 4 hd per visible (query, position) pair and head."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import attention as A
    from barq_rocm import synth

    n_embd, n_head, n_kv, hd, n_ff = 4096, 32, 8, 128, 14336
    m = args.m if args.m > 1 else 512
    mats = [("q", B.Q4_K, n_head * hd, n_embd), ("k", B.Q4_K, n_kv * hd, n_embd), ("v", B.Q6_K, n_kv * hd, n_embd),
            ("o", B.Q4_K, n_embd, n_head * hd), ("gate", B.Q4_K, n_ff, n_embd), ("up", B.Q4_K, n_ff, n_embd),
            ("down", B.Q6_K, n_embd, n_ff)]
    host = {nm: synth.gen_weights(t, n, k, 800 + i) for i, (nm, t, n, k) in enumerate(mats)}
    wbytes = sum(a.nbytes for a in host.values())
    copies = args.copies or max(2, -(-ROTATE_BYTES // wbytes))
    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    layers = [{nm: torch.from_numpy(a).cuda() for nm, a in host.items()} for _ in range(copies)]
    norm_w = torch.from_numpy((0.01 * (1.0 + 0.1 * synth.gen_f32(n_embd, 820))).astype(np.float32)).cuda()
    f = torch.from_numpy(np.array([np.float32(500000.0) ** np.float32(-2.0 * i / hd) for i in range(hd // 2)],
                                  dtype=np.float32)).cuda()
    kv = A.KVCache(be, m, copies, n_kv, hd)
    x = torch.from_numpy(synth.gen_f32(m * n_embd, 821).reshape(m, n_embd)).cuda()
    prev = torch.zeros((m, n_embd), dtype=torch.float32, device="cuda")
    res_in, res = torch.empty_like(x), torch.empty_like(x)
    nbq = n_embd // 256 * 292
    xq = torch.empty((m, nbq), dtype=torch.uint8, device="cuda")
    xq2, aq = torch.empty_like(xq), torch.empty_like(xq)
    q = torch.empty((m, n_head * hd), dtype=torch.float32, device="cuda")
    k = torch.empty((m, n_kv * hd), dtype=torch.float32, device="cuda")
    v = torch.empty((m, n_kv * hd), dtype=torch.float32, device="cuda")
    qr = torch.empty((n_head, m, hd), dtype=torch.float32, device="cuda")
    o = torch.empty((m, n_embd), dtype=torch.float32, device="cuda")
    ff = torch.empty((m, n_embd), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        c = i % copies
        L = layers[c]
        kv.clear()   # host lengths only: every step writes positions 0 .. m-1 of its layer copy
        be.add_rms_norm_quantize(B.Q8_K, x, prev, norm_w, 1e-5, sum_out=res_in, out=xq, sync=False)
        be.matmul_raw(B.Q4_K, L["q"], n_head * hd, n_embd, B.Q8_K, xq, m, q, B.MEM_DEVICE)
        be.matmul_raw(B.Q4_K, L["k"], n_kv * hd, n_embd, B.Q8_K, xq, m, k, B.MEM_DEVICE)
        be.matmul_raw(B.Q6_K, L["v"], n_kv * hd, n_embd, B.Q8_K, xq, m, v, B.MEM_DEVICE)
        kv.append_rope_q(c, q, n_head, k, v, m, 0, 1.0, f, A.ROPE_INTERLEAVED, q_out=qr)
        A.compute_attention_q8k(be, qr, kv, c, n_head, n_kv, hd, m, m, 0, sync=False, out=aq)
        be.matmul_raw(B.Q4_K, L["o"], n_embd, n_head * hd, B.Q8_K, aq, m, o, B.MEM_DEVICE)
        be.add_rms_norm_quantize(B.Q8_K, res_in, o, norm_w, 1e-5, sum_out=res, out=xq2, sync=False)
        be.ffn(B.Q4_K, L["gate"], B.Q4_K, L["up"], B.Q6_K, L["down"], n_embd, n_ff, B.Q8_K, xq2, m, sync=False,
               out=ff)

    for i in range(copies):
        step(i)
    torch.cuda.synchronize()
    steps = args.steps
    log(f"timing {steps} prefill-layer steps of {m} tokens over {copies} layer copies")
    ms, method = time_launches(step, steps, args.eager)
    ops = 2 * m * sum(n * kk for _, _, n, kk in mats) + 2 * 2 * n_head * hd * (m * (m + 1) // 2)
    tops = ops / (ms * 1e-3) / 1e12
    result = {
        "metric": f"Llama-3-8B prefill layer ({m}-token prompt, integer path) tokens/s through one layer, 1 GPU",
        "value": round(m / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": copies,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 (GEMMs) + f32 (attention)", "data": "synthetic",
        "config": {"workload": f"forward_layer prefill, {m} tokens from position 0, Q4_K_M weight mix",
                   "layer_copies": copies, "timing": method},
        "us_per_step": round(ms * 1e3, 3), "tera_ops_per_s": round(tops, 2),
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOP/s (int8)",
                     "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None, "alg_ops_per_launch": ops,
                     "scope": "the whole layer step (13 launches); the attention's f32 ops are counted at the int8 peak"},
    }
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def bench_layer(args):
    """One decode step of a Llama-3-8B layer (forward_layer,
    transformer.rs:123-144) on the integer path, every launch captured in one
    HIP graph: residual add + attn_norm -> Q8_K, q / k / v GEMVs (Q4_K, Q4_K,
    Q6_K), RoPE(q), RoPE(k) + V transpose + KV append, attention over kv_len
    cached positions, output projection (f32 -> Q8_K in the call), residual
    add + ffn_norm -> Q8_K, the dense FFN (gate/up Q4_K, down Q6_K).  Steps
    rotate over enough layer copies (weights and KV cache) that the Infinity
    Cache cannot hold them.  Algorithmic bytes: the layer's packed weights,
    the K and V rows attention reads, and the activations."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import attention as A
    from barq_rocm import synth

    n_embd, n_head, n_kv, hd, n_ff = 4096, 32, 8, 128, 14336
    kv_len = args.kv_len
    mats = [("q", B.Q4_K, n_head * hd, n_embd), ("k", B.Q4_K, n_kv * hd, n_embd), ("v", B.Q6_K, n_kv * hd, n_embd),
            ("o", B.Q4_K, n_embd, n_head * hd), ("gate", B.Q4_K, n_ff, n_embd), ("up", B.Q4_K, n_ff, n_embd),
            ("down", B.Q6_K, n_embd, n_ff)]
    host = {nm: synth.gen_weights(t, n, k, 800 + i) for i, (nm, t, n, k) in enumerate(mats)}
    wbytes = sum(a.nbytes for a in host.values())
    kv_bytes = 2 * n_kv * kv_len * hd * 4
    copies = args.copies or max(2, -(-ROTATE_BYTES // (wbytes + kv_bytes)))
    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    layers = [{nm: torch.from_numpy(a).cuda() for nm, a in host.items()} for _ in range(copies)]
    norm_w = torch.from_numpy((0.01 * (1.0 + 0.1 * synth.gen_f32(n_embd, 820))).astype(np.float32)).cuda()
    f = torch.from_numpy(np.array([np.float32(500000.0) ** np.float32(-2.0 * i / hd) for i in range(hd // 2)],
                                  dtype=np.float32)).cuda()
    steps = args.steps
    kv = A.KVCache(be, kv_len + 2 * steps + 4 * copies + 8, copies, n_kv, hd)   # two timed captures
    rng = np.random.default_rng(5)
    for c in range(copies):   # kv_len - 1 cached positions per layer copy
        kk = rng.standard_normal((n_kv, kv_len - 1, hd)).astype(np.float32)
        kv.append(c, kk, kk * 0.5, kv_len - 1, hd, mem=B.MEM_HOST)
    x = torch.from_numpy(synth.gen_f32(n_embd, 821)).cuda().reshape(1, n_embd)
    prev = torch.zeros((1, n_embd), dtype=torch.float32, device="cuda")
    res_in = torch.empty_like(x)
    res = torch.empty_like(x)
    xq = torch.empty((n_embd // 256) * 292, dtype=torch.uint8, device="cuda")
    xq2 = torch.empty_like(xq)
    q = torch.empty((1, n_head * hd), dtype=torch.float32, device="cuda")
    k = torch.empty((1, n_kv * hd), dtype=torch.float32, device="cuda")
    v = torch.empty((1, n_kv * hd), dtype=torch.float32, device="cuda")
    o = torch.empty((1, n_embd), dtype=torch.float32, device="cuda")
    ff = torch.empty((1, n_embd), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    pos = [kv_len - 1] * copies
    qkv_types = [B.Q4_K, B.Q4_K, B.Q6_K]

    qr = torch.empty((n_head, 1, hd), dtype=torch.float32, device="cuda")
    aq = torch.empty((1, (n_embd // 256) * 292), dtype=torch.uint8, device="cuda")

    def step_separate(i):
        # every reference step its own launch: RoPE q, RoPE k + v into the
        # cache, attention in f32, the o projection quantizing its input
        c = i % copies
        L = layers[c]
        be.add_rms_norm_quantize(B.Q8_K, x, prev, norm_w, 1e-5, sum_out=res_in, out=xq, sync=False)
        be.matmul_raw(B.Q4_K, L["q"], n_head * hd, n_embd, B.Q8_K, xq, 1, q, B.MEM_DEVICE)
        be.matmul_raw(B.Q4_K, L["k"], n_kv * hd, n_embd, B.Q8_K, xq, 1, k, B.MEM_DEVICE)
        be.matmul_raw(B.Q6_K, L["v"], n_kv * hd, n_embd, B.Q8_K, xq, 1, v, B.MEM_DEVICE)
        q_rope = A.apply_rope(be, q, 1, n_head, hd, pos[c], 1.0, f, A.ROPE_INTERLEAVED, sync=False)
        kv.append_rope(c, k, v, 1, pos[c], 1.0, f, A.ROPE_INTERLEAVED)
        attn = A.compute_attention(be, q_rope, kv, c, n_head, n_kv, hd, 1, pos[c] + 1, pos[c], sync=False)
        pos[c] += 1
        be.matmul_raw(B.Q4_K, L["o"], n_embd, n_head * hd, B.ACT_F32_Q8, attn.reshape(1, n_embd), 1, o, B.MEM_DEVICE)
        be.add_rms_norm_quantize(B.Q8_K, res_in, o, norm_w, 1e-5, sum_out=res, out=xq2, sync=False)
        be.ffn(B.Q4_K, L["gate"], B.Q4_K, L["up"], B.Q6_K, L["down"], n_embd, n_ff, B.Q8_K, xq2, 1, sync=False,
               out=ff)

    def step(i):
        # fused: the q/k/v projections with RoPE and the cache append in one
        # launch, the attention merge writing the o projection's Q8_K rows
        c = i % copies
        L = layers[c]
        be.add_rms_norm_quantize(B.Q8_K, x, prev, norm_w, 1e-5, sum_out=res_in, out=xq, sync=False)
        kv.qkv_append_rope(c, qkv_types, [L["q"], L["k"], L["v"]], n_head, n_embd, B.Q8_K, xq, pos[c], 1.0, f,
                           A.ROPE_INTERLEAVED, q_out=qr)
        A.compute_attention_q8k(be, qr, kv, c, n_head, n_kv, hd, 1, pos[c] + 1, pos[c], sync=False, out=aq)
        pos[c] += 1
        be.matmul_raw(B.Q4_K, L["o"], n_embd, n_head * hd, B.Q8_K, aq, 1, o, B.MEM_DEVICE)
        be.add_rms_norm_quantize(B.Q8_K, res_in, o, norm_w, 1e-5, sum_out=res, out=xq2, sync=False)
        be.ffn(B.Q4_K, L["gate"], B.Q4_K, L["up"], B.Q6_K, L["down"], n_embd, n_ff, B.Q8_K, xq2, 1, sync=False,
               out=ff)

    # warm-up outside the graph (workspace, kernel attributes): one step per layer copy
    for i in range(copies):
        step(i)
    torch.cuda.synchronize()
    log(f"timing {steps} decode-layer steps over {copies} layer copies "
        f"({copies * (wbytes + kv_bytes) / 2**20:.0f} MiB of weights and KV)")
    ms_sep, _ = time_launches(step_separate, steps, args.eager)
    for i in range(copies):
        step(i)
    torch.cuda.synchronize()
    ms, method = time_launches(step, steps, args.eager)
    alg = wbytes + kv_bytes + 4 * n_embd * 4 * 4
    gbs = alg / (ms * 1e-3) / 1e9
    result = {
        "metric": "Llama-3-8B decode layer (integer path) achieved HBM GB/s + us/step, 1 GPU",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": copies,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"forward_layer decode, 1 token, kv_len {kv_len}, Q4_K_M weight mix",
                   "layer_copies": copies, "timing": method},
        "us_per_step": round(ms * 1e3, 3), "us_per_step_separate_launches": round(ms_sep * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "alg_bytes_per_launch": alg,
                     "scope": "the whole layer step (9 launches; 15 with every reference step its own launch)"},
    }
    kv.close()
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def bench_attn(args):
    """Decode attention (compute_attention, transformer.rs:301-374) at the
    Llama-3-8B head layout: 32 query heads, 8 kv heads, head_dim 128, one new
    token against kv_len cached positions in f32.  HBM-bound: every call
    reads the layer's K and V rows once (2 * 8 * kv_len * 128 * 4 bytes).
    Calls rotate over enough cache layers (>= 1 GiB) that the Infinity Cache
    cannot hold them.  The CPU leg times the oracle's restatement of
    compute_attention (one core) on a bounded number of calls."""
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import attention as A

    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)
    n_head, n_kv, hd, kv, ql = 32, 8, 128, args.kv_len, args.q_len
    assert 1 <= ql <= kv
    layer_bytes = 2 * n_kv * kv * hd * 4
    layers = max(2, -(-ROTATE_BYTES // layer_bytes))
    log(f"attention: {n_head} heads / {n_kv} kv heads x {hd}, kv_len {kv}, {layers} cache layers "
        f"({layers * layer_bytes / 2**20:.0f} MiB)")
    cache = A.KVCache(be, kv, layers, n_kv, hd)
    g = torch.Generator(device="cuda").manual_seed(1234)
    for layer in range(layers):
        k = torch.randn((n_kv, kv, hd), generator=g, device="cuda", dtype=torch.float32)
        v = torch.randn((n_kv, kv, hd), generator=g, device="cuda", dtype=torch.float32)
        cache.append(layer, k, v, kv, hd)
        del k, v
    q = torch.randn((n_head, ql, hd), generator=g, device="cuda", dtype=torch.float32)
    out = torch.empty((ql, n_head, hd), dtype=torch.float32, device="cuda")
    lib = be._lib

    def launch(i):
        B._lib.check(lib.barq_rocm_attention(be.h, q.data_ptr(), cache.c, i % layers, n_head, n_kv, hd, ql, kv,
                                             kv - ql, out.data_ptr(), B.MEM_DEVICE))
    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    ms, method = time_launches(launch, args.steps, args.eager)
    ms_eager, _ = time_launches(launch, args.steps, True)
    alg = layer_bytes + 2 * ql * n_head * hd * 4
    gbs = alg / (ms * 1e-3) / 1e9
    # causal: query i sees kv - ql + i + 1 positions; two FMAs (q.k, p.v) per dim per visible position
    flops = 2 * 2 * n_head * hd * sum(kv - ql + i + 1 for i in range(ql))

    # parity of layer 0 against the oracle, and the CPU leg
    launch(0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kh = np.stack([cache.get_head(0, h)[0] for h in range(n_kv)])
    vh = np.stack([cache.get_head(0, h)[1] for h in range(n_kv)])
    qn = q.cpu().numpy()
    from oracle import oracle as O
    t0 = time.perf_counter()
    ref = O.attention(qn, kh, vh, n_head, ql, kv, kv - ql)
    calls, t_cpu = 1, time.perf_counter() - t0
    while not args.no_cpu and t_cpu < min(args.cpu_seconds, 20.0):
        O.attention(qn, kh, vh, n_head, ql, kv, kv - ql)
        calls += 1
        t_cpu = time.perf_counter() - t0
    err = float(np.max(np.abs(got - ref)) / np.max(np.abs(vh)))
    cpu_gbs = alg * calls / t_cpu / 1e9
    # prompt chunks of 32+ rows run the f32-MFMA kernel: compute-bound
    mfma = ql >= int(os.environ.get("BARQ_ATTN_MFMA_MIN_Q", "32"))
    tflops = flops / (ms * 1e-3) / 1e12
    if mfma:
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": F32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s (f32)",
                "frac": round(tflops / F32_MFMA_PEAK_TFLOPS, 4), "traffic": None, "alg_flops_per_launch": flops,
                "scope": "one call: the MFMA prompt kernel"}
    else:
        roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "alg_bytes_per_launch": alg,
                "scope": "one call: the split kernel and the split-combine kernel"}
    result = {
        "metric": f"{'decode' if ql == 1 else 'prompt-chunk'} attention (Llama-3-8B heads, q_len {ql}, kv_len {kv}) "
                  + ("achieved f32 TFLOP/s + us/call, 1 GPU" if mfma else "achieved HBM GB/s + us/call, 1 GPU"),
        "value": round(tflops, 2) if mfma else round(gbs, 2), "unit": "TFLOP/s" if mfma else "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"attention 32 q heads / 8 kv heads x 128, q_len {ql}, kv_len {kv}, f32 KV cache",
                   "cache_layers_rotated": layers, "timing": method},
        "us_per_call": round(ms * 1e3, 3), "us_per_call_eager": round(ms_eager * 1e3, 3),
        "gflops": round(flops / (ms * 1e-3) / 1e9, 1),
        "parity_max_err_rel_to_max_v": err,
        "roofline": roof,
        "cpu_baseline": {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"{calls} calls of the oracle's compute_attention restatement on layer 0",
                         "us_per_call": round(t_cpu / calls * 1e6, 1)},
    }
    cache.close()
    be.close()
    print(json.dumps(result), flush=True)
    return 0


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the quantized-linear path here is single-GPU by design "
              f"(--gpus {args.gpus} is not supported; run with --gpus 1)", flush=True)
        return 2
    import numpy as np
    import torch

    import barq_rocm as B
    from barq_rocm import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.norm:
        return bench_norm(args)
    if args.attn:
        return bench_attn(args)
    if args.ffn:
        return bench_ffn(args)
    if args.layer:
        return bench_layer(args)
    if args.prefill:
        return bench_prefill(args)
    if args.decode:
        return bench_decode(args)
    if args.config == 5:
        return bench_moe(args)
    cfg = synth.CONFIGS[args.config]
    w_type, n, k, m = cfg["w_type"], cfg["n_rows"], cfg["k"], cfg["m"]
    workload = cfg["name"]
    if args.m > 1 and args.config in (1, 2, 3):
        m = args.m
        workload = f"{cfg['name']}, {m} activation rows (small decode batch)"
    log(f"generating {cfg['name']}")
    t, w, x = synth.linear_inputs(args.config, m=m)
    if args.w_type:
        # the same shape and activation with weights of another format
        w_type = getattr(B, args.w_type)
        w = synth.gen_weights(w_type, n, k, synth.sub_seed(synth.config_seed(args.config), 10))
        act_name = "Q8_K" if B.Q8_PARTNER[w_type] == B.Q8_K else "Q8_0"
        workload = (f"C{args.config} shape with {args.w_type} weights: {n}x{k}, "
                    + (f"batch 1, x->{act_name}" if m == 1 else f"M={m}, X->{act_name}"))
    at = B.Q8_PARTNER[w_type]
    wbytes = w.nbytes
    copies = args.copies or max(2, -(-ROTATE_BYTES // wbytes))
    be = B.Backend(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    be.set_stream(stream.cuda_stream)

    w0 = torch.from_numpy(w).cuda()
    ws = [w0] + [w0.clone() for _ in range(copies - 1)]
    xd = torch.from_numpy(x).cuda()
    xq = be.quantize_act(at, xd, sync=False)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    if m == 1:
        def launch(i):
            be.matvec_raw(w_type, ws[i % copies], n, k, at, xq, y, B.MEM_DEVICE)
    else:
        def launch(i):
            be.matmul_raw(w_type, ws[i % copies], n, k, at, xq, m, y, B.MEM_DEVICE)

    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps over {copies} weight copies ({copies * wbytes / 2**20:.0f} MiB)")
    ms, method = time_launches(launch, args.steps, args.eager)
    ms_eager, _ = time_launches(launch, args.steps, True)

    def qlaunch(i):
        be.quantize_act_raw(at, xd, m, k, xq, B.MEM_DEVICE)
    q_ms, _ = time_launches(qlaunch, args.steps, args.eager)

    alg = algorithmic_bytes(w_type, n, k, m)
    fixed = {}
    if m == 1 and not args.no_fixed:
        # What a launch costs apart from its bytes: a one-element fill kernel
        # timed the same way on the same stream (the graph's per-launch floor),
        # and the same GEMV over twice the rows, whose extra time gives the
        # streaming rate once the launch is under way.
        t1 = torch.zeros(1, device="cuda")

        def flaunch(i):
            t1.fill_(float(i))
        floor_ms, _ = time_launches(flaunch, args.steps, args.eager)
        w2 = torch.cat([w0, w0])
        copies2 = max(2, -(-ROTATE_BYTES // (2 * wbytes)))
        ws2 = [w2] + [w2.clone() for _ in range(copies2 - 1)]
        y2 = torch.empty(2 * n, dtype=torch.float32, device="cuda")

        def launch2(i):
            be.matvec_raw(w_type, ws2[i % copies2], 2 * n, k, at, xq, y2, B.MEM_DEVICE)
        for i in range(min(args.warmup, 500)):
            launch2(i)
        torch.cuda.synchronize()
        ms2, _ = time_launches(launch2, args.steps, args.eager)
        extra = algorithmic_bytes(w_type, 2 * n, k, 1) - alg
        fixed = {"launch_floor_us": round(floor_ms * 1e3, 3), "us_per_call_2x_rows": round(ms2 * 1e3, 3),
                 "marginal_gbs": round(extra / ((ms2 - ms) * 1e-3) / 1e9, 1) if ms2 > ms else None}
        del ws2, w2
        # the streaming-read floor of the same weight bytes, same copies, graph and stream
        sink = torch.zeros(1, dtype=torch.int32, device="cuda")

        def slaunch(i):
            B._lib.check(be._lib.barq_rocm_stream_read(be.h, ws[i % copies].data_ptr(), wbytes, sink.data_ptr()))
        for i in range(min(args.warmup, 500)):
            slaunch(i)
        torch.cuda.synchronize()
        st_ms, _ = time_launches(slaunch, args.steps, args.eager)
        fixed.update({"stream_floor_us": round(st_ms * 1e3, 3),
                      "stream_floor_gbs": round(wbytes / (st_ms * 1e-3) / 1e9, 1),
                      "us_over_stream_floor": round((ms - st_ms) * 1e3, 3)})
    us = ms * 1e3
    gbs = alg / (ms * 1e-3) / 1e9
    # correctness of the timed output against the oracle
    ok = None
    try:
        from oracle import oracle as orc
        rows = np.linspace(0, m - 1, min(m, 16)).astype(int)   # a spread of rows keeps the oracle quick
        rb = B.row_bytes(at, k)
        xq_h = xq.cpu().numpy()
        sub = np.concatenate([xq_h[r * rb:(r + 1) * rb] for r in rows])
        ref = orc.matmul(w_type, w, n, k, at, sub, len(rows))
        yy = y.cpu().numpy().reshape(m, n)[rows]
        ok = float(np.linalg.norm(yy - ref) / np.linalg.norm(ref))
    except Exception as e:
        log(f"parity check skipped: {e}")

    fmt_name = {B.Q4_0: "Q4_0", B.Q8_0: "Q8_0", B.Q4_K: "Q4_K", B.Q6_K: "Q6_K", B.Q4_0_BARQ: "Q4_0_BARQ"}.get(w_type, "quantized")
    metric = METRIC if args.config == 2 and not args.w_type else f"{fmt_name} GEMV achieved HBM GB/s (% of peak) + µs/call, 1 GPU"
    result = {
        "metric": metric,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": workload, "n_rows": n, "k": k, "batch": m, "weight_copies": copies,
                   "weight_bytes_per_copy": wbytes, "timing": method},
        "us_per_call": round(us, 3),
        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "us_per_call_eager": round(ms_eager * 1e3, 3),
        "act_quant_us": round(q_ms * 1e3, 3),
        **fixed,
        "parity_rel_err": ok,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "alg_bytes_per_launch": alg},
    }
    if m >= 16:
        # the batched path is bound by int8 MFMA: 2*M*N*K ops per launch
        ops = 2.0 * m * n * k
        tops = ops / (ms * 1e-3) / 1e12
        result["metric"] = f"{fmt_name} batched GEMM int8 TOP/s (% of dense int8 MFMA peak), 1 GPU"
        result["value"] = round(tops, 2)
        result["unit"] = "TOP/s"
        result["roofline"] = {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS,
                              "unit": "TOP/s (int8)", "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": None,
                              "alg_ops_per_launch": ops, "alg_bytes_per_launch": alg,
                              "hbm_gbs_alg": round(gbs, 2)}
    if args.probe_copy:
        src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy probe: 5 x 256 MiB device copies")
    small_batch = args.config in (1, 2, 3) and m > 1   # the counter runs and the CPU sample are one-token
    if not args.no_traffic and not small_batch:
        log("measuring HBM traffic per launch (rocprofv3 --pmc child runs)")
        traffic, detail = measure_traffic(args.config, args.w_type)
        result["roofline"]["traffic"] = round(traffic) if traffic else None
        result["roofline"]["traffic_detail"] = detail
    if not args.no_cpu and not small_batch:
        log("timing the CPU baseline")
        if m == 1:
            result["cpu_baseline"] = cpu_baseline(w_type, w, x[0], n, k, args.cpu_seconds, alg)
        else:
            result["cpu_baseline"] = cpu_baseline_gemm(w_type, w, x, n, k, m, args.cpu_seconds)
    be.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
