// Device side of the fused MoE helpers (models/src/moe_fused.rs): top-k
// routing, grouping of assignments by expert, row gather, SwiGLU and the
// weighted scatter-add.  The expert contractions themselves run on the GEMV /
// MFMA kernels.
#include "common.hpp"
#include "launch.hpp"
#include "q8k_block.hpp"

namespace barq {

constexpr int MOE_MAX_EXPERTS = 256;
constexpr int MOE_MAX_TOPK = 64;
constexpr int MOE_FUSED_MAX = 2048;   // assignments the fused grouping + gather handles
constexpr float F32_EPSILON = 1.1920929e-7f;

// reduce_expert_assignments (moe_fused.rs:147-194) on one row of k slots
// held by the calling thread (ci: expert ids, id < 0 an absent slot; cw:
// weights).  Keeps the slots with weight >= min_w (none: the largest, the
// later slot winning ties, as Iterator::max_by with partial_cmp does), sorts
// them by weight descending (stable), keeps at most keep_max and divides by
// their sequential sum floored at f32::EPSILON.  The kept slots end up first;
// returns their number.
__device__ int ser_reduce_row(int* ci, float* cw, int k, int keep_max, float min_w) {
    int n = 0, best = -1;
    float bw = 0.0f;
    for (int i = 0; i < k; i++) {
        const int e = ci[i];
        const float w = cw[i];
        if (e < 0) continue;
        if (best < 0 || !(bw > w)) { best = e; bw = w; }
        if (w >= min_w) { ci[n] = e; cw[n] = w; n++; }   // n <= i: reads stay ahead of writes
    }
    if (n == 0 && best >= 0) { ci[0] = best; cw[0] = bw; n = 1; }
    for (int i = 1; i < n; i++) {
        const int ti = ci[i];
        const float tw = cw[i];
        int j = i;
        while (j > 0 && cw[j - 1] < tw) { ci[j] = ci[j - 1]; cw[j] = cw[j - 1]; j--; }
        ci[j] = ti;
        cw[j] = tw;
    }
    if (n > keep_max) n = keep_max;
    float sum = -0.0f;
    for (int i = 0; i < n; i++) sum += cw[i];
    sum = fmaxf(sum, F32_EPSILON);
    for (int i = 0; i < n; i++) cw[i] = cw[i] / sum;
    return n;
}

// select_top_k_experts (moe_fused.rs:95-144), one thread per row: a stable
// descending sort keeps equal logits in index order, so the first k picks
// are the largest values with the lowest index winning ties; softmax over
// the kept k with the max subtracted and the denominator floored at
// f32::EPSILON.  k = clamp(top_k, 1, n_experts) (:121).  With keep_max > 0
// the row then goes through reduce_expert_assignments (the MoE forward of
// advanced/src/moe.rs:157-162); dropped slots get id -1, weight 0.
__global__ __launch_bounds__(64) void moe_route_kernel(const float* __restrict__ logits, int rows, int ne,
                                                       int k, int keep_max, float min_w,
                                                       int32_t* __restrict__ ids, float* __restrict__ weights) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float* row = logits + (size_t)r * ne;
    uint64_t taken[MOE_MAX_EXPERTS / 64] = {0, 0, 0, 0};
    int sel[MOE_MAX_TOPK];
    float sw[MOE_MAX_TOPK];
    for (int i = 0; i < k; i++) {
        int best = -1;
        float bv = 0.0f;
        for (int e = 0; e < ne; e++) {
            if ((taken[e >> 6] >> (e & 63)) & 1u) continue;
            const float v = row[e];
            if (best < 0 || v > bv) { best = e; bv = v; }
        }
        taken[best >> 6] |= (uint64_t)1 << (best & 63);
        sel[i] = best;
    }
    float mx = -INFINITY;
    for (int i = 0; i < k; i++) mx = fmaxf(mx, row[sel[i]]);
    float denom = 0.0f;
    for (int i = 0; i < k; i++) denom += expf(row[sel[i]] - mx);
    denom = fmaxf(denom, F32_EPSILON);
    for (int i = 0; i < k; i++) sw[i] = expf(row[sel[i]] - mx) / denom;
    const int n = keep_max > 0 ? ser_reduce_row(sel, sw, k, keep_max, min_w) : k;
    for (int i = 0; i < k; i++) {
        ids[(size_t)r * k + i] = i < n ? sel[i] : -1;
        weights[(size_t)r * k + i] = i < n ? sw[i] : 0.0f;
    }
}

hipError_t moe_route_launch(const float* logits, size_t rows, size_t n_experts, size_t top_k,
                            int32_t* ids, float* weights, hipStream_t s, size_t max_active, float min_weight) {
    if (rows == 0) return hipSuccess;
    // keep_max in [1, top_k] when reducing (a "no cap" max_active such as
    // usize::MAX keeps every slot), 0 = route only
    const int keep = max_active == 0 ? 0 : (int)(max_active < top_k ? max_active : top_k);
    hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, s, logits,
                       (int)rows, (int)n_experts, (int)top_k, keep, min_weight, ids, weights);
    return hipGetLastError();
}

// reduce_expert_assignments on given rows x k slots (in place allowed)
__global__ __launch_bounds__(64) void moe_reduce_kernel(const int32_t* ids, const float* weights, int rows, int k,
                                                        int keep_max, float min_w, int32_t* out_ids,
                                                        float* out_weights) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    int ci[MOE_MAX_TOPK];
    float cw[MOE_MAX_TOPK];
    for (int i = 0; i < k; i++) {
        ci[i] = ids[(size_t)r * k + i];
        cw[i] = weights[(size_t)r * k + i];
    }
    const int n = ser_reduce_row(ci, cw, k, keep_max, min_w);
    for (int i = 0; i < k; i++) {
        out_ids[(size_t)r * k + i] = i < n ? ci[i] : -1;
        out_weights[(size_t)r * k + i] = i < n ? cw[i] : 0.0f;
    }
}

hipError_t moe_reduce_launch(const int32_t* ids, const float* weights, size_t rows, size_t k, size_t max_active,
                             float min_weight, int32_t* out_ids, float* out_weights, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    // keep_max = clamp(max_active, 1, k): a "no cap" value keeps every slot
    const int keep = max_active == 0 ? 1 : (int)(max_active < k ? max_active : k);
    hipLaunchKernelGGL(moe_reduce_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, s, ids, weights,
                       (int)rows, (int)k, keep, min_weight, out_ids, out_weights);
    return hipGetLastError();
}

// batch_by_expert (moe_fused.rs:196-223): one workgroup builds the CSR
// grouping.  Assignments are visited in ascending (token, routing slot)
// order; ids outside [0, n_experts) are skipped (batches.get_mut -> None).
// Each assignment's place inside its expert is its rank among the earlier
// assignments of that expert, so the fill is parallel and deterministic.
// rowpos[t*k+i] is the grouped row of assignment (t, i), or -1.
constexpr int MOE_GROUP_THREADS = 256;

__global__ __launch_bounds__(MOE_GROUP_THREADS) void moe_group_kernel(const int32_t* __restrict__ ids,
                                                                      const float* __restrict__ weights, int rows,
                                                                      int k, int ne, int32_t* __restrict__ offsets,
                                                                      int32_t* __restrict__ tokens,
                                                                      float* __restrict__ wts,
                                                                      int32_t* __restrict__ rowpos) {
    __shared__ int cnt[MOE_MAX_EXPERTS + 1];
    __shared__ int cid[MOE_GROUP_THREADS];
    const int tid = threadIdx.x;
    for (int e = tid; e <= ne; e += MOE_GROUP_THREADS) cnt[e] = 0;
    __syncthreads();
    const int n = rows * k;
    for (int a = tid; a < n; a += MOE_GROUP_THREADS) {
        const int e = ids[a];
        if (e >= 0 && e < ne) atomicAdd(&cnt[e + 1], 1);
    }
    __syncthreads();
    // cnt[e] <- first row of expert e: one wave scans four entries per lane
    if (tid < 64) {
        int v[4], run = 0;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = 4 * tid + i + 1;
            v[i] = idx <= ne ? cnt[idx] : 0;
            run += v[i];
        }
        int inc = run;
        #pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(inc, o);
            if (tid >= o) inc += t;
        }
        int p = inc - run;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = 4 * tid + i + 1;
            p += v[i];
            if (idx <= ne) cnt[idx] = p;
        }
    }
    __syncthreads();
    for (int e = tid; e <= ne; e += MOE_GROUP_THREADS) offsets[e] = cnt[e];
    const int total = cnt[ne];
    for (int c0 = 0; c0 < n; c0 += MOE_GROUP_THREADS) {
        const int a = c0 + tid;
        int e = a < n ? ids[a] : -1;
        if (e >= ne) e = -1;
        cid[tid] = e < 0 ? -1 : e;
        __syncthreads();
        if (e >= 0) {
            int r = 0;
            for (int j = 0; j < tid; j++) r += cid[j] == e;
            const int pos = cnt[e] + r;
            tokens[pos] = a / k;
            wts[pos] = weights[a];
            rowpos[a] = pos;
        } else if (a < n) {
            rowpos[a] = -1;
        }
        __syncthreads();
        if (e >= 0) atomicAdd(&cnt[e], 1);
        __syncthreads();
    }
    // rows past the last assignment (skipped ids) point at token 0, so that
    // consumers may process all rows * k rows without knowing the count
    for (int p = total + tid; p < n; p += MOE_GROUP_THREADS) {
        tokens[p] = 0;
        wts[p] = 0.0f;
    }
}

hipError_t moe_group_launch(const int32_t* ids, const float* weights, size_t rows, size_t top_k,
                            size_t n_experts, int32_t* offsets, int32_t* tokens, float* wts,
                            int32_t* rowpos, hipStream_t s) {
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(MOE_GROUP_THREADS), 0, s, ids, weights, (int)rows, (int)top_k,
                       (int)n_experts, offsets, tokens, wts, rowpos);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void moe_gather_kernel(const float4* __restrict__ x, const int32_t* __restrict__ tokens,
                                                         int n_assign, int h4, float4* __restrict__ xg) {
    const int i = blockIdx.y;
    const int t = tokens[i];
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < h4; c += gridDim.x * blockDim.x)
        xg[(size_t)i * h4 + c] = x[(size_t)t * h4 + c];
}

hipError_t moe_gather_launch(const float* x, const int32_t* tokens, size_t n_assign, size_t hidden,
                             float* xg, hipStream_t s) {
    if (n_assign == 0) return hipSuccess;
    const int h4 = (int)(hidden / 4);
    const unsigned gx = (unsigned)((h4 + 255) / 256 < 64 ? (h4 + 255) / 256 : 64);
    hipLaunchKernelGGL(moe_gather_kernel, dim3(gx, (unsigned)n_assign), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(x), tokens, (int)n_assign, h4,
                       reinterpret_cast<float4*>(xg));
    return hipGetLastError();
}

// Silu x / (1 + exp(-x)) (ops.rs:191-211), then the gate*up product
// (moe_fused.rs:61-66).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     size_t n, float* __restrict__ h) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float gv = g[i];
        const float a = gv / (1.0f + expf(-gv));
        h[i] = a * u[i];
    }
}

hipError_t swiglu_launch(const float* g, const float* u, size_t n, float* h, hipStream_t s) {
    if (n == 0) return hipSuccess;
    size_t grid = (n + 255) / 256;
    if (grid > 16384) grid = 16384;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)grid), dim3(256), 0, s, g, u, n, h);
    return hipGetLastError();
}

// moe_group_kernel and quantize_q8_k_gather_kernel in one launch, for at
// most MOE_FUSED_MAX assignments: every workgroup groups the assignments
// itself in LDS (counts, prefix, then each 256-assignment chunk ranked per
// wave with ballots: one round per distinct expert in the wave), so it knows
// the token of each grouped row it quantizes; workgroup 0 also writes the
// offsets / tokens / wts / rowpos arrays that the later kernels read.  The
// positions are the ones moe_group_kernel assigns (rank among the earlier
// assignments of the same expert).
__global__ __launch_bounds__(256) void moe_group_gather_q8k_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ weights, int rows, int k, int ne,
    const float* __restrict__ x, int nbr, uint8_t* __restrict__ out, int nb, int32_t* __restrict__ offsets,
    int32_t* __restrict__ tokens, float* __restrict__ wts, int32_t* __restrict__ rowpos) {
    __shared__ int start[MOE_MAX_EXPERTS + 1];
    __shared__ int wcnt[4][MOE_MAX_EXPERTS];
    __shared__ int tokl[MOE_FUSED_MAX];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool writer = blockIdx.x == 0;
    const int n = rows * k;
    for (int e = tid; e <= ne; e += 256) start[e] = 0;
    for (int i = tid; i < 4 * MOE_MAX_EXPERTS; i += 256) (&wcnt[0][0])[i] = 0;
    __syncthreads();
    for (int a = tid; a < n; a += 256) {
        const int e = ids[a];
        if (e >= 0 && e < ne) atomicAdd(&start[e + 1], 1);
    }
    __syncthreads();
    // exclusive prefix: start[e] <- first grouped row of expert e (one wave, four entries per lane)
    if (tid < 64) {
        int v[4], run = 0;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = 4 * tid + i + 1;
            v[i] = idx <= ne ? start[idx] : 0;
            run += v[i];
        }
        int inc = run;
        #pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(inc, o);
            if (tid >= o) inc += t;
        }
        int p = inc - run;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const int idx = 4 * tid + i + 1;
            p += v[i];
            if (idx <= ne) start[idx] = p;
        }
    }
    __syncthreads();
    if (writer)
        for (int e = tid; e <= ne; e += 256) offsets[e] = start[e];
    const int total = start[ne];
    for (int c0 = 0; c0 < n; c0 += 256) {
        const int a = c0 + tid;
        int e = a < n ? ids[a] : -1;
        if (e >= ne) e = -1;
        int rank = 0;
        uint64_t todo = __ballot(e >= 0);
        while (todo) {   // wave-uniform: one round per distinct expert in the wave
            const int leader = __ffsll((unsigned long long)todo) - 1;
            const int el = __builtin_amdgcn_readlane(e, leader);   // leader is wave-uniform
            const uint64_t m = __ballot(e == el);
            if (e == el) rank = __popcll(m & ((1ull << lane) - 1ull));
            if (lane == leader) wcnt[wave][el] = __popcll(m);
            todo &= ~m;
        }
        __syncthreads();
        if (e >= 0) {
            int pos = start[e] + rank;
            for (int w = 0; w < wave; w++) pos += wcnt[w][e];
            tokl[pos] = a;
            if (writer) {
                tokens[pos] = a / k;
                wts[pos] = weights[a];
                rowpos[a] = pos;
            }
        } else if (a < n && writer) {
            rowpos[a] = -1;
        }
        __syncthreads();
        for (int e2 = tid; e2 < ne; e2 += 256) {
            start[e2] += wcnt[0][e2] + wcnt[1][e2] + wcnt[2][e2] + wcnt[3][e2];
            wcnt[0][e2] = wcnt[1][e2] = wcnt[2][e2] = wcnt[3][e2] = 0;
        }
        __syncthreads();
    }
    // rows past the last assignment (skipped ids) point at token 0
    if (writer)
        for (int p = total + tid; p < n; p += 256) {
            tokens[p] = 0;
            wts[p] = 0.0f;
        }
    const int b = blockIdx.x * 4 + wave;
    if (b >= nb) return;   // whole waves
    const int i = b / nbr, cb = b - i * nbr;
    const int tok = i < total ? tokl[i] / k : 0;
    const float4 v = reinterpret_cast<const float4*>(x + ((size_t)tok * nbr + cb) * 256)[lane];
    const float vv[4] = {v.x, v.y, v.z, v.w};
    q8_k_block(vv, lane, out + (size_t)b * 292);
}

// BARQ_MOE_FUSED_GROUP=0 keeps grouping and gather-quantize in two launches
int moe_fused_group_enabled() { return tuning_env(TUNE_MOE_FUSED_GROUP, 1); }

hipError_t moe_group_gather_q8k_launch(const int32_t* ids, const float* weights, size_t rows, size_t top_k,
                                       size_t n_experts, const float* x, size_t hidden, void* out, int32_t* offsets,
                                       int32_t* tokens, float* wts, int32_t* rowpos, hipStream_t s) {
    const size_t n = rows * top_k, nbr = hidden / 256, nb = n * nbr;
    if (n == 0 || n > (size_t)MOE_FUSED_MAX || n_experts == 0 || n_experts > (size_t)MOE_MAX_EXPERTS ||
        hidden % 256 != 0 || nb > (size_t)INT32_MAX)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_group_gather_q8k_kernel, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, ids, weights,
                       (int)rows, (int)top_k, (int)n_experts, x, (int)nbr, static_cast<uint8_t*>(out), (int)nb, offsets,
                       tokens, wts, rowpos);
    return hipGetLastError();
}

// dispatch_experts accumulation (moe_fused.rs:292-299): per token, expert
// contributions are added in ascending expert id order (the order batches
// are processed), each as out += y * w with the product rounded first.
__global__ __launch_bounds__(256) void moe_scatter_kernel(const float* __restrict__ yg,
                                                          const int32_t* __restrict__ ids,
                                                          const float* __restrict__ weights,
                                                          const int32_t* __restrict__ rowpos, int k,
                                                          int hidden, float* __restrict__ out, int parts,
                                                          size_t part_stride) {
    const int t = blockIdx.y;
    const int32_t* tid = ids + (size_t)t * k;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < hidden; c += gridDim.x * blockDim.x) {
        float acc = 0.0f;
        // ascending expert id; equal ids keep routing order (stable)
        int last_e = -1, last_i = -1;
        for (int n = 0; n < k; n++) {
            int be = 0x7fffffff, bi = -1;
            for (int i = 0; i < k; i++) {
                const int e = tid[i];
                if (rowpos[(size_t)t * k + i] < 0) continue;
                const bool after = e > last_e || (e == last_e && i > last_i);
                if (after && (e < be || (e == be && i < bi))) { be = e; bi = i; }
            }
            if (bi < 0) break;
            const size_t at = (size_t)rowpos[(size_t)t * k + bi] * hidden + c;
            float yv = yg[at];
            for (int q = 1; q < parts; q++) yv += yg[at + q * part_stride];
            const float p = yv * weights[(size_t)t * k + bi];
            acc = acc + p;
            last_e = be; last_i = bi;
        }
        out[(size_t)t * hidden + c] = acc;
    }
}

hipError_t moe_scatter_launch(const float* yg, const int32_t* ids, const float* weights,
                              const int32_t* rowpos, size_t rows, size_t top_k, size_t hidden,
                              float* out, hipStream_t s, int parts, size_t part_stride) {
    if (rows == 0) return hipSuccess;
    const unsigned gx = (unsigned)((hidden + 255) / 256 < 64 ? (hidden + 255) / 256 : 64);
    hipLaunchKernelGGL(moe_scatter_kernel, dim3(gx, (unsigned)rows), dim3(256), 0, s, yg, ids, weights,
                       rowpos, (int)top_k, (int)hidden, out, parts, part_stride);
    return hipGetLastError();
}

}  // namespace barq
