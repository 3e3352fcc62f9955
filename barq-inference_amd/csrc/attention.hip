// Attention on device: RoPE, head transpose, the KV-cache copy and the
// attention kernel of a LlamaTransformer layer.
//
//   apply_rope      models/src/transformer.rs:514-562 (Interleaved / SplitHalf)
//   transpose_heads models/src/transformer.rs:598-611
//   compute_attention models/src/transformer.rs:301-374:
//     kv_h = h * n_head_kv / n_head                                (:318)
//     score_j = (q . K[j]) * (1 / sqrt(head_dim))                  (:311,327-335)
//     score_j = -inf for j >= start_pos + i + 1                    (:337-342)
//     p = softmax(score); out[i, h, :] = sum_j p_j V[j, :]        (:344-356)
//
// Layouts (the reference's): q is [n_head, q_len, head_dim] (apply_rope's
// output); the cache holds, per layer and kv head, positions x head_dim
// contiguous (KVCache, models/src/context.rs:245-340), here preallocated to
// max_size positions; out is [q_len, n_head, head_dim].
//
// The attention kernel streams K and V rows from HBM once per kv head for all
// the query heads that share it (GQA), split over the positions so that
// enough workgroups run: a row of head_dim floats is read by head_dim / 8
// lanes (two float4 each), every lane keeps its own online-softmax state
// (running max, sum, and its 8 output dims) for each query head, and the
// states are merged in LDS and then across splits.  Exponentials are base 2
// on scores pre-scaled by log2(e) (v_exp_f32), so the weights agree with the
// reference's expf to a few ulp, not bit for bit; sums run in a different
// order from the reference's sequential ones.
#include "common.hpp"
#include "launch.hpp"
#include "mfma_common.hpp"
#include "q8k_block.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <functional>
#include <queue>
#include <utility>
#include <vector>

namespace barq {

// ---- RoPE / transpose ----------------------------------------------------------
// One thread per (position, head, pair).  out[h * out_head_stride + p * hd + ...]
// so that the rotated rows can go straight into a cache.
template <int LAYOUT>
__global__ __launch_bounds__(256)
void rope_kernel(const float* __restrict__ x, float* __restrict__ out, int seq, int heads, int hd, long long start_pos,
                 float freq_scale, const float* __restrict__ inv_freq, size_t out_head_stride) {
    const int half = hd / 2;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)seq * heads * half) return;
    const int i = (int)(t % half);
    const size_t ph = t / half;
    const int h = (int)(ph % heads), p = (int)(ph / heads);
    // (abs_pos as f32 * rope_freq_scale) * rope_inv_freq[i]
    const float angle = ((float)(start_pos + p) * freq_scale) * inv_freq[i];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    const float* src = x + ((size_t)p * heads + h) * hd;
    float* dst = out + (size_t)h * out_head_stride + (size_t)p * hd;
    const int i0 = LAYOUT == ROPE_INTERLEAVED ? 2 * i : i;
    const int i1 = LAYOUT == ROPE_INTERLEAVED ? 2 * i + 1 : i + half;
    const float x0 = src[i0], x1 = src[i1];
    dst[i0] = x0 * cs - x1 * sn;
    dst[i1] = x0 * sn + x1 * cs;
}

__global__ __launch_bounds__(256)
void transpose_heads_kernel(const float* __restrict__ x, float* __restrict__ out, int seq, int heads, int hd,
                            size_t out_head_stride) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)seq * heads * hd) return;
    const int d = (int)(t % hd);
    const size_t ph = t / hd;
    const int h = (int)(ph % heads), p = (int)(ph / heads);
    out[(size_t)h * out_head_stride + (size_t)p * hd + d] = x[t];
}

// RoPE of q, RoPE of k into the cache and the copy of v into the cache in
// one launch (apply_rope twice and transpose_heads, transformer.rs:222-245
// and 514-611): slot s of a position is query head s (s < n_q), kv head
// s - n_q of k, or of v; one thread per pair of dims.  The angles and the
// rotation are rope_kernel's, so the results are the same bits.
template <int LAYOUT>
__global__ __launch_bounds__(256)
void rope_qkv_kernel(const float* __restrict__ qx, const float* __restrict__ kx, const float* __restrict__ vx,
                     float* __restrict__ q_out, float* __restrict__ k_out, float* __restrict__ v_out, int seq, int n_q,
                     int n_kv, int hd, long long start_pos, float freq_scale, const float* __restrict__ inv_freq,
                     size_t cache_head_stride) {
    const int half = hd / 2, slots = n_q + 2 * n_kv;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)seq * slots * half) return;
    const int i = (int)(t % half);
    const size_t ps = t / half;
    const int sl = (int)(ps % slots), p = (int)(ps / slots);
    if (sl >= n_q + n_kv) {   // v: transpose_heads into the cache
        const int h = sl - n_q - n_kv;
        const float* src = vx + ((size_t)p * n_kv + h) * hd;
        float* dst = v_out + (size_t)h * cache_head_stride + (size_t)p * hd;
        dst[2 * i] = src[2 * i];
        dst[2 * i + 1] = src[2 * i + 1];
        return;
    }
    const bool is_q = sl < n_q;
    const int h = is_q ? sl : sl - n_q, heads = is_q ? n_q : n_kv;
    const float angle = ((float)(start_pos + p) * freq_scale) * inv_freq[i];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    const float* src = (is_q ? qx : kx) + ((size_t)p * heads + h) * hd;
    float* dst = is_q ? q_out + ((size_t)h * seq + p) * hd : k_out + (size_t)h * cache_head_stride + (size_t)p * hd;
    const int i0 = LAYOUT == ROPE_INTERLEAVED ? 2 * i : i;
    const int i1 = LAYOUT == ROPE_INTERLEAVED ? 2 * i + 1 : i + half;
    const float x0 = src[i0], x1 = src[i1];
    dst[i0] = x0 * cs - x1 * sn;
    dst[i1] = x0 * sn + x1 * cs;
}

hipError_t rope_qkv_launch(int layout, const float* qx, const float* kx, const float* vx, float* q_out, float* k_out,
                           float* v_out, size_t seq, size_t n_q, size_t n_kv, size_t hd, size_t start_pos,
                           float freq_scale, const float* inv_freq, size_t cache_head_stride, hipStream_t s) {
    const size_t n = seq * (n_q + 2 * n_kv) * (hd / 2);
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (layout == ROPE_INTERLEAVED)
        hipLaunchKernelGGL(rope_qkv_kernel<ROPE_INTERLEAVED>, dim3(grid), dim3(256), 0, s, qx, kx, vx, q_out, k_out,
                           v_out, (int)seq, (int)n_q, (int)n_kv, (int)hd, (long long)start_pos, freq_scale, inv_freq,
                           cache_head_stride);
    else
        hipLaunchKernelGGL(rope_qkv_kernel<ROPE_SPLIT_HALF>, dim3(grid), dim3(256), 0, s, qx, kx, vx, q_out, k_out,
                           v_out, (int)seq, (int)n_q, (int)n_kv, (int)hd, (long long)start_pos, freq_scale, inv_freq,
                           cache_head_stride);
    return hipGetLastError();
}

hipError_t rope_launch(int layout, const float* x, float* out, size_t seq, size_t heads, size_t hd, size_t start_pos,
                       float freq_scale, const float* inv_freq, size_t out_head_stride, hipStream_t s) {
    const size_t n = seq * heads * (hd / 2);
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)((n + 255) / 256);
    if (layout == ROPE_INTERLEAVED)
        hipLaunchKernelGGL(rope_kernel<ROPE_INTERLEAVED>, dim3(grid), dim3(256), 0, s, x, out, (int)seq, (int)heads,
                           (int)hd, (long long)start_pos, freq_scale, inv_freq, out_head_stride);
    else
        hipLaunchKernelGGL(rope_kernel<ROPE_SPLIT_HALF>, dim3(grid), dim3(256), 0, s, x, out, (int)seq, (int)heads,
                           (int)hd, (long long)start_pos, freq_scale, inv_freq, out_head_stride);
    return hipGetLastError();
}

hipError_t transpose_heads_launch(const float* x, float* out, size_t seq, size_t heads, size_t hd,
                                  size_t out_head_stride, hipStream_t s) {
    const size_t n = seq * heads * hd;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(transpose_heads_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, out, (int)seq,
                       (int)heads, (int)hd, out_head_stride);
    return hipGetLastError();
}

// ---- attention -----------------------------------------------------------------
constexpr int ATT_THREADS = 256;
constexpr float LOG2E = 1.44269504088896340736f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// K/V rows are streamed once per call: loaded with the non-temporal hint
// (measured in one run: 55.1 -> 49.5 us at 32K positions, 14.1 -> 13.5 us at 4K),
// through a buffer descriptor over `bytes` bytes from `base`: reads at or past
// the limit return zeros and touch no memory.  Cache policy 2 is the
// non-temporal bit.
typedef float f32x4n __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kv_rows(const float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 kv_ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const f32x4n v = __builtin_bit_cast(f32x4n, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Partial state of one (query row, head, split): running max m (log2 units),
// sum l, then HD output sums.  Stored as HD + 2 floats.
//
// Grid: x = split, y = head group (kv head for G > 1; query head for G == 1),
// z = query row i.  The workgroup covers positions [split * chunk, ...) of
// the visible prefix [0, min(kv_len, start_pos + i + 1)).
template <int HD, int G>
__global__ __launch_bounds__(ATT_THREADS)
void attn_kernel(const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
                 size_t layer_off, size_t head_stride, int n_head, int n_head_kv, int q_len, int kv_len,
                 long long start_pos, int chunk, float score_scale, float* __restrict__ part, float* __restrict__ out) {
    constexpr int LPR = HD / 8;              // lanes per K/V row
    constexpr int R = ATT_THREADS / LPR;     // rows per pass
    static_assert(LPR == 8 || LPR == 16 || LPR == 32, "head_dim 64, 128 or 256");
    __shared__ float red_o[R][G][HD];
    __shared__ float red_ml[R][G][2];
    __shared__ float red_ms[G][2];

    const int t = threadIdx.x, c = t % LPR, r = t / LPR;
    const int split = blockIdx.x, grp = blockIdx.y, i = blockIdx.z, n_split = gridDim.x;
    const int hk = G > 1 ? grp : (int)((long long)grp * n_head_kv / n_head);
    const long long vis = start_pos + i + 1;
    const int valid = (int)(vis < kv_len ? vis : kv_len);
    const int j0 = split * chunk, j1 = min(valid, j0 + chunk);

    // query rows of the group's heads (pre-scaled: score * log2e is the exponent)
    float qv[G][8];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        const int h = G > 1 ? grp * G + g : grp;
        const float4* qp = reinterpret_cast<const float4*>(q + ((size_t)h * q_len + i) * HD);
        const float4 a = qp[c], b = qp[c + LPR];
        qv[g][0] = a.x; qv[g][1] = a.y; qv[g][2] = a.z; qv[g][3] = a.w;
        qv[g][4] = b.x; qv[g][5] = b.y; qv[g][6] = b.z; qv[g][7] = b.w;
    }
    float m[G], l[G], o[G][8];
    #pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
        #pragma unroll
        for (int d = 0; d < 8; d++) o[g][d] = 0.0f;
    }

    // lane c of a row holds dims 4c..4c+3 and 4(c+LPR)..: each load
    // instruction reads whole contiguous half-rows
    const float* kh = kc + layer_off + (size_t)hk * head_stride;
    const float* vh = vc + layer_off + (size_t)hk * head_stride;
    // P passes of R rows form a block; the next block's rows are loaded
    // while this block's are scored, so every lane keeps K/V loads in
    // flight.  The softmax state moves once per block: all P scores first,
    // then one rescale of the running sums by the block's new maximum.
    constexpr int P = G <= 4 ? 2 : 1;
    struct Rows {
        float4 k[P][2], v[P][2];
    };
    // Rows are read through buffer descriptors limited to [j0, j1): a row
    // past the range reads as zeros without a memory access (its score is
    // masked and its weight is 0), so a block's loads need no condition.
    const __amdgpu_buffer_rsrc_t kr = kv_rows(kh + (size_t)j0 * HD, (uint32_t)(j1 - j0) * (HD * 4));
    const __amdgpu_buffer_rsrc_t vr = kv_rows(vh + (size_t)j0 * HD, (uint32_t)(j1 - j0) * (HD * 4));
    auto load = [&](Rows& b, int blk) {
        #pragma unroll
        for (int p = 0; p < P; p++) {
            const uint32_t off = (uint32_t)(blk - j0 + p * R + r) * (HD * 4) + (uint32_t)c * 16;
            b.k[p][0] = kv_ld(kr, off); b.k[p][1] = kv_ld(kr, off + LPR * 16);
            b.v[p][0] = kv_ld(vr, off); b.v[p][1] = kv_ld(vr, off + LPR * 16);
        }
    };
    auto block = [&](const Rows& b, int blk) {
        #pragma unroll
        for (int g = 0; g < G; g++) {
            float sc[P];
            float bm = -INFINITY;
            #pragma unroll
            for (int p = 0; p < P; p++) {
                const float4 k0 = b.k[p][0], k1 = b.k[p][1];
                float dot = qv[g][0] * k0.x;
                dot = __builtin_fmaf(qv[g][1], k0.y, dot);
                dot = __builtin_fmaf(qv[g][2], k0.z, dot);
                dot = __builtin_fmaf(qv[g][3], k0.w, dot);
                dot = __builtin_fmaf(qv[g][4], k1.x, dot);
                dot = __builtin_fmaf(qv[g][5], k1.y, dot);
                dot = __builtin_fmaf(qv[g][6], k1.z, dot);
                dot = __builtin_fmaf(qv[g][7], k1.w, dot);
                dot = group_sum<LPR>(dot);
                // (q . k) / sqrt(hd) * log2(e); rows past the range do not count
                sc[p] = blk + p * R + r < j1 ? dot * score_scale : -INFINITY;
                bm = fmaxf(bm, sc[p]);
            }
            // No branch on a block without live rows: a branch around the
            // V products lets the compiler's wait insertion assume the V
            // loads may still be in flight at the next block's loads into
            // the same registers, and it waits for every load there.  With
            // no live row so far (mn = -inf) the reference point 0 gives
            // corr = e = 0; with no live row in the block but some before,
            // corr = exp2(0) = 1 and e = 0, leaving the state as it was.
            const float mn = fmaxf(m[g], bm);
            const float ref = mn == -INFINITY ? 0.0f : mn;
            const float corr = fast_exp2(m[g] - ref);  // 0 while m is -inf
            m[g] = mn;
            l[g] *= corr;
            #pragma unroll
            for (int d = 0; d < 8; d++) o[g][d] *= corr;
            #pragma unroll
            for (int p = 0; p < P; p++) {
                const float e = fast_exp2(sc[p] - ref);  // 0 for rows past the range
                const float4 v0 = b.v[p][0], v1 = b.v[p][1];
                l[g] += e;
                o[g][0] = __builtin_fmaf(e, v0.x, o[g][0]);
                o[g][1] = __builtin_fmaf(e, v0.y, o[g][1]);
                o[g][2] = __builtin_fmaf(e, v0.z, o[g][2]);
                o[g][3] = __builtin_fmaf(e, v0.w, o[g][3]);
                o[g][4] = __builtin_fmaf(e, v1.x, o[g][4]);
                o[g][5] = __builtin_fmaf(e, v1.y, o[g][5]);
                o[g][6] = __builtin_fmaf(e, v1.z, o[g][6]);
                o[g][7] = __builtin_fmaf(e, v1.w, o[g][7]);
            }
        }
    };
    if (j0 < j1) {
        // NB row buffers used in turn (no register copies between blocks),
        // each refilled NB blocks ahead as soon as it has been scored.  The
        // loads carry no condition (past the range they read zeros), so
        // every block waits for its own loads only: with a conditional
        // issue the compiler's wait counts cover both paths, and each block
        // would also wait for the loads issued after it.
        // Scheduling barriers keep the loads where they are written (the
        // scheduler otherwise gathers all loads after the blocks).
        constexpr int NB = 2;
        Rows rows[NB];
        #pragma unroll
        for (int q = 0; q < NB; q++) {
            load(rows[q], j0 + q * R * P);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int blk = j0; blk < j1; blk += NB * R * P) {
            #pragma unroll
            for (int q = 0; q < NB; q++) {
                __builtin_amdgcn_sched_barrier(0);
                block(rows[q], blk + q * R * P);
                __builtin_amdgcn_sched_barrier(0);
                load(rows[q], blk + (q + NB) * R * P);
            }
        }
    }

    // merge the R row states of the workgroup
    #pragma unroll
    for (int g = 0; g < G; g++) {
        #pragma unroll
        for (int d = 0; d < 4; d++) {
            red_o[r][g][4 * c + d] = o[g][d];
            red_o[r][g][4 * (c + LPR) + d] = o[g][4 + d];
        }
        if (c == 0) {
            red_ml[r][g][0] = m[g];
            red_ml[r][g][1] = l[g];
        }
    }
    __syncthreads();
    // each row state's weight exp2(m_rr - M) once per (row, head), in place
    // of its max (then the same sums in the same order for every dim): one
    // thread per (head, row state), each head's R states an aligned group of
    // lanes (G * R <= ATT_THREADS)
    static_assert(G * R <= ATT_THREADS && R <= 32, "one thread per row state");
    if (t < G * R) {
        const int g = t / R, rr = t % R;
        const float mr = red_ml[rr][g][0];
        const float M = group_max<R>(mr);
        const float w = M == -INFINITY ? 0.0f : fast_exp2(mr - M);
        const float L = group_sum<R>(red_ml[rr][g][1] * w);
        red_ml[rr][g][0] = w;
        if (rr == 0) {
            red_ms[g][0] = M;
            red_ms[g][1] = L;
        }
    }
    __syncthreads();
    for (int e = t; e < G * HD; e += ATT_THREADS) {
        const int g = e / HD, d = e % HD;
        const float M = red_ms[g][0], L = red_ms[g][1];
        float O = 0.0f;
        if (M != -INFINITY) {
            #pragma unroll
            for (int rr = 0; rr < R; rr++) O = __builtin_fmaf(red_o[rr][g][d], red_ml[rr][g][0], O);
        }
        const int h = G > 1 ? grp * G + g : grp;
        if (n_split == 1) {
            out[((size_t)i * n_head + h) * HD + d] = O / L;
        } else {
            float* pp = part + (((size_t)i * n_head + h) * n_split + split) * (HD + 2);
            pp[2 + d] = O;
            if (d == 0) {
                pp[0] = M;
                pp[1] = L;
            }
        }
    }
}

constexpr int ATT_MAX_SPLIT = 1024;

// One output head: out value of dim t (t < HD) from the n_split partial
// states at pp, by NT threads t = 0 .. NT - 1 (all of them call it: it
// synchronises the workgroup).  The split maxima and weights are spread over
// the threads; the output sums run over SUB = 1024 / HD subsets of the splits
// (split s in subset s % SUB, in increasing order), then are added in LDS in
// subset order.  With NT < 1024 each thread runs 1024 / NT subsets one after
// another, so the sums and their order do not depend on NT: the Q8_K merge
// (heads side by side) quantizes exactly the f32 merge's values.
template <int HD>
struct CombineLds {
    float w[ATT_MAX_SPLIT];
    float red[1024 / HD][HD];
    float wred[2][1024 / 64];
};

template <int HD, int NT>
__device__ __forceinline__ float attn_combine_head(const float* __restrict__ pp, int n_split, CombineLds<HD>& sm,
                                                   int t) {
    constexpr int NWV = NT / 64, SUB = 1024 / HD, K = 1024 / NT, STEP = NT / HD, PRE = 8;
    static_assert(NT % HD == 0 && 1024 % NT == 0, "threads per head");
    const int lane = t & 63, wave = t >> 6;
    const int sub = t / HD, d = t % HD;   // subsets sub + STEP j, j < K
    // every load of the first PRE rounds is issued before any reduction
    float ov[K][PRE];
    #pragma unroll
    for (int j = 0; j < K; j++)
        #pragma unroll
        for (int u = 0; u < PRE; u++) {
            const int s = sub + STEP * j + SUB * u;
            ov[j][u] = s < n_split ? pp[(size_t)s * (HD + 2) + 2 + d] : 0.0f;
        }
    // the maximum and sum of the splits t + NT j (j < K), loaded with the
    // output sums above (n_split <= ATT_MAX_SPLIT = 1024, so these are all of
    // this thread's splits): no load waits once the reductions start
    static_assert(ATT_MAX_SPLIT <= 1024, "one split per virtual lane");
    float Msj[K], Lsj[K];
    #pragma unroll
    for (int j = 0; j < K; j++) {
        const int s = t + NT * j;
        Msj[j] = s < n_split ? pp[(size_t)s * (HD + 2)] : -INFINITY;
        Lsj[j] = s < n_split ? pp[(size_t)s * (HD + 2) + 1] : 0.0f;
    }
    float M = Msj[0];
    #pragma unroll
    for (int j = 1; j < K; j++) M = fmaxf(M, Msj[j]);
    M = wave_max_all(M);
    if (lane == 0) sm.wred[0][wave] = M;
    __syncthreads();
    M = sm.wred[0][0];
    #pragma unroll
    for (int u = 1; u < NWV; u++) M = fmaxf(M, sm.wred[0][u]);
    // The denominator in the 1024-thread merge's order whatever NT is: thread
    // t plays the 1024 lanes t + NT j (j < K), each holding its one split; a
    // reduction per 64 of those lanes (a real wave holds 64 consecutive ones);
    // then the 16 wave partials in lane order.  So the Q8_K merge's rows are
    // the f32 merge's to the bit.
    float Lj[K];
    #pragma unroll
    for (int j = 0; j < K; j++) {
        const int s = t + NT * j;
        float L = 0.0f;
        if (s < n_split) {
            const float ws = Msj[j] == -INFINITY ? 0.0f : fast_exp2(Msj[j] - M);
            sm.w[s] = ws;
            L = Lsj[j] * ws;
        }
        L = wave_sum_all(L);
        Lj[j] = L;
    }
    if (lane == 0) {
        #pragma unroll
        for (int j = 0; j < K; j++) sm.wred[1][NWV * j + wave] = Lj[j];
    }
    __syncthreads();
    float L = sm.wred[1][0];
    #pragma unroll
    for (int u = 1; u < 1024 / 64; u++) L += sm.wred[1][u];
    #pragma unroll
    for (int j = 0; j < K; j++) {
        const int sj = sub + STEP * j;
        float O = 0.0f;
        #pragma unroll
        for (int u = 0; u < PRE; u++) {
            const int s = sj + SUB * u;
            if (s < n_split) O = __builtin_fmaf(ov[j][u], sm.w[s], O);
        }
        for (int s = sj + SUB * PRE; s < n_split; s += SUB) O = __builtin_fmaf(pp[(size_t)s * (HD + 2) + 2 + d], sm.w[s], O);
        sm.red[sj][d] = O;
    }
    __syncthreads();
    float acc = 0.0f;
    if (t < HD) {
        acc = sm.red[0][t];
        #pragma unroll
        for (int u = 1; u < SUB; u++) acc += sm.red[u][t];
        acc = acc / L;
    }
    return acc;
}

// out[i, h, :] from the n_split partial states of (i, h): one workgroup of
// 1024 threads per (h, i).
template <int HD>
__global__ __launch_bounds__(1024)
void attn_combine_kernel(const float* __restrict__ part, int n_split, int n_head, float* __restrict__ out) {
    __shared__ CombineLds<HD> sm;
    const int h = blockIdx.x, i = blockIdx.y, t = threadIdx.x;
    const float v = attn_combine_head<HD, 1024>(part + ((size_t)i * n_head + h) * n_split * (HD + 2), n_split, sm, t);
    if (t < HD) out[((size_t)i * n_head + h) * HD + t] = v;
}

// The same merge with the output row written as Q8_K blocks (the o
// projection's activation): workgroup (b, i) merges the 256 / HD heads of
// block b of row i side by side (1024 / (256 / HD) threads each), then one
// wave quantizes the block (q8_k_block: the bytes quantize_q8_k_kernel
// writes for the same values).
template <int HD>
__global__ __launch_bounds__(1024)
void attn_combine_q8k_kernel(const float* __restrict__ part, int n_split, int n_head, uint8_t* __restrict__ out) {
    constexpr int NH = 256 / HD, NT = 1024 / NH;
    __shared__ CombineLds<HD> sm[NH];
    __shared__ __align__(16) float vals[256];
    const int b = blockIdx.x, i = blockIdx.y, t = threadIdx.x;
    const int hh = t / NT, tg = t % NT, h = b * NH + hh;
    const float v = attn_combine_head<HD, NT>(part + ((size_t)i * n_head + h) * n_split * (HD + 2), n_split, sm[hh], tg);
    if (tg < HD) vals[hh * HD + tg] = v;
    __syncthreads();
    if (t < 64) {
        const float4 v4 = reinterpret_cast<const float4*>(vals)[t];
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
        q8_k_block(vv, t, out + ((size_t)i * (n_head * HD / 256) + b) * Q8_K_BYTES);
    }
}

// Position blocks of 32 that query block qb sees (am_qblock's range).
__host__ __device__ __forceinline__ int am_qblock_blocks(int qb, int q_len, int kv_len, long long start_pos) {
    const int i_last = qb * 32 + 31 < q_len - 1 ? qb * 32 + 31 : q_len - 1;
    const long long vis_last = start_pos + i_last + 1;
    const int j_end = (int)(vis_last < kv_len ? vis_last : kv_len);
    return (j_end + 31) / 32;
}

// The merge for a few splits (the prompt kernel's): one thread per output
// value, 256 per workgroup (the 256 / HD heads of one Q8_K block of row i);
// Q8 writes the block's Q8_K bytes (q8_k_block) instead of the f32 values.
template <int HD, bool Q8>
__global__ __launch_bounds__(256)
void attn_combine_few_kernel(const float* __restrict__ part, int stride, int chunk, int n_head, int q_len, int kv_len,
                             long long start_pos, float* __restrict__ out, uint8_t* __restrict__ out_q8) {
    __shared__ __align__(16) float vals[256];
    const int b = blockIdx.x, i = blockIdx.y, t = threadIdx.x;
    const int h = b * (256 / HD) + t / HD, d = t % HD;
    // the pieces of row i's query block (attn_mfma_kernel's list)
    const int n_split = (am_qblock_blocks(i / 32, q_len, kv_len, start_pos) + chunk - 1) / chunk;
    const float* pp = part + ((size_t)i * n_head + h) * stride * (HD + 2);
    float M = -INFINITY;
    for (int sp = 0; sp < n_split; sp++) M = fmaxf(M, pp[(size_t)sp * (HD + 2)]);
    float L = 0.0f, O = 0.0f;
    for (int sp = 0; sp < n_split; sp++) {
        const float ms = pp[(size_t)sp * (HD + 2)];
        const float w = ms == -INFINITY ? 0.0f : fast_exp2(ms - M);
        L = __builtin_fmaf(pp[(size_t)sp * (HD + 2) + 1], w, L);
        O = __builtin_fmaf(pp[(size_t)sp * (HD + 2) + 2 + d], w, O);
    }
    const float v = O / L;
    if constexpr (!Q8) {
        out[((size_t)i * n_head + h) * HD + d] = v;
    } else {
        vals[t] = v;
        __syncthreads();
        if (t < 64) {
            const float4 v4 = reinterpret_cast<const float4*>(vals)[t];
            const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
            q8_k_block(vv, t, out_q8 + ((size_t)i * (n_head * HD / 256) + b) * Q8_K_BYTES);
        }
    }
}

bool attention_supported(size_t head_dim) { return head_dim == 64 || head_dim == 128 || head_dim == 256; }

// ---- prompt chunks on MFMA ----------------------------------------------------
// For q_len >= 32 (BARQ_ATTN_MFMA_MIN_Q) and head_dim 128 a workgroup covers
// 32 query rows of W query heads that share one kv head (one wave per head)
// and walks the visible positions in blocks of 32 with
// v_mfma_f32_32x32x2_f32 (f32 products and sums, as the VALU path):
//   S^T[kv, q] = K[kv, :] . Q[q, :]   A = K rows (lane c: row c, dims 64 g ..),
//                                     B = Q^T (lane c: query c, the same dims)
//   online softmax per query column: a lane holds 16 positions of its query,
//   the other 16 sit in lane c ^ 32
//   O^T[d, q] += V[kv, d] P[q, kv]    B = P^T straight from S^T's registers
//                                     (step s pairs positions 8(s/4) + s%4 and
//                                     +4, which lanes c and c + 32 hold as
//                                     register s); A = V^T with output row i of
//                                     block b standing for dim 4 i + b, so one
//                                     16-byte read per lane feeds the four blocks.
// Each block's K and V rows are copied once per workgroup into LDS by
// buffer->LDS loads one block ahead (two stages), in rows of 528 bytes (one
// pad piece: conflict-free fragment reads); rows at or past kv_len read as
// zero.  Exponentials are base 2 on pre-scaled scores, like the split kernel.
typedef float f32x16a __attribute__((ext_vector_type(16)));
constexpr int AM_RS = 528, AM_PIECES = 33, AM_BLK = 32 * AM_RS;
constexpr int AM_INSTR = (32 * AM_PIECES + 63) / 64;   // load instructions per K or V block (17)

// the buffer->LDS loads of one block (K and V) split over the workgroup's W waves
template <int W>
__device__ __forceinline__ void am_issue(uint8_t* stage, i32x4v kr, i32x4v vr, uint32_t soff, int wave, int l) {
    #pragma unroll
    for (int q = 0; q < (2 * AM_INSTR + W - 1) / W; q++) {
        const int idx = q * W + wave;
        if (idx < 2 * AM_INSTR) {
            const int kvsel = idx >= AM_INSTR, ii = idx - kvsel * AM_INSTR;
            const int p = ii * 64 + l, row = p / AM_PIECES, piece = p - row * AM_PIECES;
            if (p < 32 * AM_PIECES) {
                const uint32_t voff = (uint32_t)row * 512u + 16u * (uint32_t)(piece < 32 ? piece : 0);
                lds_load16(kvsel ? vr : kr, stage + kvsel * AM_BLK + 1024 * ii, voff, soff);
            }
        }
    }
}

// One 32-row query block qb of the workgroup's W heads.  With n_split > 1
// the workgroup takes split `split` of the block's visible positions (a
// contiguous run of 32-position blocks) and stores its partial state (max in
// log2 units, sum, unnormalised output) in the split kernel's layout for the
// merge kernels; an empty run stores (-inf, 0, 0).
template <int W>
__device__ __forceinline__ void am_qblock(uint8_t (&lds)[2][2 * AM_BLK], const float* __restrict__ q,
                                          const float* __restrict__ kc, const float* __restrict__ vc, size_t layer_off,
                                          size_t head_stride, int n_head, int n_head_kv, int q_len, int kv_len,
                                          long long start_pos, float score_scale, float* __restrict__ out, int qb,
                                          int chunk = 0, int split = 0, int stride = 1,
                                          float* __restrict__ part = nullptr, int grp = -1) {
    constexpr int HD = 128;
    const int l = threadIdx.x & 63, c = l & 31, g = l >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = (grp < 0 ? (int)blockIdx.y : grp) * W + wave;
    const int hk = (int)((long long)h * n_head_kv / n_head);   // the same for the W heads
    const int i0 = qb * 32, qi = i0 + c;
    const bool q_ok = qi < q_len;

    const float* kh = kc + layer_off + (size_t)hk * head_stride;
    const float* vh = vc + layer_off + (size_t)hk * head_stride;
    const i32x4v kr = make_rsrc4(kh, (uint32_t)kv_len * 512u);
    const i32x4v vr = make_rsrc4(vh, (uint32_t)kv_len * 512u);
    const int nblk_all = am_qblock_blocks(qb, q_len, kv_len, start_pos);
    // chunk > 0: this workgroup takes blocks [split, split + 1) * chunk of
    // the query block's range and writes a partial state
    const int b_lo = chunk > 0 ? min(split * chunk, nblk_all) : 0;
    const int nblk = chunk > 0 ? min(b_lo + chunk, nblk_all) : nblk_all;
    if (b_lo < nblk) am_issue<W>(lds[0], kr, vr, (uint32_t)b_lo * 32u * 512u, wave, l);

    float qv[64];
    {
        const float4* qp = reinterpret_cast<const float4*>(q + ((size_t)h * q_len + (q_ok ? qi : 0)) * HD + 64 * g);
        #pragma unroll
        for (int u = 0; u < 16; u++) {
            const float4 t = q_ok ? qp[u] : make_float4(0.f, 0.f, 0.f, 0.f);
            qv[4 * u] = t.x; qv[4 * u + 1] = t.y; qv[4 * u + 2] = t.z; qv[4 * u + 3] = t.w;
        }
    }
    const long long vis_q = start_pos + qi + 1;   // this lane's query sees positions below vis_q

    f32x16a o0 = {}, o1 = {}, o2 = {}, o3 = {};
    float m = -INFINITY, lsum = 0.0f;
    for (int b = b_lo; b < nblk; b++) {
        const int j0 = 32 * b;
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        __syncthreads();   // block b is in its stage; every wave is done with the other one
        if (b + 1 < nblk) am_issue<W>(lds[(b + 1 - b_lo) & 1], kr, vr, (uint32_t)(j0 + 32) * 512u, wave, l);
        const uint8_t* ks = lds[(b - b_lo) & 1];
        const uint8_t* vs = ks + AM_BLK;
        f32x16a sa = {}, sb = {};
        #pragma unroll
        for (int u = 0; u < 16; u++) {
            const float4 kk = *reinterpret_cast<const float4*>(ks + c * AM_RS + 256 * g + 16 * u);
            sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.x, qv[4 * u], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.y, qv[4 * u + 1], sb, 0, 0, 0);
            sa = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.z, qv[4 * u + 2], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.w, qv[4 * u + 3], sb, 0, 0, 0);
        }
        float sc[16];
        float bm = -INFINITY;
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            const int kv = j0 + 8 * (r >> 2) + 4 * g + (r & 3);
            const bool vis = kv < kv_len && kv < vis_q;
            sc[r] = vis ? (sa[r] + sb[r]) * score_scale : -INFINITY;
            bm = fmaxf(bm, sc[r]);
        }
        {   // with the other half-wave (one gfx950 half-wave swap, no LDS round trip)
            auto hb = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, bm), __builtin_bit_cast(int, bm), false, false);
            bm = fmaxf(__builtin_bit_cast(float, (int)hb[0]), __builtin_bit_cast(float, (int)hb[1]));
        }
        // Position 0 is visible to every query, so without a split mn is
        // finite from the first block on; a split that starts later can hold
        // blocks a query sees none of (mn = -inf): exponents then use 0 as
        // the reference, so they are 0 instead of NaN and the state stays
        // (-inf, 0, 0).
        const float mn = fmaxf(m, bm);
        const float mref = mn == -INFINITY ? 0.0f : mn;
        const float corr = fast_exp2(m - mref);   // 0 while m is -inf
        m = mn;
        float p[16];
        float rs = 0.0f;
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            p[r] = fast_exp2(sc[r] - mref);   // 0 for masked positions
            rs += p[r];
        }
        rs = swap32_add(rs, rs);   // + the other half-wave's, as v + v[lane ^ 32]
        lsum = lsum * corr + rs;
        o0 *= corr; o1 *= corr; o2 *= corr; o3 *= corr;
        #pragma unroll
        for (int st = 0; st < 16; st++) {
            const int kv = 8 * (st >> 2) + 4 * g + (st & 3);
            const float4 vv = *reinterpret_cast<const float4*>(vs + kv * AM_RS + 16 * c);
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, p[st], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, p[st], o1, 0, 0, 0);
            o2 = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, p[st], o2, 0, 0, 0);
            o3 = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, p[st], o3, 0, 0, 0);
        }
    }
    if (chunk > 0) {
        if (q_ok) {
            float* pp = part + (((size_t)qi * n_head + h) * stride + split) * (HD + 2);
            if (g == 0) {
                pp[0] = m;
                pp[1] = lsum;
            }
            #pragma unroll
            for (int r = 0; r < 16; r++) {
                const int i = 8 * (r >> 2) + 4 * g + (r & 3);
                float* d = pp + 2 + 4 * i;   // 8-byte aligned rows: two float2 stores
                *reinterpret_cast<float2*>(d) = make_float2(o0[r], o1[r]);
                *reinterpret_cast<float2*>(d + 2) = make_float2(o2[r], o3[r]);
            }
        }
        return;
    }
    if (q_ok) {
        float* op = out + ((size_t)qi * n_head + h) * HD;
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            const int i = 8 * (r >> 2) + 4 * g + (r & 3);
            *reinterpret_cast<float4*>(op + 4 * i) = make_float4(o0[r] / lsum, o1[r] / lsum, o2[r] / lsum, o3[r] / lsum);
        }
    }
}

// Causal prompts leave query block qb with qb + 1 position blocks (plus the
// cached prefix).  PAIR: workgroup x takes the long block nqb - 1 - x and
// then the short block x, so every workgroup has about the same work (used
// when the pairs alone fill the CUs).  Otherwise, with chunk > 0, each query
// block's range is cut into pieces of chunk blocks, and workgroup x takes
// piece x of the list that runs from the longest query block down (so no
// workgroup has more than chunk blocks, whatever the query block); with
// chunk == 0 workgroup x takes query block nqb - 1 - x whole.
template <int W, bool PAIR>
__global__ __launch_bounds__(64 * W)
void attn_mfma_kernel(const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
                      size_t layer_off, size_t head_stride, int n_head, int n_head_kv, int q_len, int kv_len,
                      long long start_pos, float score_scale, float* __restrict__ out, float* __restrict__ part,
                      int chunk, int stride) {
    __shared__ __align__(16) uint8_t lds[2][2 * AM_BLK];
    const int nqb = (q_len + 31) / 32, x = blockIdx.x;
    if (!PAIR && chunk > 0) {
        // the list is ordered by length across the head groups: workgroup x
        // takes piece x / G of head group x % G (G = n_head / W groups; the
        // grid is one-dimensional here)
        const int groups = n_head / W;
        const int grp = x % groups;
        int qb = nqb - 1, rem = x / groups;
        for (; qb >= 0; qb--) {
            const int pieces = (am_qblock_blocks(qb, q_len, kv_len, start_pos) + chunk - 1) / chunk;
            if (rem < pieces) break;
            rem -= pieces;
        }
        if (qb < 0) return;   // past the list (the grid is its length)
        am_qblock<W>(lds, q, kc, vc, layer_off, head_stride, n_head, n_head_kv, q_len, kv_len, start_pos, score_scale,
                     out, qb, chunk, rem, stride, part, grp);
        return;
    }
    const int qb_long = nqb - 1 - x;
    am_qblock<W>(lds, q, kc, vc, layer_off, head_stride, n_head, n_head_kv, q_len, kv_len, start_pos, score_scale, out,
                 qb_long);
    if (PAIR && x < qb_long) {
        __syncthreads();   // every wave is done with the stages
        am_qblock<W>(lds, q, kc, vc, layer_off, head_stride, n_head, n_head_kv, q_len, kv_len, start_pos, score_scale,
                     out, x);
    }
}

static int attn_mfma_min_q() { return tuning_env(TUNE_ATTN_MFMA_MIN_Q, 32); }

// The prompt path: head_dim 128, q_len at the threshold, and a kv head's
// rows addressable by the 32-bit buffer offsets of its K/V loads.
static bool attn_mfma_path(const AttnArgs& a) {
    return a.head_dim == 128 && a.q_len >= (size_t)attn_mfma_min_q() && a.kv_len < ((size_t)1 << 23);
}

static int cu_count_attn();

// Launch plan of the prompt kernel: W query heads per workgroup (W divides
// the GQA group), query-block pairing when the pairs alone fill the CUs, and
// otherwise pieces of `chunk` position blocks (partial states merged by
// attn_combine_few_kernel): chunk is the work per CU if the blocks of all
// query blocks were shared evenly, so no workgroup runs much longer than the
// average.  The plan assumes the chunk's queries are the last q_len of the
// kv_len positions (a prompt); at launch only the piece counts follow the
// actual start position, within `stride` pieces per query block (the
// workspace bound).
struct AmPlan {
    int w;
    int chunk;    // position blocks per piece; 0: whole query blocks, no partial states
    int stride;   // partial states per (query row, head)
    bool pair;
    unsigned nqb, groups;
};

static AmPlan attn_mfma_plan_uncached(size_t n_head, size_t n_head_kv, size_t q_len, size_t kv_len);

// The plan of the last (n_head, n_head_kv, q_len, kv_len, device) this
// thread asked for: the workspace query and the launch ask in turn.
static AmPlan attn_mfma_plan(size_t n_head, size_t n_head_kv, size_t q_len, size_t kv_len) {
    struct Entry {
        size_t key[4];
        int dev;
        AmPlan plan;
        bool valid;
    };
    thread_local Entry last = {{0, 0, 0, 0}, -1, AmPlan{}, false};
    if (tuning_env(TUNE_ATTN_MFMA_SPLIT) > 0) return attn_mfma_plan_uncached(n_head, n_head_kv, q_len, kv_len);
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    if (last.valid && last.dev == dev && last.key[0] == n_head && last.key[1] == n_head_kv && last.key[2] == q_len &&
        last.key[3] == kv_len)
        return last.plan;
    const AmPlan p = attn_mfma_plan_uncached(n_head, n_head_kv, q_len, kv_len);
    last = Entry{{n_head, n_head_kv, q_len, kv_len}, dev, p, true};
    return p;
}

static AmPlan attn_mfma_plan_uncached(size_t n_head, size_t n_head_kv, size_t q_len, size_t kv_len) {
    AmPlan p{};
    const size_t grp = (n_head_kv && n_head % n_head_kv == 0) ? n_head / n_head_kv : 1;
    p.w = grp % 4 == 0 ? 4 : grp % 2 == 0 ? 2 : 1;
    p.nqb = (unsigned)((q_len + 31) / 32);
    p.groups = (unsigned)(n_head / p.w);
    const size_t cus = (size_t)cu_count_attn();
    p.pair = (size_t)(p.nqb / 2) * p.groups >= cus;
    p.chunk = 0;
    p.stride = 1;
    // the merge writes whole Q8_K blocks (256 values: two heads of 128)
    if (p.pair || (n_head * 128) % 256 != 0) return p;
    const long long start = kv_len > q_len ? (long long)(kv_len - q_len) : 0;
    size_t total = 0;
    int longest = 0;
    for (unsigned qb = 0; qb < p.nqb; qb++) {
        const int nb = am_qblock_blocks((int)qb, (int)q_len, (int)kv_len, start);
        total += (size_t)nb;
        longest = nb > longest ? nb : longest;
    }
    (void)total;
    // Choose the chunk by simulating the launch in units of one position
    // block: the pieces in the kernel's order (each costing its blocks + 1.5
    // for its fixed part: the query rows, the first copy, the partial state),
    // every CU holding up to two workgroups that share it equally, each
    // further piece going to the CU that frees a slot first.  Candidates cut
    // the longest query block into k = 1 .. 64 pieces; ties keep fewer
    // pieces.  The model picks the measured best at 512, 768 and 1024 tokens
    // (Llama-3-8B heads, us per call, chunk: time): 512 tokens 6: 55.5, 3:
    // 59.3, 8: 61.8, 4: 63.3; 768 tokens 6: 86.2, 12: 97, 4: 97.6, 5: 99.3,
    // 8: 100, 16: 102.3, 24: 122; 1024 tokens 11: 132, 6: 138, 32 (whole
    // query blocks): 157.4, 8: 157.6.  (With a fixed part of 1 block it chose
    // 5 at 768 tokens.)
    std::vector<int> nbs(p.nqb);
    for (unsigned qb = 0; qb < p.nqb; qb++) nbs[qb] = am_qblock_blocks((int)qb, (int)q_len, (int)kv_len, start);
    auto simulate = [&](int c) {
        std::vector<double> jobs;   // the kernel's order: query blocks longest first, then the head groups
        for (int qb = (int)p.nqb - 1; qb >= 0; qb--)
            for (int b = 0; b < nbs[qb]; b += c) {
                const double len = (nbs[qb] - b < c ? nbs[qb] - b : c) + 1.5;
                for (unsigned g = 0; g < p.groups; g++) jobs.push_back(len);
            }
        struct Cu { double t, w[2]; int n; };
        std::vector<Cu> cu(cus, Cu{0.0, {0.0, 0.0}, 0});
        size_t next = 0;
        for (int pass = 0; pass < 2; pass++)
            for (size_t k = 0; k < cus && next < jobs.size(); k++) cu[k].w[cu[k].n++] = jobs[next++];
        auto event = [](const Cu& u) {
            return u.n == 2 ? u.t + 2.0 * (u.w[0] < u.w[1] ? u.w[0] : u.w[1]) : u.t + u.w[0];
        };
        typedef std::pair<double, size_t> Ev;
        std::priority_queue<Ev, std::vector<Ev>, std::greater<Ev>> heap;
        for (size_t k = 0; k < cus; k++)
            if (cu[k].n) heap.push(Ev(event(cu[k]), k));
        double end = 0.0;
        while (!heap.empty()) {
            const Ev ev = heap.top();
            heap.pop();
            Cu& u = cu[ev.second];
            if (u.n == 2) {   // the shorter job ends; the other has done as much
                const int done = u.w[0] < u.w[1] ? 0 : 1;
                u.w[0] = u.w[1 - done] - u.w[done];
                u.n = 1;
            } else {
                u.n = 0;
            }
            u.t = ev.first;
            end = ev.first > end ? ev.first : end;
            if (next < jobs.size()) u.w[u.n++] = jobs[next++];
            if (u.n) heap.push(Ev(event(u), ev.second));
        }
        return end;
    };
    size_t chunk = (size_t)longest;
    double best = simulate(longest);
    for (int k = 2; k <= 64 && k <= longest; k++) {
        const int c = (longest + k - 1) / k;
        if ((size_t)c >= chunk) continue;
        // more than eight pieces per CU never measured faster; the bound
        // also keeps the simulation to a few thousand pieces
        size_t n = 0;
        for (int nb : nbs) n += (size_t)((nb + c - 1) / c);
        if (n * p.groups > 8 * cus) break;   // smaller chunks only add pieces
        const double e = simulate(c);
        if (e < best - 1e-9) {
            best = e;
            chunk = (size_t)c;
        }
    }
    const int ovr = tuning_env(TUNE_ATTN_MFMA_SPLIT);   // pieces of the longest query block (tuning)
    if (ovr > 0) chunk = ((size_t)longest + (size_t)ovr - 1) / (size_t)ovr;
    if (chunk < 1) chunk = 1;
    if (chunk >= (size_t)longest) return p;   // every query block in one piece
    const size_t nbmax = (kv_len + 31) / 32;
    p.chunk = (int)chunk;
    p.stride = (int)((nbmax + chunk - 1) / chunk);
    return p;
}

static int cu_count_attn() {
    static std::atomic<int> n[64] = {};   // per device; racing callers store the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = n[dev].load(std::memory_order_relaxed);
    if (!v) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        n[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

size_t attention_workspace(size_t n_head, size_t head_dim, size_t q_len, size_t kv_len, size_t n_head_kv) {
    if (head_dim == 128 && q_len >= (size_t)attn_mfma_min_q() && kv_len < ((size_t)1 << 23)) {
        const AmPlan p = attn_mfma_plan(n_head, n_head_kv, q_len, kv_len);
        return p.chunk > 0 ? (size_t)p.stride * n_head * q_len * (head_dim + 2) * sizeof(float) : 0;
    }
    int ns = 0, chunk = 0;
    attention_plan(n_head, n_head_kv, q_len, kv_len, &ns, &chunk);
    return ns > 1 ? (size_t)ns * n_head * q_len * (head_dim + 2) * sizeof(float) : 0;
}


// Splits: at most about three workgroups per four CUs in all, whole
// multiples of 64 positions each.  A CU that runs two workgroups while
// others run one finishes last, so the launch keeps to one per CU; fewer,
// longer workgroups keep more loads in flight each.  Measured on MI355X
// (Llama-3-8B heads, us per call, targets 192 / 256 / 320 / 512 workgroups):
// 4096 positions 10.96 / 11.09 / 11.08 / 11.73, 4097 11.03 / 11.00 / 13.30 /
// 13.27, 8192 15.62 / 15.88 / 15.92 / 16.04, 16384 25.13 / 25.39 / 31.01 /
// 25.68; the decode layer about 51.5 / 51.6 / 53.9 / 53.9.
void attention_plan(size_t n_head, size_t n_head_kv, size_t q_len, size_t kv_len, int* n_split, int* chunk) {
    const size_t g = (n_head_kv && n_head % n_head_kv == 0) ? n_head / n_head_kv : 1;
    const size_t groups = (g == 1 || g > 8 || (g & (g - 1))) ? n_head : n_head_kv;
    const size_t wg = groups * (q_len ? q_len : 1);
    const int wg_override = tuning_env(TUNE_ATTN_WG);   // workgroup-count target (tuning)
    const size_t cus = (size_t)cu_count_attn();
    const size_t target = wg_override > 0 ? (size_t)wg_override : (cus * 3 / 4 > 0 ? cus * 3 / 4 : 1);
    size_t ns = (target + wg - 1) / wg;
    size_t max_ns = (kv_len + 63) / 64;
    if (max_ns > (size_t)ATT_MAX_SPLIT) max_ns = ATT_MAX_SPLIT;
    if (ns > max_ns) ns = max_ns;
    // at most 2^20 positions per split: the split kernel addresses its rows
    // with 32-bit byte offsets (under 1 GiB at head_dim 256)
    const size_t min_ns = (kv_len + ((size_t)1 << 20) - 1) >> 20;
    if (ns < min_ns) ns = min_ns;
    if (ns < 1) ns = 1;
    size_t ch = (kv_len + ns - 1) / ns;
    ch = (ch + 63) / 64 * 64;
    ns = (kv_len + ch - 1) / ch;
    if (ns < 1) ns = 1;
    *n_split = (int)ns;
    *chunk = (int)ch;
}

// Whether attention_launch writes a.out_q8 itself (the split path's merge
// emits Q8_K rows); otherwise it writes f32 rows to a.out and the caller
// quantizes them.
bool attention_q8_direct(const AttnArgs& a) {
    if ((a.n_head * a.head_dim) % 256 != 0) return false;
    if (attn_mfma_path(a)) return attn_mfma_plan(a.n_head, a.n_head_kv, a.q_len, a.kv_len).chunk > 0;
    int ns = 0, chunk = 0;
    attention_plan(a.n_head, a.n_head_kv, a.q_len, a.kv_len, &ns, &chunk);
    return ns > 1;
}

template <int HD, int G>
static hipError_t attn_launch_t(const AttnArgs& a, int ns, int chunk, int groups, hipStream_t s) {
    const float scale = (1.0f / sqrtf((float)HD)) * LOG2E;
    hipLaunchKernelGGL((attn_kernel<HD, G>), dim3(ns, groups, (unsigned)a.q_len), dim3(ATT_THREADS), 0, s, a.q, a.k,
                       a.v, a.layer_off, a.head_stride, (int)a.n_head, (int)a.n_head_kv, (int)a.q_len, (int)a.kv_len,
                       (long long)a.start_pos, chunk, scale, a.part, a.out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ns == 1) return e;
    if (a.out_q8 && attention_q8_direct(a))
        hipLaunchKernelGGL(attn_combine_q8k_kernel<HD>, dim3((unsigned)(a.n_head * HD / 256), (unsigned)a.q_len),
                           dim3(1024), 0, s, a.part, ns, (int)a.n_head, a.out_q8);
    else
        hipLaunchKernelGGL(attn_combine_kernel<HD>, dim3((unsigned)a.n_head, (unsigned)a.q_len), dim3(1024), 0, s,
                           a.part, ns, (int)a.n_head, a.out);
    return hipGetLastError();
}

template <int HD>
static hipError_t attn_launch_hd(const AttnArgs& a, hipStream_t s) {
    int ns = 0, chunk = 0;
    attention_plan(a.n_head, a.n_head_kv, a.q_len, a.kv_len, &ns, &chunk);
    const size_t g = (a.n_head_kv && a.n_head % a.n_head_kv == 0) ? a.n_head / a.n_head_kv : 1;
    switch (g) {
    case 2: return attn_launch_t<HD, 2>(a, ns, chunk, (int)a.n_head_kv, s);
    case 4: return attn_launch_t<HD, 4>(a, ns, chunk, (int)a.n_head_kv, s);
    case 8: return attn_launch_t<HD, 8>(a, ns, chunk, (int)a.n_head_kv, s);
    default: return attn_launch_t<HD, 1>(a, ns, chunk, (int)a.n_head, s);
    }
}

hipError_t attention_launch(const AttnArgs& a, hipStream_t s) {
    if (a.q_len == 0 || a.n_head == 0) return hipSuccess;
    if (attn_mfma_path(a)) {
        const float scale = (1.0f / sqrtf(128.0f)) * LOG2E;
        const AmPlan p = attn_mfma_plan(a.n_head, a.n_head_kv, a.q_len, a.kv_len);
        const int w = p.w;
        const bool pair = p.pair;
        unsigned nx = pair ? (p.nqb + 1) / 2 : p.nqb;
        if (p.chunk > 0) {   // the pieces of every query block at the actual start position
            nx = 0;
            for (unsigned qb = 0; qb < p.nqb; qb++)
                nx += (unsigned)((am_qblock_blocks((int)qb, (int)a.q_len, (int)a.kv_len, (long long)a.start_pos) +
                                  p.chunk - 1) / p.chunk);
        }
        const dim3 grid = p.chunk > 0 ? dim3(nx * p.groups, 1, 1) : dim3(nx, p.groups, 1);
#define BARQ_AM_LAUNCH(W_, P_)                                                                                    \
    hipLaunchKernelGGL((attn_mfma_kernel<W_, P_>), grid, dim3(64 * W_), 0, s, a.q, a.k, a.v, a.layer_off,           \
                       a.head_stride, (int)a.n_head, (int)a.n_head_kv, (int)a.q_len, (int)a.kv_len,               \
                       (long long)a.start_pos, scale, a.out, a.part, p.chunk, p.stride)
        if (w == 4) { if (pair) BARQ_AM_LAUNCH(4, true); else BARQ_AM_LAUNCH(4, false); }
        else if (w == 2) { if (pair) BARQ_AM_LAUNCH(2, true); else BARQ_AM_LAUNCH(2, false); }
        else { if (pair) BARQ_AM_LAUNCH(1, true); else BARQ_AM_LAUNCH(1, false); }
#undef BARQ_AM_LAUNCH
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || p.chunk == 0) return e;
        // (the plan splits only when the rows are whole Q8_K blocks)
        const dim3 cg((unsigned)(a.n_head * 128 / 256), (unsigned)a.q_len);
        if (a.out_q8)
            hipLaunchKernelGGL((attn_combine_few_kernel<128, true>), cg, dim3(256), 0, s, a.part, p.stride, p.chunk,
                               (int)a.n_head, (int)a.q_len, (int)a.kv_len, (long long)a.start_pos, a.out, a.out_q8);
        else
            hipLaunchKernelGGL((attn_combine_few_kernel<128, false>), cg, dim3(256), 0, s, a.part, p.stride, p.chunk,
                               (int)a.n_head, (int)a.q_len, (int)a.kv_len, (long long)a.start_pos, a.out, a.out_q8);
        return hipGetLastError();
    }
    switch (a.head_dim) {
    case 64: return attn_launch_hd<64>(a, s);
    case 128: return attn_launch_hd<128>(a, s);
    case 256: return attn_launch_hd<256>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace barq
