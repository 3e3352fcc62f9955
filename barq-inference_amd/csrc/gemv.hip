// Batch-1 quantized GEMV kernels for gfx950: y[n] = sum_k W[n,k] x[k].
//
// Integer path (x already quantized to Q8_0 / Q8_K): weight blocks stay packed
// in HBM and are read once with 16-byte loads; nibbles and 6-bit scales are
// unpacked in registers; the activation vector is staged into LDS once per
// workgroup; products run on v_dot4_i32_i8 and the per-lane partial sums are
// reduced across the wave with DPP.  Each wave owns R consecutive rows.
//
// Literal path (x in f32): the same lane slicing, weights dequantized in
// registers bit-identically to the reference decoders (barq_core/src/gguf.rs)
// and multiplied into f32 accumulators — the arithmetic of
// blas::gemv_f32(dequant(W), x) (blas.rs:292-303) up to summation order.
#include "gemv_formats.hpp"
#include "launch.hpp"

namespace barq {

template <class F>
__device__ __forceinline__ void stage_act(const ActLds& a, const uint8_t* __restrict__ xq, int k) {
    if constexpr (F::ACT_BLOCK == 256) {
        stage_q8k(a, xq, k / 256);
    } else {
        stage_q8_0_copy(a, xq, k / 32);
        __syncthreads();
        stage_sums16(a, k);
    }
}

template <class F, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q8_kernel(const uint8_t* __restrict__ W, size_t row_bytes, const uint8_t* __restrict__ xq,
                    float* __restrict__ y, int n_rows, int k) {
    extern __shared__ __align__(16) uint8_t smem[];
    const ActLds a = act_lds_layout(smem, k, F::ACT_BLOCK);
    stage_act<F>(a, xq, k);
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    const int n_it = (k + 4095) / 4096;

    float acc[R];
    #pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        const bool act = F::active(it, lane, nblk);
        typename F::X xs;
        typename F::Wt w[R];
        if (act) {
            #pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = min(row0 + r, n_rows - 1);
                if constexpr (F::LANES_PER_BLOCK) F::load_w(w[r], W + (size_t)row * row_bytes, it, lane);
                else F::load_w(w[r], W + (size_t)row * row_bytes, it, lane, nblk);
            }
            if constexpr (F::LANES_PER_BLOCK) F::load_x(xs, a, it, lane);
            else F::load_x(xs, a, it, lane, nblk);
            #pragma unroll
            for (int r = 0; r < R; r++) acc[r] += F::dot(w[r], xs, lane);
        }
    }

    #pragma unroll
    for (int r = 0; r < R; r++) {
        const float s = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n_rows) y[row0 + r] = s;
    }
}

template <class F, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64)
void gemv_f32_kernel(const uint8_t* __restrict__ W, size_t row_bytes, const float* __restrict__ x,
                     float* __restrict__ y, int n_rows, int k) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    stage_f32(xs, x, k);
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    const int n_it = (k + 4095) / 4096;

    float acc[R];
    #pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        if (!F::active(it, lane, nblk)) continue;
        typename F::Wt w[R];
        #pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, n_rows - 1);
            if constexpr (F::LANES_PER_BLOCK) F::load_w(w[r], W + (size_t)row * row_bytes, it, lane);
            else F::load_w(w[r], W + (size_t)row * row_bytes, it, lane, nblk);
        }
        // two-block formats: the second block of the last lane may be absent
        const int kbase = it * 4096;
        #pragma unroll
        for (int g = 0; g < 16; g++) {
            const int off = kbase + F::xoff(lane, g);
            if (off >= k) continue;
            const float4 xv = *reinterpret_cast<const float4*>(xs + off);
            #pragma unroll
            for (int r = 0; r < R; r++) {
                float v[4];
                F::deq4(w[r], lane, g, v);
                acc[r] = __builtin_fmaf(v[0], xv.x, acc[r]);
                acc[r] = __builtin_fmaf(v[1], xv.y, acc[r]);
                acc[r] = __builtin_fmaf(v[2], xv.z, acc[r]);
                acc[r] = __builtin_fmaf(v[3], xv.w, acc[r]);
            }
        }
    }

    #pragma unroll
    for (int r = 0; r < R; r++) {
        const float s = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < n_rows) y[row0 + r] = s;
    }
}

// ---- launch configuration ---------------------------------------------------
// (rows per wave, waves per workgroup) for the integer path.  The default for
// each format was chosen by sweeping on MI355X; gemv_set_config overrides it.
struct GemvCfg { int r, waves; };
static GemvCfg g_cfg_override = {0, 0};

void gemv_set_config(int rows_per_wave, int waves) { g_cfg_override = {rows_per_wave, waves}; }

template <class F, int R, int WAVES>
static hipError_t launch_q8(const uint8_t* W, size_t row_bytes, const uint8_t* xq, float* y,
                            int n_rows, int k, hipStream_t s) {
    const int rows_per_block = R * WAVES;
    const unsigned grid = (unsigned)((n_rows + rows_per_block - 1) / rows_per_block);
    const size_t lds = act_lds_bytes(k, F::ACT_BLOCK);
    hipLaunchKernelGGL((gemv_q8_kernel<F, R, WAVES>), dim3(grid), dim3(WAVES * 64), lds, s,
                       W, row_bytes, xq, y, n_rows, k);
    return hipGetLastError();
}

template <class F>
static hipError_t dispatch_q8(const uint8_t* W, size_t row_bytes, const uint8_t* xq, float* y,
                              int n_rows, int k, hipStream_t s, GemvCfg def) {
    GemvCfg c = g_cfg_override.r ? g_cfg_override : def;
#define BARQ_GEMV_CASE(RR, WW) \
    if (c.r == RR && c.waves == WW) return launch_q8<F, RR, WW>(W, row_bytes, xq, y, n_rows, k, s);
    BARQ_GEMV_CASE(1, 4) BARQ_GEMV_CASE(2, 4) BARQ_GEMV_CASE(4, 4) BARQ_GEMV_CASE(8, 4)
    BARQ_GEMV_CASE(1, 8) BARQ_GEMV_CASE(2, 8) BARQ_GEMV_CASE(4, 8)
    BARQ_GEMV_CASE(2, 2) BARQ_GEMV_CASE(4, 2) BARQ_GEMV_CASE(8, 2) BARQ_GEMV_CASE(4, 1)
#undef BARQ_GEMV_CASE
    return launch_q8<F, 2, 4>(W, row_bytes, xq, y, n_rows, k, s);
}

template <class F, int R, int WAVES>
static hipError_t launch_f32(const uint8_t* W, size_t row_bytes, const float* x, float* y,
                             int n_rows, int k, hipStream_t s) {
    const int rows_per_block = R * WAVES;
    const unsigned grid = (unsigned)((n_rows + rows_per_block - 1) / rows_per_block);
    const size_t lds = (size_t)k * 4;
    hipLaunchKernelGGL((gemv_f32_kernel<F, R, WAVES>), dim3(grid), dim3(WAVES * 64), lds, s,
                       W, row_bytes, x, y, n_rows, k);
    return hipGetLastError();
}

hipError_t gemv_q8_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq,
                          float* y, hipStream_t s) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const int n = (int)n_rows, kk = (int)k;
    switch (w_type) {
    case TYPE_Q4_K: return dispatch_q8<FmtQ4K>(w, k / 256 * 144, x, y, n, kk, s, {4, 4});
    case TYPE_Q6_K: return dispatch_q8<FmtQ6K>(w, k / 256 * 210, x, y, n, kk, s, {2, 4});
    case TYPE_Q4_0: return dispatch_q8<FmtQ40>(w, k / 32 * 18, x, y, n, kk, s, {2, 4});
    case TYPE_Q8_0: return dispatch_q8<FmtQ80>(w, k / 32 * 34, x, y, n, kk, s, {2, 4});
    case TYPE_Q4_0_BARQ: return dispatch_q8<FmtQ40Barq>(w, k / 32 * 20, x, y, n, kk, s, {2, 4});
    default: return hipErrorInvalidValue;
    }
}

size_t gemv_q8_lds_bytes(int w_type, size_t k) {
    return act_lds_bytes((int)k, (w_type == TYPE_Q4_K || w_type == TYPE_Q6_K) ? 256 : 32);
}

hipError_t gemv_f32_launch(int w_type, const void* W, size_t n_rows, size_t k, const float* x,
                           float* y, hipStream_t s) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const int n = (int)n_rows, kk = (int)k;
    switch (w_type) {
    case TYPE_Q4_K: return launch_f32<FmtQ4K, 2, 4>(w, k / 256 * 144, x, y, n, kk, s);
    case TYPE_Q6_K: return launch_f32<FmtQ6K, 2, 4>(w, k / 256 * 210, x, y, n, kk, s);
    case TYPE_Q4_0: return launch_f32<FmtQ40, 2, 4>(w, k / 32 * 18, x, y, n, kk, s);
    case TYPE_Q8_0: return launch_f32<FmtQ80, 2, 4>(w, k / 32 * 34, x, y, n, kk, s);
    case TYPE_Q4_0_BARQ: return launch_f32<FmtQ40Barq, 2, 4>(w, k / 32 * 20, x, y, n, kk, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace barq
