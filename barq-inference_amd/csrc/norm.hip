// RMSNorm (models/src/transformer.rs:148-172), alone and fused with the
// activation quantizer that the next projection consumes.
//
//   eps' = max(eps, f32::EPSILON)                      (:158)
//   sum_sq = sum of x^2 over the row                   (:162)
//   rms_inv = 1 / sqrt(sum_sq / n + eps')              (:163-164)
//   y = (x * rms_inv) * w                              (:166)
//
// One workgroup (a wave per 256 elements, up to 16) per row; the row is held in registers, so the
// fused variant reads x once and writes only Q8_K / Q8_0 blocks.  The sum of
// squares runs in a fixed tree order (per lane, then DPP rows and lane swaps
// across the wave, then the wave partials in order); the reference sums
// sequentially, so the two agree to float rounding, not bit for bit.  Every
// later step (the products and the quantizer) is the reference's own
// sequence of single IEEE operations.
#include "common.hpp"
#include "launch.hpp"
#include "q8k_block.hpp"

namespace barq {

constexpr int NORM_MAX_WAVES = 16;

// The Q8_K blocks come from q8_k_block (q8k_block.hpp): a wave per block, four
// elements per lane, the bytes quantize_q8_k_kernel writes for the same values.

// Q8_0 block of 32 = lanes 8g .. 8g + 7 (4 elements each): d = amax / 127
// (stored f16), q = roundf(x * (1 / d)).
__device__ __forceinline__ void norm_q8_0_block(const float (&vv)[4], int lane, uint8_t* __restrict__ blk) {
    float a = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
    a = group_max<8>(a);
    const float d = a / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int l8 = lane & 7;
    uint32_t packed = 0;
    #pragma unroll
    for (int j = 0; j < 4; j++) packed |= (uint32_t)((int)roundf(vv[j] * id) & 0xFF) << (8 * j);
    // bytes 2 + 4 l8 .. : 2-byte aligned, so two 16-bit stores
    uint16_t* qs = reinterpret_cast<uint16_t*>(blk + 2 + 4 * l8);
    qs[0] = (uint16_t)(packed & 0xFFFFu);
    qs[1] = (uint16_t)(packed >> 16);
    if (l8 == 0) *reinterpret_cast<uint16_t*>(blk) = f32_to_f16_bits(d);
}

// W waves, V float4 chunks per lane: chunk i of wave w is float4
// 64 (w + W i) + lane, i.e. lane `lane` of 256-element block w + W i.
// OUT: 0 f32 rows, 1 Q8_K, 2 Q8_0.
// With d non-null the row normalized is x + d (add_vectors, transformer.rs:
// 505-510, the residual adds of forward_layer :136, :143), stored to sum when
// sum is non-null.
template <int W, int V, int OUT>
__global__ __launch_bounds__(64 * W)
void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ d, const float* __restrict__ w, int n,
                     float eps, float* __restrict__ sum, void* __restrict__ out) {
    __shared__ float part[W];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t row = blockIdx.x;
    const int n4 = n / 4;
    const float4* xr = reinterpret_cast<const float4*>(x + row * (size_t)n);
    const float4* dr = d ? reinterpret_cast<const float4*>(d + row * (size_t)n) : nullptr;
    const float4* wr = reinterpret_cast<const float4*>(w);
    float4 v[V], wv[V];
    // the weight is loaded with x, so the row costs one memory round trip
    #pragma unroll
    for (int i = 0; i < V; i++) {
        const int f = 64 * (wave + W * i) + lane;
        v[i] = f < n4 ? xr[f] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        wv[i] = f < n4 ? wr[f] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (dr) {
        #pragma unroll
        for (int i = 0; i < V; i++) {
            const int f = 64 * (wave + W * i) + lane;
            if (f < n4) {
                const float4 dv = dr[f];
                v[i] = make_float4(v[i].x + dv.x, v[i].y + dv.y, v[i].z + dv.z, v[i].w + dv.w);
                // f32 rows: the sum is stored before them (a caller's out == sum ends with the norm)
                if (OUT == 0 && sum) reinterpret_cast<float4*>(sum + row * (size_t)n)[f] = v[i];
            }
        }
    }
    float ss = 0.0f;
    #pragma unroll
    for (int i = 0; i < V; i++) {
        ss = ss + v[i].x * v[i].x;
        ss = ss + v[i].y * v[i].y;
        ss = ss + v[i].z * v[i].z;
        ss = ss + v[i].w * v[i].w;
    }
    ss = wave_sum_all(ss);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    float sum_sq = part[0];
    #pragma unroll
    for (int i = 1; i < W; i++) sum_sq = sum_sq + part[i];
    const float e = fmaxf(eps, 1.1920929e-7f);
    const float rms_inv = 1.0f / sqrtf(sum_sq / (float)n + e);
    #pragma unroll
    for (int i = 0; i < V; i++) {
        const int blk = wave + W * i, f = 64 * blk + lane;
        if (64 * blk >= n4) break;   // whole waves: n is a multiple of 256 for the quantized outputs
        float y[4] = {(v[i].x * rms_inv) * wv[i].x, (v[i].y * rms_inv) * wv[i].y, (v[i].z * rms_inv) * wv[i].z,
                      (v[i].w * rms_inv) * wv[i].w};
        if constexpr (OUT == 0) {
            if (f < n4) reinterpret_cast<float4*>(static_cast<float*>(out) + row * (size_t)n)[f] =
                make_float4(y[0], y[1], y[2], y[3]);
        } else if constexpr (OUT == 1) {
            uint8_t* o = static_cast<uint8_t*>(out) + (row * (size_t)(n / 256) + blk) * Q8_K_BYTES;
            q8_k_block(y, lane, o);
        } else {
            uint8_t* o = static_cast<uint8_t*>(out) + (row * (size_t)(n / 32) + 8 * blk + (lane >> 3)) * Q8_0_BYTES;
            norm_q8_0_block(y, lane, o);
        }
    }
    // quantized rows: the sum x + d is stored last, since a store issued before
    // the reduction made the compiler wait for it (vmcnt counts stores too)
    if (OUT != 0 && dr && sum) {
        #pragma unroll
        for (int i = 0; i < V; i++) {
            const int f = 64 * (wave + W * i) + lane;
            if (f < n4) reinterpret_cast<float4*>(sum + row * (size_t)n)[f] = v[i];
        }
    }
}

// One wave per 256 elements up to 16 waves (short rows still spread over
// many SIMDs), then up to four float4 chunks per lane.
template <int W, int OUT>
static hipError_t launch_norm_w(const float* x, const float* d, const float* w, size_t rows, size_t n, float eps,
                                float* sum, void* out, hipStream_t s) {
    const size_t chunks = (n / 4 + 64 * W - 1) / (64 * W);   // float4 chunks per lane
#define BARQ_NORM_CASE(VV) \
    if (chunks <= VV) { \
        hipLaunchKernelGGL((rms_norm_kernel<W, VV, OUT>), dim3((unsigned)rows), dim3(64 * W), 0, s, x, d, w, (int)n, \
                           eps, sum, out); \
        return hipGetLastError(); \
    }
    BARQ_NORM_CASE(1) BARQ_NORM_CASE(2) BARQ_NORM_CASE(4)
#undef BARQ_NORM_CASE
    return hipErrorInvalidValue;
}

template <int OUT>
static hipError_t launch_norm(const float* x, const float* d, const float* w, size_t rows, size_t n, float eps,
                              float* sum, void* out, hipStream_t s) {
    const size_t blocks = (n + 255) / 256;
    if (blocks <= 1) return launch_norm_w<1, OUT>(x, d, w, rows, n, eps, sum, out, s);
    if (blocks <= 2) return launch_norm_w<2, OUT>(x, d, w, rows, n, eps, sum, out, s);
    if (blocks <= 4) return launch_norm_w<4, OUT>(x, d, w, rows, n, eps, sum, out, s);
    if (blocks <= 8) return launch_norm_w<8, OUT>(x, d, w, rows, n, eps, sum, out, s);
    return launch_norm_w<16, OUT>(x, d, w, rows, n, eps, sum, out, s);
}

// rows of up to 16 waves x 4 float4 chunks per lane (16384 elements) are held in registers
bool rms_norm_supported(size_t n) { return n > 0 && n % 4 == 0 && n <= 4 * 4 * 64 * NORM_MAX_WAVES; }

hipError_t rms_norm_launch(const float* x, const float* w, size_t rows, size_t n, float eps, float* y,
                           hipStream_t s) {
    if (rows == 0) return hipSuccess;
    return launch_norm<0>(x, nullptr, w, rows, n, eps, nullptr, y, s);
}

hipError_t rms_norm_quantize_launch(int act_type, const float* x, const float* w, size_t rows, size_t n, float eps,
                                    void* out, hipStream_t s) {
    return add_rms_norm_launch(act_type, x, nullptr, w, rows, n, eps, nullptr, out, s);
}

hipError_t add_rms_norm_launch(int out_type, const float* x, const float* d, const float* w, size_t rows, size_t n,
                               float eps, float* sum, void* out, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (out_type == TYPE_F32) return launch_norm<0>(x, d, w, rows, n, eps, sum, out, s);
    if (n % 256 != 0) return hipErrorInvalidValue;
    return out_type == TYPE_Q8_K ? launch_norm<1>(x, d, w, rows, n, eps, sum, out, s)
                                 : launch_norm<2>(x, d, w, rows, n, eps, sum, out, s);
}

// add_bias (transformer.rs:444-465) and final_output's output.bias
// (:487-495): y[r, j] += bias[j], one f32 addition per element.
__global__ __launch_bounds__(256) void add_bias_kernel(float* __restrict__ y, const float* __restrict__ bias,
                                                       size_t n, uint32_t dim) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = y[i] + bias[i % dim];
}

hipError_t add_bias_launch(float* y, const float* bias, size_t rows, size_t dim, hipStream_t s) {
    const size_t n = rows * dim;
    if (n == 0) return hipSuccess;
    const size_t g = (n + 255) / 256;
    hipLaunchKernelGGL(add_bias_kernel, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(256), 0, s, y, bias, n,
                       (uint32_t)dim);
    return hipGetLastError();
}

}  // namespace barq
