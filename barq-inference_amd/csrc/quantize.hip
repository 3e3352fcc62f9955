// Activation quantizers (llama.cpp block_q8_0 / block_q8_K; the reference has
// no implementation — Q8_K is only a type id, gguf.rs:132) and the
// reference's own Q4_0 encoder (quant/src/q4_0.rs:23-67).
//
// All arithmetic is single IEEE operations (division is correctly rounded in
// HIP by default), so results are bit-identical to the CPU restatement.
#include "common.hpp"
#include "launch.hpp"
#include "q8k_block.hpp"

namespace barq {

// Q8_0: one lane per element, 32 lanes per block.
// d = amax/127 (stored f16), id = d ? 1/d : 0, q = roundf(x*id).
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ x,
                                                            uint8_t* __restrict__ out, size_t nb) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nb * 32) return;  // whole 32-lane groups exit together
    const size_t b = e / 32;
    const int l = (int)(e % 32);
    const float v = x[e];
    float a = fabsf(v);
    a = group_max<32>(a);
    const float d = a / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)roundf(v * id);
    uint8_t* blk = out + b * 34;
    blk[2 + l] = (uint8_t)(int8_t)q;
    if (l == 0) *reinterpret_cast<uint16_t*>(blk) = f32_to_f16_bits(d);
}

__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float* __restrict__ x,
                                                            uint8_t* __restrict__ out, size_t nb) {
    const size_t b = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;  // whole waves exit together
    const int lane = threadIdx.x & 63;
    const float4 v = reinterpret_cast<const float4*>(x + b * 256)[lane];
    const float vv[4] = {v.x, v.y, v.z, v.w};
    q8_k_block(vv, lane, out + b * 292);
}

// Q8_K of rows x[rows_idx[i]] (a MoE row gather fused into the quantizer);
// nbr blocks per row.
__global__ __launch_bounds__(256) void quantize_q8_k_gather_kernel(const float* __restrict__ x,
                                                                   const int32_t* __restrict__ rows_idx, size_t nbr,
                                                                   uint8_t* __restrict__ out, size_t nb) {
    const size_t b = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;
    const int lane = threadIdx.x & 63;
    const size_t i = b / nbr, cb = b - i * nbr;
    const float4 v = reinterpret_cast<const float4*>(x + ((size_t)rows_idx[i] * nbr + cb) * 256)[lane];
    const float vv[4] = {v.x, v.y, v.z, v.w};
    q8_k_block(vv, lane, out + b * 292);
}

// The two SwiGLU roundings of the reference:
//   MoE expert FFN: silu(g) = g / (1 + exp(-g)) rounded first, then * u
//     (ops::Silu, ops.rs:191-211; the product of moe_fused.rs:61-66);
//   dense FFN: (g * (1 / (1 + exp(-g)))) * u (transformer.rs:394-399).
template <bool DENSE>
__device__ __forceinline__ float swiglu_form(float g, float u) {
    if constexpr (DENSE) {
        return (g * (1.0f / (1.0f + expf(-g)))) * u;
    } else {
        const float a = g / (1.0f + expf(-g));
        return a * u;
    }
}

// Q8_K of h = swiglu(g, u): the SwiGLU product is formed in registers and
// never stored.
template <bool DENSE>
__global__ __launch_bounds__(256) void swiglu_q8_k_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                          uint8_t* __restrict__ out, size_t nb) {
    const size_t b = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;
    const int lane = threadIdx.x & 63;
    const float4 gv = reinterpret_cast<const float4*>(g + b * 256)[lane];
    const float4 uv = reinterpret_cast<const float4*>(u + b * 256)[lane];
    const float ga[4] = {gv.x, gv.y, gv.z, gv.w}, ua[4] = {uv.x, uv.y, uv.z, uv.w};
    float vv[4];
    #pragma unroll
    for (int j = 0; j < 4; j++) vv[j] = swiglu_form<DENSE>(ga[j], ua[j]);
    q8_k_block(vv, lane, out + b * 292);
}

// Q8_0 of the dense FFN's h (one lane per element, as quantize_q8_0_kernel)
__global__ __launch_bounds__(256) void swiglu_q8_0_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                          uint8_t* __restrict__ out, size_t nb) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nb * 32) return;
    const size_t b = e / 32;
    const int l = (int)(e % 32);
    const float v = swiglu_form<true>(g[e], u[e]);
    float a = fabsf(v);
    a = group_max<32>(a);
    const float d = a / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)roundf(v * id);
    uint8_t* blk = out + b * 34;
    blk[2 + l] = (uint8_t)(int8_t)q;
    if (l == 0) *reinterpret_cast<uint16_t*>(blk) = f32_to_f16_bits(d);
}

// f32 h of the dense FFN (n elements)
__global__ __launch_bounds__(256) void swiglu_f32_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                         float* __restrict__ h, size_t n) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) h[e] = swiglu_form<true>(g[e], u[e]);
}

// quant::Q4_0::quantize (quant/src/q4_0.rs:23-67): scale = max_abs/8 (0 for an
// all-zero block), q = clamp(round(x/scale) as i8, -8, 7) with Rust's
// half-away-from-zero round and saturating cast; element i goes to the low
// (even i) or high (odd i) nibble of byte i/2.  20-byte blocks.
__global__ __launch_bounds__(256) void quantize_q4_0_barq_kernel(const float* __restrict__ x,
                                                                 uint8_t* __restrict__ out, size_t nb) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nb * 32) return;
    const size_t b = e / 32;
    const int l = (int)(e % 32);
    const float v = x[e];
    float a = fabsf(v);
    a = group_max<32>(a);
    const float scale = a == 0.0f ? 0.0f : a / 8.0f;
    int q = 0;
    if (scale != 0.0f) {
        const float r = roundf(v / scale);
        q = (r != r) ? 0 : (r > 127.0f ? 127 : (r < -128.0f ? -128 : (int)r));
    }
    q = q < -8 ? -8 : (q > 7 ? 7 : q);
    const uint32_t nib = (uint32_t)q & 0x0Fu;
    const uint32_t other = __shfl_xor(nib, 1);
    uint8_t* blk = out + b * 20;
    if ((l & 1) == 0) blk[4 + l / 2] = (uint8_t)(nib | (other << 4));
    if (l == 0) *reinterpret_cast<float*>(blk) = scale;
}

hipError_t quantize_q8_0_launch(const float* x, size_t n_rows, size_t k, void* out, hipStream_t s) {
    const size_t nb = n_rows * (k / 32);
    if (nb == 0) return hipSuccess;
    const size_t threads = nb * 32;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       x, static_cast<uint8_t*>(out), nb);
    return hipGetLastError();
}

hipError_t quantize_q8_k_launch(const float* x, size_t n_rows, size_t k, void* out, hipStream_t s) {
    const size_t nb = n_rows * (k / 256);
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_k_kernel, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x,
                       static_cast<uint8_t*>(out), nb);
    return hipGetLastError();
}

hipError_t quantize_q8_k_gather_launch(const float* x, const int32_t* rows_idx, size_t n_rows, size_t k, void* out,
                                      hipStream_t s) {
    const size_t nbr = k / 256, nb = n_rows * nbr;
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q8_k_gather_kernel, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, rows_idx, nbr,
                       static_cast<uint8_t*>(out), nb);
    return hipGetLastError();
}

hipError_t swiglu_q8_k_launch(const float* g, const float* u, size_t n_rows, size_t k, void* out, hipStream_t s) {
    const size_t nb = n_rows * (k / 256);
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_q8_k_kernel<false>, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, g, u,
                       static_cast<uint8_t*>(out), nb);
    return hipGetLastError();
}

hipError_t ffn_swiglu_launch(int out_type, const float* g, const float* u, size_t n_rows, size_t n, void* out,
                             hipStream_t s) {
    const size_t total = n_rows * n;
    if (total == 0) return hipSuccess;
    if (out_type == TYPE_Q8_K) {
        const size_t nb = total / 256;
        hipLaunchKernelGGL(swiglu_q8_k_kernel<true>, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, g, u,
                           static_cast<uint8_t*>(out), nb);
    } else if (out_type == TYPE_Q8_0) {
        const size_t nb = total / 32;
        hipLaunchKernelGGL(swiglu_q8_0_kernel, dim3((unsigned)((nb * 32 + 255) / 256)), dim3(256), 0, s, g, u,
                           static_cast<uint8_t*>(out), nb);
    } else {
        hipLaunchKernelGGL(swiglu_f32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, g, u,
                           static_cast<float*>(out), total);
    }
    return hipGetLastError();
}

// quant::Q4_K::quantize (quant/src/q4_k.rs:23-73), the quant crate's own
// 4-bit format: blocks of 256 (the last one may be shorter); per block the
// f32 min and max (folds that skip NaN), scale_max = max - min,
// q = clamp(round((x - min) / scale_max * 15), 0, 15) (7.5 -> 8 when
// scale_max is 0; Rust's half-away-from-zero round, NaN -> 0 as `as u8`
// does), two per byte, low nibble first.  A block is 8 + ceil(len/2) bytes.
// One wave per block, four elements per lane.
__global__ __launch_bounds__(256) void quantize_q4_k_barq_kernel(const float* __restrict__ x, size_t n,
                                                                 uint8_t* __restrict__ out, size_t nb) {
    const size_t b = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nb) return;
    const int lane = threadIdx.x & 63;
    const size_t e0 = b * 256;
    const int len = (int)(n - e0 < 256 ? n - e0 : 256);
    float v[4];
    float mn = INFINITY, mx = -INFINITY;
    #pragma unroll
    for (int j = 0; j < 4; j++) {
        const int i = 4 * lane + j;
        v[j] = i < len ? x[e0 + i] : 0.0f;
        if (i < len) {
            mn = fminf(mn, v[j]);
            mx = fmaxf(mx, v[j]);
        }
    }
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, off));
        mx = fmaxf(mx, __shfl_xor(mx, off));
    }
    const float range = mx - mn;
    uint32_t q[4];
    #pragma unroll
    for (int j = 0; j < 4; j++) {
        const float t = range == 0.0f ? 7.5f : (v[j] - mn) / range * 15.0f;
        const float r = fminf(fmaxf(roundf(t), 0.0f), 15.0f);
        q[j] = (r == r && 4 * lane + j < len) ? (uint32_t)r : 0u;   // NaN -> 0; past the block: 0
    }
    uint8_t* p = out + b * Q4_K_BARQ_BYTES;
    if (lane == 0) {
        reinterpret_cast<float*>(p)[0] = mn;
        reinterpret_cast<float*>(p)[1] = range;
    }
    const int nbytes = (len + 1) / 2;
    if (2 * lane < nbytes) p[8 + 2 * lane] = (uint8_t)(q[0] | (q[1] << 4));
    if (2 * lane + 1 < nbytes) p[9 + 2 * lane] = (uint8_t)(q[2] | (q[3] << 4));
}

hipError_t quantize_q4_k_barq_launch(const float* x, size_t n, uint8_t* out, hipStream_t s) {
    const size_t nb = (n + 255) / 256;
    if (nb == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q4_k_barq_kernel, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, s, x, n, out, nb);
    return hipGetLastError();
}

hipError_t quantize_q4_0_barq_launch(const float* x, size_t n, uint8_t* out, hipStream_t s) {
    const size_t nb = n / 32;
    if (nb == 0) return hipSuccess;
    const size_t threads = nb * 32;
    hipLaunchKernelGGL(quantize_q4_0_barq_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       x, out, nb);
    return hipGetLastError();
}

}  // namespace barq
