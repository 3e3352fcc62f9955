// Dequantize kernels: GGUF blocks -> f32, bit-identical to the reference's
// load-time decoders (barq_core/src/gguf.rs).  One thread produces four
// consecutive outputs and stores them as one float4, so the f32 writes (the
// dominant traffic: 4 B per element against 0.5-1.1 B read) are coalesced.
// Compiled with -ffp-contract=off: d1*q - m1 rounds the product and the
// difference separately, as Rust does (gguf.rs:804,814).
#include "common.hpp"
#include "launch.hpp"

namespace barq {

__device__ __forceinline__ uint32_t ld4_a2(const uint8_t* p) {
    // 4 bytes at a 2-byte aligned address
    return ld_u16(p) | (ld_u16(p + 2) << 16);
}

template <int TYPE>
__device__ __forceinline__ void deq4_at(const uint8_t* __restrict__ src, size_t e, float v[4]) {
    if constexpr (TYPE == TYPE_Q4_0) {
        // llama.cpp block_q4_0; equals gguf.rs:521-578 applied to the adapted block
        const uint8_t* p = src + (e / 32) * 18;
        const int i = (int)(e % 32);
        const float d = f16_bits_to_f32(ld_u16(p));
        uint32_t q = ld4_a2(p + 2 + (i & 15));
        if (i >= 16) q >>= 4;
        #pragma unroll
        for (int j = 0; j < 4; j++) v[j] = (float)((int)((q >> (8 * j)) & 15u) - 8) * d;
    } else if constexpr (TYPE == TYPE_Q4_0_BARQ) {
        // gguf.rs:540-574: element i = nibble (i%2 ? high : low) of byte i/2, sign-extended
        const uint8_t* p = src + (e / 32) * 20;
        const int i = (int)(e % 32);
        const float scale = *reinterpret_cast<const float*>(p);
        const uint32_t q = ld_u16(p + 4 + i / 2);
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            int n = (q >> (4 * j)) & 15;
            int qs = n >= 8 ? n - 16 : n;
            v[j] = (float)qs * scale;
        }
    } else if constexpr (TYPE == TYPE_Q4_K_BARQ) {
        // quant/src/q4_k.rs:76-132: f32 scale_min, f32 scale_max (the range),
        // 128 nibble bytes (element i: low nibble of byte i/2 if i is even);
        // y = scale_min + (q / 15) * scale_max
        const uint8_t* p = src + (e / 256) * Q4_K_BARQ_BYTES;
        const int i = (int)(e % 256);
        const float smin = *reinterpret_cast<const float*>(p);
        const float srange = *reinterpret_cast<const float*>(p + 4);
        const uint32_t q = ld_u16(p + 8 + i / 2);
        #pragma unroll
        for (int j = 0; j < 4; j++) v[j] = smin + ((float)((q >> (4 * j)) & 15u) / 15.0f) * srange;
    } else if constexpr (TYPE == TYPE_Q8_0) {
        // gguf.rs:658-676: (q as i8) as f32 * scale
        const uint8_t* p = src + (e / 32) * 34;
        const int i = (int)(e % 32);
        const float d = f16_bits_to_f32(ld_u16(p));
        const uint32_t q = ld4_a2(p + 2 + i);
        #pragma unroll
        for (int j = 0; j < 4; j++) v[j] = (float)(int8_t)((q >> (8 * j)) & 0xFFu) * d;
    } else if constexpr (TYPE == TYPE_Q4_K) {
        // gguf.rs:756-819 with get_scale_min_k4 (:825-837)
        const uint8_t* p = src + (e / 256) * 144;
        const int w = (int)(e % 256);
        const int j64 = w / 64, lp = w % 64;
        const int is = 2 * j64 + (lp >= 32);
        const int l = lp & 31;
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(p);
        const float d = f16_bits_to_f32(dd & 0xFFFFu);
        const float dmin = f16_bits_to_f32(dd >> 16);
        const uint8_t* q = p + 4;
        int sc, m;
        if (is < 4) {
            sc = q[is] & 63;
            m = q[is + 4] & 63;
        } else {
            sc = (q[is + 4] & 0xF) | ((q[is - 4] >> 6) << 4);
            m = (q[is + 4] >> 4) | ((q[is] >> 6) << 4);
        }
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        uint32_t qs = *reinterpret_cast<const uint32_t*>(p + 16 + 32 * j64 + l);
        if (lp >= 32) qs >>= 4;
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            const float prod = d1 * (float)((qs >> (8 * j)) & 15u);
            v[j] = prod - m1;
        }
    } else if constexpr (TYPE == TYPE_Q6_K) {
        // gguf.rs:863-910
        const uint8_t* p = src + (e / 256) * 210;
        const int w = (int)(e % 256);
        const int h = w / 128, r = w % 128, qd = r / 32, l = r % 32;
        const uint32_t ql = ld4_a2(p + 64 * h + 32 * (qd & 1) + l);
        const uint32_t qh = ld4_a2(p + 128 + 32 * h + l);
        const int sc = (int8_t)p[192 + 8 * h + l / 16 + 2 * qd];
        const float d = f16_bits_to_f32(ld_u16(p + 208));
        const float dd = d * (float)sc;
        const uint32_t lo = (qd >= 2) ? (ql >> 4) : ql;
        const uint32_t hb = qh >> (2 * qd);
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            const int q = (int)(((lo >> (8 * j)) & 15u) | (((hb >> (8 * j)) & 3u) << 4)) - 32;
            v[j] = dd * (float)q;
        }
    } else if constexpr (TYPE == TYPE_Q8_K) {
        // llama.cpp dequantize_row_q8_K: y = d * q
        const uint8_t* p = src + (e / 256) * 292;
        const int i = (int)(e % 256);
        const float d = *reinterpret_cast<const float*>(p);
        const uint32_t q = *reinterpret_cast<const uint32_t*>(p + 4 + i);
        #pragma unroll
        for (int j = 0; j < 4; j++) v[j] = d * (float)(int8_t)((q >> (8 * j)) & 0xFFu);
    } else if constexpr (TYPE == TYPE_F16) {
        // gguf.rs:456-469
        const uint2 q = *reinterpret_cast<const uint2*>(src + e * 2);
        v[0] = f16_bits_to_f32(q.x & 0xFFFFu);
        v[1] = f16_bits_to_f32(q.x >> 16);
        v[2] = f16_bits_to_f32(q.y & 0xFFFFu);
        v[3] = f16_bits_to_f32(q.y >> 16);
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ src,
                                                      float4* __restrict__ out, size_t n4) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n4; t += stride) {
        float v[4];
        deq4_at<TYPE>(src, t * 4, v);
        out[t] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

static unsigned grid_for(size_t n4) {
    size_t g = (n4 + 255) / 256;
    const size_t cap = 256 * 64;  // 64 workgroups per CU on 256 CUs, then grid-stride
    return (unsigned)(g < cap ? (g ? g : 1) : cap);
}

hipError_t dequant_launch(int type, const void* blocks, size_t n_elems, float* out, hipStream_t s) {
    const uint8_t* src = static_cast<const uint8_t*>(blocks);
    float4* o = reinterpret_cast<float4*>(out);
    const size_t n4 = n_elems / 4;
    if (n4 == 0) return hipSuccess;
    const dim3 g(grid_for(n4)), b(256);
    switch (type) {
    case TYPE_Q4_0: hipLaunchKernelGGL(dequant_kernel<TYPE_Q4_0>, g, b, 0, s, src, o, n4); break;
    case TYPE_Q4_0_BARQ: hipLaunchKernelGGL(dequant_kernel<TYPE_Q4_0_BARQ>, g, b, 0, s, src, o, n4); break;
    case TYPE_Q4_K_BARQ: hipLaunchKernelGGL(dequant_kernel<TYPE_Q4_K_BARQ>, g, b, 0, s, src, o, n4); break;
    case TYPE_Q8_0: hipLaunchKernelGGL(dequant_kernel<TYPE_Q8_0>, g, b, 0, s, src, o, n4); break;
    case TYPE_Q4_K: hipLaunchKernelGGL(dequant_kernel<TYPE_Q4_K>, g, b, 0, s, src, o, n4); break;
    case TYPE_Q6_K: hipLaunchKernelGGL(dequant_kernel<TYPE_Q6_K>, g, b, 0, s, src, o, n4); break;
    case TYPE_Q8_K: hipLaunchKernelGGL(dequant_kernel<TYPE_Q8_K>, g, b, 0, s, src, o, n4); break;
    case TYPE_F16: hipLaunchKernelGGL(dequant_kernel<TYPE_F16>, g, b, 0, s, src, o, n4); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- get_embeddings (models/src/transformer.rs:96-119) ---------------------
// Output row t is row tokens[t] of the table decoded as dequant_kernel
// decodes it (the same deq4_at, so bit-identical to decoding the whole
// table and copying the row); ids outside [0, n_rows) give a zero row, as
// the reference leaves those rows of its zero-initialised output.  One
// workgroup column per token (grid.y), k4 = k / 4 float4 outputs per row.
template <int TYPE>
__global__ __launch_bounds__(256) void get_rows_kernel(const uint8_t* __restrict__ table, size_t row_bytes,
                                                       uint32_t n_rows, const int32_t* __restrict__ tokens,
                                                       float4* __restrict__ out, uint32_t k4) {
    const int32_t id = tokens[blockIdx.y];
    const bool in = id >= 0 && (uint32_t)id < n_rows;
    const uint8_t* row = table + (size_t)(in ? id : 0) * row_bytes;
    float4* o = out + (size_t)blockIdx.y * k4;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < k4; i += gridDim.x * 256) {
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (in) {
            if constexpr (TYPE == TYPE_F32) {
                const float4 f = reinterpret_cast<const float4*>(row)[i];
                v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
            } else {
                deq4_at<TYPE>(row, (size_t)i * 4, v);
            }
        }
        o[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

hipError_t get_rows_launch(int type, const void* table, size_t row_bytes, size_t n_rows, size_t k,
                           const int32_t* tokens, size_t n_tokens, float* out, hipStream_t s) {
    const uint8_t* src = static_cast<const uint8_t*>(table);
    const uint32_t k4 = (uint32_t)(k / 4);
    if (n_tokens == 0 || k4 == 0) return hipSuccess;
    const unsigned gx = (unsigned)((k4 + 255) / 256 < 64 ? (k4 + 255) / 256 : 64);
    for (size_t t0 = 0; t0 < n_tokens; t0 += 65535) {
        const dim3 g(gx, (unsigned)(n_tokens - t0 < 65535 ? n_tokens - t0 : 65535)), b(256);
        float4* o = reinterpret_cast<float4*>(out + t0 * k);
        const int32_t* tk = tokens + t0;
        const uint32_t nr = (uint32_t)n_rows;
        switch (type) {
        case TYPE_F32: hipLaunchKernelGGL(get_rows_kernel<TYPE_F32>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_F16: hipLaunchKernelGGL(get_rows_kernel<TYPE_F16>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_Q4_0: hipLaunchKernelGGL(get_rows_kernel<TYPE_Q4_0>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_Q4_0_BARQ: hipLaunchKernelGGL(get_rows_kernel<TYPE_Q4_0_BARQ>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_Q8_0: hipLaunchKernelGGL(get_rows_kernel<TYPE_Q8_0>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_Q4_K: hipLaunchKernelGGL(get_rows_kernel<TYPE_Q4_K>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_Q6_K: hipLaunchKernelGGL(get_rows_kernel<TYPE_Q6_K>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        case TYPE_Q8_K: hipLaunchKernelGGL(get_rows_kernel<TYPE_Q8_K>, g, b, 0, s, src, row_bytes, nr, tk, o, k4); break;
        default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---- split-scale decoders of the reference's QuantizedCudaOps --------------
// backend/src/cuda_quant.rs:44-75 (packed sign-extended nibbles, block b uses
// scales[b] and quants[b*ceil(bs/2) ..]) and :77-102 (signed bytes,
// quants[b*bs ..]).  Outputs the reference leaves unwritten stay 0 (its
// output vectors are zero-initialised, :245,270,295 and :116).
__global__ __launch_bounds__(256) void dequant_split_kernel(int kind_q8_0, const uint8_t* __restrict__ quants,
                                                            size_t n_quants, const float* __restrict__ scales,
                                                            size_t n_scales, size_t bs, float* __restrict__ out,
                                                            size_t n_out) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t qstride = (bs + 1) / 2;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_out; i += stride) {
        const size_t b = i / bs, rel = i - b * bs;
        float v = 0.0f;
        if (b < n_scales) {
            if (kind_q8_0) {
                const size_t qi = b * bs + rel;
                if (qi < n_quants) v = (float)(int8_t)quants[qi] * scales[b];
            } else {
                const size_t qi = b * qstride + rel / 2;
                if (qi < n_quants) {
                    int q = (quants[qi] >> ((rel & 1) ? 4 : 0)) & 0x0F;
                    if (q >= 8) q -= 16;
                    v = (float)q * scales[b];
                }
            }
        }
        out[i] = v;
    }
}

hipError_t dequant_split_launch(int kind_q8_0, const uint8_t* quants, size_t n_quants,
                                const float* scales, size_t n_scales, size_t block_size,
                                float* out, size_t n_out, hipStream_t s) {
    if (n_out == 0) return hipSuccess;
    size_t g = (n_out + 255) / 256;
    if (g > 16384) g = 16384;
    hipLaunchKernelGGL(dequant_split_kernel, dim3((unsigned)g), dim3(256), 0, s, kind_q8_0, quants,
                       n_quants, scales, n_scales, block_size, out, n_out);
    return hipGetLastError();
}

}  // namespace barq
