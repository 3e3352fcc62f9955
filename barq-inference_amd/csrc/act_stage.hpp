// Staging of the activation vector into LDS for the GEMV kernels.
//
// Q8_K blocks (f32 d, i8 qs[256], i16 bsums[16]; 292 B) and Q8_0 blocks
// (f16 d, i8 qs[32]; 34 B) are restaged into a 16-byte aligned
// structure-of-arrays so every lane reads its K-slice with ds_read_b128:
//   qs  : int8[K]
//   d   : f32[K / block]
//   s16 : int32[K / 16]   (sums of 16 consecutive qs; Q8_K bsums)
#pragma once
#include "common.hpp"

namespace barq {

struct ActLds {
    int8_t* qs;
    float* d;
    int* s16;
};

__host__ __device__ constexpr size_t act_lds_bytes(int k, int block) {
    return (size_t)k + (size_t)(k / block) * 4 + (size_t)(k / 16) * 4;
}

__device__ __forceinline__ ActLds act_lds_layout(uint8_t* smem, int k, int block) {
    ActLds a;
    a.qs = reinterpret_cast<int8_t*>(smem);
    a.d = reinterpret_cast<float*>(smem + k);
    a.s16 = reinterpret_cast<int*>(smem + k + (k / block) * 4);
    return a;
}

// Q8_K: 292-byte blocks are 73 dwords and dword aligned.
__device__ __forceinline__ void stage_q8k(ActLds a, const uint8_t* __restrict__ xq, int nsb) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(xq);
    uint32_t* qs32 = reinterpret_cast<uint32_t*>(a.qs);
    for (int t = threadIdx.x; t < nsb * 73; t += blockDim.x) {
        int b = t / 73, o = t - b * 73;
        uint32_t v = src[t];
        if (o == 0) {
            a.d[b] = __builtin_bit_cast(float, v);
        } else if (o <= 64) {
            qs32[b * 64 + o - 1] = v;
        } else {
            int g = (o - 65) * 2;
            a.s16[b * 16 + g] = (int)(int16_t)(v & 0xFFFFu);
            a.s16[b * 16 + g + 1] = (int)(int16_t)(v >> 16);
        }
    }
}

// Q8_0: 34-byte blocks are 17 half-words; the 16-element sums are computed
// after the copy (caller runs a __syncthreads between the two passes).
__device__ __forceinline__ void stage_q8_0_copy(ActLds a, const uint8_t* __restrict__ xq, int nb) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(xq);
    uint16_t* qs16 = reinterpret_cast<uint16_t*>(a.qs);
    for (int t = threadIdx.x; t < nb * 17; t += blockDim.x) {
        int b = t / 17, o = t - b * 17;
        uint32_t v = src[t];
        if (o == 0) a.d[b] = f16_bits_to_f32(v);
        else qs16[b * 16 + o - 1] = (uint16_t)v;
    }
}

__device__ __forceinline__ void stage_sums16(ActLds a, int k) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a.qs);
    for (int g = threadIdx.x; g < k / 16; g += blockDim.x) {
        int s = 0;
        for (int t = 0; t < 4; t++) s = sdot4(q[g * 4 + t], 0x01010101u, s);
        a.s16[g] = s;
    }
}

// f32 activations for the literal (f32) GEMV: plain copy to LDS.
__device__ __forceinline__ void stage_f32(float* xs, const float* __restrict__ x, int k) {
    const float4* s = reinterpret_cast<const float4*>(x);
    float4* d = reinterpret_cast<float4*>(xs);
    for (int t = threadIdx.x; t < k / 4; t += blockDim.x) d[t] = s[t];
}

}  // namespace barq
