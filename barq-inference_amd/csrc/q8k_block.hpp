// The Q8_K block quantizer shared by the activation quantizers
// (quantize.hip) and the fused MoE grouping + gather (moe.hip).
#pragma once
#include "common.hpp"

namespace barq {

// Q8_K: one wave per 256-element block, 4 elements per lane.
// max = the signed value of the first element with the largest |x|;
// iscale = -127/max; q = min(127, rint(iscale*x)); d = 1/iscale;
// bsums[g] = sum of q[16g .. 16g+16).  An all-zero block stores zeros.
__device__ __forceinline__ void q8_k_block(const float (&vv)[4], int lane, uint8_t* __restrict__ blk) {
    float ba = 0.0f, bv = 0.0f;
    int bi = 0x7fffffff;
    #pragma unroll
    for (int j = 0; j < 4; j++) {
        const float ax = fabsf(vv[j]);
        if (ax > ba) { ba = ax; bv = vv[j]; bi = 4 * lane + j; }
    }
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(ba, off);
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (oa > ba || (oa == ba && oi < bi)) { ba = oa; bv = ov; bi = oi; }
    }
    if (ba == 0.0f) {
        reinterpret_cast<uint32_t*>(blk + 4)[lane] = 0u;
        if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(blk + 260 + 2 * (lane >> 2)) = 0;
        if (lane == 0) *reinterpret_cast<float*>(blk) = 0.0f;
        return;
    }
    const float iscale = -127.0f / bv;
    int q[4];
    #pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = (int)rintf(iscale * vv[j]);
        q[j] = t < 127 ? t : 127;
    }
    const uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                            ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    reinterpret_cast<uint32_t*>(blk + 4)[lane] = packed;
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(blk + 260 + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *reinterpret_cast<float*>(blk) = 1.0f / iscale;
}

}  // namespace barq
