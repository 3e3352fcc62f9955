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
    // the largest |x| of the block (DPP rows and lane swaps; NaN never wins:
    // fmaxf returns the other operand), then the first element holding it:
    // the lowest lane with such an element, and in that lane the lowest j
    float a = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
    const float ba = wave_max_all(fmaxf(a, 0.0f));
    const bool hit = fabsf(vv[0]) == ba || fabsf(vv[1]) == ba || fabsf(vv[2]) == ba || fabsf(vv[3]) == ba;
    const uint64_t lanes = __ballot(hit && ba != 0.0f);
    const float mine = fabsf(vv[0]) == ba ? vv[0] : fabsf(vv[1]) == ba ? vv[1] : fabsf(vv[2]) == ba ? vv[2] : vv[3];
    const float bv = lanes ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine),
                                                                                 (int)__builtin_ctzll(lanes)))
                           : 0.0f;
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
    const int s = quad_isum(q[0] + q[1] + q[2] + q[3]);
    if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(blk + 260 + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *reinterpret_cast<float*>(blk) = 1.0f / iscale;
}

}  // namespace barq
