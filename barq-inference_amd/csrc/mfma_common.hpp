// Helpers shared by the int8-MFMA GEMM kernels: raw buffer descriptors,
// buffer->LDS direct loads, explicit vmcnt waits and packed 16-bit multiply.
#pragma once
#include "common.hpp"

namespace barq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Two u16 lanes of a and s multiplied (low 16 bits each).  With bytes of a
// below 16 and s below 8 no product crosses a byte, so four byte-sized
// products are formed at once.
__device__ __forceinline__ uint32_t mul_u16x2(uint32_t a, uint32_t s) {
    const s16x2 r = __builtin_bit_cast(s16x2, a) * __builtin_bit_cast(s16x2, s);
    return __builtin_bit_cast(uint32_t, r);
}

// A raw buffer descriptor (base, byte limit; stride 0) as four SGPRs.  Reads
// at or beyond the limit return zero, which pads ragged row tiles.
__device__ __forceinline__ i32x4v make_rsrc4(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return i32x4v{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is written on purpose (the LDS destination)
// Buffer -> LDS direct loads: lane i's bytes land at the wave's LDS base +
// i * size (M0 holds the base).  Issued as inline asm so the compiler's
// wait-count insertion does not treat every in-flight stage as a pending
// write to the stage being read (it would drain them all); the kernels wait
// on their own loads with wait_vmcnt before each barrier.
__device__ __forceinline__ void lds_load16(i32x4v r, void* lds_wave_base, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(m0), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
// The same with the non-temporal hint (`nt`), for the streamed GEMV weight
// slices: measured on MI355X in one run, the 128256 x 4096 Q6_K GEMV 72.5 ->
// 67.6 us and the 4096 x 4096 Q4_0 GEMV 4.34 -> 4.08 us with it.  (The
// register GEMV, whose lanes re-read block headers, and the grouped GEMM
// measured slower with it.)
__device__ __forceinline__ void lds_load16_nt(i32x4v r, void* lds_wave_base, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :: "s"(m0), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
__device__ __forceinline__ void lds_load4(i32x4v r, void* lds_wave_base, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 :: "s"(m0), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
__device__ __forceinline__ void lds_load4_nt(i32x4v r, void* lds_wave_base, uint32_t voff, uint32_t soff) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen nt lds"
                 :: "s"(m0), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0) with the other counters left alone
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4));
}

}  // namespace barq
