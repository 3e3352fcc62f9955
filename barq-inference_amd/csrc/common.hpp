// Device-side helpers shared by the gfx950 kernels: block geometry, byte
// loads that tolerate the 2-byte alignment of GGUF blocks, f16 conversion
// and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

namespace barq {

// Launch-shape overrides for tuning sweeps (BARQ_GEMM_*, BARQ_GEMV_*,
// BARQ_MOE_*, BARQ_ATTN_*).  The environment is read once, when a handle is
// created (Tuning::from_env); every call made through that handle sees the
// same snapshot, so a launcher and the workspace sizing that precedes it
// cannot disagree, and no call reads the environment while another thread
// may be changing it.  Unset keeps the measured default.
enum Tune : int {
    TUNE_GEMM_BM, TUNE_GEMM_KG, TUNE_GEMM_NS, TUNE_GEMM_KS, TUNE_GEMM_XCD, TUNE_GEMM_IMPL, TUNE_GEMM_MIN_M,
    TUNE_GEMV_DMA, TUNE_GEMV_DMA_TYPES, TUNE_GEMV_MULTI_MAX, TUNE_GEMV_CFG_R, TUNE_GEMV_CFG_W,
    TUNE_MOE_GEMV, TUNE_MOE_FUSED_GROUP, TUNE_ATTN_WG, TUNE_GEMV_GLU, TUNE_GEMM_DEFER, TUNE_ATTN_MFMA_MIN_Q, TUNE_ATTN_MFMA_SPLIT, TUNE_GEMV_LDS, TUNE_COUNT
};

struct Tuning {
    bool set[TUNE_COUNT] = {};
    int val[TUNE_COUNT] = {};

    static Tuning from_env() {
        static const char* const names[TUNE_COUNT] = {
            "BARQ_GEMM_BM", "BARQ_GEMM_KG", "BARQ_GEMM_NS", "BARQ_GEMM_KS", "BARQ_GEMM_XCD", "BARQ_GEMM_IMPL",
            "BARQ_GEMM_MIN_M", "BARQ_GEMV_DMA", "BARQ_GEMV_DMA_TYPES", "BARQ_GEMV_MULTI_MAX", nullptr, nullptr,
            "BARQ_MOE_GEMV", "BARQ_MOE_FUSED_GROUP", "BARQ_ATTN_WG", "BARQ_GEMV_GLU", "BARQ_GEMM_DEFER", "BARQ_ATTN_MFMA_MIN_Q", "BARQ_ATTN_MFMA_SPLIT",
            "BARQ_GEMV_LDS"};
        Tuning t;
        for (int i = 0; i < TUNE_COUNT; i++) {
            if (!names[i]) continue;
            if (const char* e = getenv(names[i])) {
                t.set[i] = true;
                t.val[i] = atoi(e);
            }
        }
        // BARQ_GEMV_CFG = "R,W": rows per wave and waves per workgroup
        int r = 0, w = 0;
        if (const char* e = getenv("BARQ_GEMV_CFG"))
            if (sscanf(e, "%d,%d", &r, &w) == 2) {
                t.set[TUNE_GEMV_CFG_R] = t.set[TUNE_GEMV_CFG_W] = true;
                t.val[TUNE_GEMV_CFG_R] = r;
                t.val[TUNE_GEMV_CFG_W] = w;
            }
        return t;
    }
};

// The snapshot of the handle whose call is running on this thread (set by
// the C ABI entry points for the duration of a call; null: defaults).
inline thread_local const Tuning* t_tuning = nullptr;

inline int tuning_env(Tune key, int def = 0) {
    const Tuning* t = t_tuning;
    return t && t->set[key] ? t->val[key] : def;
}

struct TuningScope {
    const Tuning* prev;
    explicit TuningScope(const Tuning* t) : prev(t_tuning) { t_tuning = t; }
    ~TuningScope() { t_tuning = prev; }
    TuningScope(const TuningScope&) = delete;
    TuningScope& operator=(const TuningScope&) = delete;
};

// GGUF block geometry (barq_core/src/gguf.rs:168-186 block sizes; bytes
// from gguf.rs:529-530,645,747,854 and llama.cpp block_q4_0/block_q8_K).
constexpr int QK4_0 = 32, Q4_0_BYTES = 18;
constexpr int Q4_0_BARQ_BYTES = 20;
constexpr int Q4_K_BARQ_BYTES = 136;   // the quant crate's own Q4_K (quant/src/q4_k.rs)
constexpr int QK8_0 = 32, Q8_0_BYTES = 34;
constexpr int QK_K = 256, Q4_K_BYTES = 144, Q6_K_BYTES = 210, Q8_K_BYTES = 292;

constexpr int TYPE_F32 = 0, TYPE_F16 = 1, TYPE_Q4_0 = 2, TYPE_Q8_0 = 8,
              TYPE_Q4_K = 12, TYPE_Q6_K = 14, TYPE_Q8_K = 15,
              TYPE_Q4_0_BARQ = 0x10002, TYPE_Q4_K_BARQ = 0x1000C;

constexpr int WAVE = 64;

// IEEE binary16 -> binary32 (v_cvt_f32_f16: exact widening, as
// half::f16::to_f32 used at gguf.rs:661,763,768,869).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits);
    return (float)h;
}

// binary32 -> binary16, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// 16-byte vector with 4-byte alignment: global_load_dwordx4 needs only
// dword alignment on gfx9 family hardware.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ uint4 ld16_a4(const uint8_t* p) {
    u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes starting at a 2-byte aligned address p.  Reads only bytes in
// [floor4(p), p + 16): a dword-aligned 16-byte load plus, when p is not
// dword aligned, the 2 bytes at p+14, then a funnel shift.  Safe at the end
// of a block or buffer.
__device__ __forceinline__ uint4 ld16_a2(const uint8_t* p) {
    uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3u;
    const uint8_t* q = p - sh;
    uint4 a = ld16_a4(q);
    uint32_t e = *reinterpret_cast<const uint16_t*>(q + (sh ? 16 : 12));
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(a.y, a.x, sh);
    r.y = __builtin_amdgcn_alignbyte(a.z, a.y, sh);
    r.z = __builtin_amdgcn_alignbyte(a.w, a.z, sh);
    r.w = __builtin_amdgcn_alignbyte(e, a.w, sh);
    return r;
}

// 8 bytes at a 2-byte aligned address p, reading only [floor4(p), p + 8).
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {
    uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3u;
    const uint8_t* qb = p - sh;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(qb);
    uint32_t a0 = q[0], a1 = q[1];
    uint32_t e = *reinterpret_cast<const uint16_t*>(qb + (sh ? 8 : 4));
    uint2 r;
    r.x = __builtin_amdgcn_alignbyte(a1, a0, sh);
    r.y = __builtin_amdgcn_alignbyte(e, a1, sh);
    return r;
}

// sdot4: 4 x (i8 * i8) + acc  (v_dot4_i32_i8)
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int acc) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, acc, false);
}

// ---- wave64 reductions ----------------------------------------------------
// Sum over a row of 16 lanes with DPP (quad_perm, half-mirror, mirror); every
// lane of the row ends with the row's total.
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    return v;
}

// Sum R per-lane partials (one per row) over the 64 lanes with the gfx950
// lane-swap instructions: two rows fold into one register per swap, so R rows
// cost ~R/2 swaps + one 16-lane DPP reduction instead of R full reductions.
// Afterwards lane row_lane4(r) holds the total of row r.
__device__ __forceinline__ float swap32_add(float a, float b) {
    auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), false, false);
    // s[0] = [a lanes 0-31 | b lanes 0-31], s[1] = [a lanes 32-63 | b lanes 32-63]
    return __builtin_bit_cast(float, (int)s[0]) + __builtin_bit_cast(float, (int)s[1]);
}

// rows of 16 lanes: a = [a0 a1 a2 a3], b = [b0 b1 b2 b3] -> [a0+a1, b0+b1, a2+a3, b2+b3]
__device__ __forceinline__ float swap16_add(float a, float b) {
    auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), false, false);
    return __builtin_bit_cast(float, (int)s[0]) + __builtin_bit_cast(float, (int)s[1]);
}

// r -> lane holding its total after reduce4 (rows a,b,c,d -> 0, 32, 16, 48)
__host__ __device__ constexpr int row_lane4(int r) { return r == 0 ? 0 : r == 1 ? 32 : r == 2 ? 16 : 48; }

// Reduce up to four rows; unused rows pass 0.
__device__ __forceinline__ float reduce4(float a, float b, float c, float d) {
    const float ab = swap32_add(a, b);   // [a 32 | b 32]
    const float cd = swap32_add(c, d);   // [c 32 | d 32]
    const float v = swap16_add(ab, cd);     // rows of 16: a, c, b, d
    return row16_sum(v);
}

// Sum over aligned groups of N lanes (N = 8, 16 or 32); every lane of the
// group gets the sum.  Within a row of 16 lanes: quad swaps, then the
// half-row and row mirrors; across two rows: the gfx950 row swap.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 8 || N == 16 || N == 32, "groups of 8, 16 or 32 lanes");
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    if constexpr (N >= 16)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    if constexpr (N >= 32) v = swap16_add(v, v);
    return v;
}

// Maximum over aligned groups of N lanes, the same exchanges as group_sum.
template <int N>
__device__ __forceinline__ float group_max(float v) {
    static_assert(N == 8 || N == 16 || N == 32, "groups of 8, 16 or 32 lanes");
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true)));
    if constexpr (N >= 16)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true)));
    if constexpr (N >= 32) {
        auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
        v = fmaxf(__builtin_bit_cast(float, (int)a[0]), __builtin_bit_cast(float, (int)a[1]));
    }
    return v;
}

// Maximum over a row of 16 lanes with DPP (the exchanges of row16_sum).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true)));
    return v;
}

// Maximum over the whole wave, in every lane: row16_max, then the row and
// half-wave swaps (no LDS round trips).  Every lane must be active.
__device__ __forceinline__ float wave_max_all(float v) {
    v = row16_max(v);
    auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    v = fmaxf(__builtin_bit_cast(float, (int)a[0]), __builtin_bit_cast(float, (int)a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (int)b[0]), __builtin_bit_cast(float, (int)b[1]));
}

// Sum over the whole wave, in every lane, in a fixed order: row16_sum, then
// the row pairs, then the halves.  Every lane must be active.
__device__ __forceinline__ float wave_sum_all(float v) {
    v = row16_sum(v);
    v = swap16_add(v, v);
    return swap32_add(v, v);
}

// Lanes l < 32 get the value of lane l + 32 (one gfx950 half-wave swap, no
// LDS round trip); lanes l >= 32 keep their own.
__device__ __forceinline__ float upper_half(float v) {
    auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)s[1]);
}

// Integer sum over each aligned group of four lanes (quad permutes).
__device__ __forceinline__ int quad_isum(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
    return v;
}

}  // namespace barq
