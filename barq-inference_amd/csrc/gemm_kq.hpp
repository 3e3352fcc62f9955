#pragma once
// Batched K-quant x Q8_K GEMM on gfx950 int8 MFMA: Y[m, n] = sum_k X[m, k] W[n, k]
// for Q4_K and Q6_K weights (GGUF rows, blocks along k) and Q8_K activation
// rows.  This is the prefill path and the MoE expert-group path; a grouped
// launch covers every expert of a MoE step, reading each expert's row range
// from device-side offsets (no host round trip).
//
// Workgroup tile: BM activation rows x 128 weight rows.  Each wave owns a
// 32-column slice (and, with eight waves, half of the BM rows) and issues
// v_mfma_i32_32x32x32_i8, whose K = 32 covers one Q4_K sub-block or two Q6_K
// sub-blocks; every lane's 16 k-values belong to a single sub-block, so the
// sub-block scale can be folded into that lane's int8 operand:
//   Q4_K: s*q with s = 8*s1 + s0 (s1, s0 in [0, 7]): s1*q and s0*q are <= 105
//         and come from one packed 16-bit multiply per four weights; the mins
//         are a third pass against m_j broadcast over the sub-block.
//   Q6_K: w = s*(q - 32) in [-4064, 4096] = 256*h + l, h in [-16, 16] and l in
//         [-128, 127]: the two bytes of w + 128, the low one less 128.
// The integer results per super-block are exact; the f32 epilogue is
//   Q4_K: y += dx * (d * (8*Ch + Cl) - dmin * Cm)
//   Q6_K: y += dx * d * (256*Ch + Cl)
//
// Data movement: NS LDS stages, each one super-block of the tile, filled by
// buffer->LDS direct loads NS-1 super-blocks ahead of the MFMAs with one
// barrier per super-block.  Activation rows are stored with a 16-byte pad
// (272-byte rows: conflict-free fragment reads); Q6_K blocks are copied as the
// dword-aligned 224-byte window around each 210-byte block (the kernel needs
// an even number of super-blocks per row so that window offset is uniform),
// placed 240 bytes apart for the same reason.
#include "launch.hpp"
#include "mfma_common.hpp"

#include <atomic>
#include <cstdlib>
#include <utility>

namespace barq {

constexpr int KQ_BN = 128;       // weight rows per workgroup
constexpr int KQ_MAXE = 64;      // expert weight pointers carried by a grouped launch

struct KQWeights {
    const uint8_t* w[KQ_MAXE];
};

// XC: 16-byte chunks per staged activation row: the 256 quants, for Q4_K the
// 16 bsums (sub-block sums for the mins), and one pad chunk that keeps rows
// of a 32-row fragment read on distinct LDS banks.  A staged weight row is
// PIECES 16-byte chunks (RS bytes), of which the first WP come from memory.
// Q6_K rows carry one pad chunk (a second copy of chunk 13): at the 224-byte
// stride lanes n and n + 4 of a fragment read start on the same bank, which
// measured as LDS bank conflicts in 69 % of the grouped down projection's LDS
// cycles; 240 bytes (60 dwords) puts the eight lanes of each read phase on
// distinct banks.
struct KQ4 {
    static constexpr int TYPE = TYPE_Q4_K, BB = Q4_K_BYTES, RS = 144, PIECES = 9, WP = 9, XC = 19, XRS = 16 * XC;
    static __device__ __forceinline__ uint32_t soff(int b) { return (uint32_t)b * 144u; }
};
struct KQ6 {
    static constexpr int TYPE = TYPE_Q6_K, BB = Q6_K_BYTES, RS = 240, PIECES = 15, WP = 14, XC = 17, XRS = 16 * XC;
    // the dword-aligned start of block b's window (row bytes are a multiple of 4)
    static __device__ __forceinline__ uint32_t soff(int b) { return (uint32_t)b * 210u & ~3u; }
};

// LDS stage layout and per-wave load counts
template <class F, int BM, int NW>
struct KQL {
    static constexpr int X_CHUNKS = BM * F::XC;                // activation rows in 16-byte chunks
    static constexpr int X_INSTR_ALL = (X_CHUNKS + 63) / 64;
    static constexpr int XQ = 0;
    static constexpr int W = X_INSTR_ALL * 1024;
    static constexpr int W_INSTR_ALL = KQ_BN * F::PIECES / 64;
    static constexpr int XD = W + KQ_BN * F::RS;
    static constexpr int XD_LOADS = BM < 64 ? 1 : BM / 64;
    static constexpr int STAGE = XD + XD_LOADS * 256;
    static constexpr int X_INSTR = (X_INSTR_ALL + NW - 1) / NW;
    static constexpr int W_INSTR = (W_INSTR_ALL + NW - 1) / NW;
    static constexpr int LOADS_MIN = X_INSTR_ALL / NW + W_INSTR_ALL / NW;
    static constexpr int LOADS_MIN_W = W_INSTR_ALL / NW;   // when activation loads may be skipped
    // 32x32 MFMA row tiles per wave; 16-row tiles use the 16x16 path (two column blocks per wave)
    static constexpr int MTW = BM >= 32 ? BM / 32 / (NW / 4) : 1;
    static_assert(KQ_BN * F::PIECES % 64 == 0, "weight tile is whole load instructions");
    static_assert(F::RS == 16 * F::PIECES, "weight rows are whole chunks");
};

template <class F, int BM, int NW>
struct KQOff {
    uint32_t x[KQL<F, BM, NW>::X_INSTR];
    uint32_t w[KQL<F, BM, NW>::W_INSTR];
    uint32_t xd;
};

template <class F, int BM, int NW>
__device__ __forceinline__ void kq_offsets(KQOff<F, BM, NW>& o, uint32_t xrb, uint32_t wrb, int wave, int l) {
    using L = KQL<F, BM, NW>;
    #pragma unroll
    for (int q = 0; q < L::X_INSTR; q++) {
        const int p = (q * NW + wave) * 64 + l, r = p / F::XC, c = p - r * F::XC;
        // quants at 4 + 16c, bsums at 260 + 16 (c - 16); the pad chunk reloads chunk 0
        o.x[q] = (uint32_t)r * xrb + 4u + 16u * (uint32_t)(c < F::XC - 1 ? c : 0);
    }
    #pragma unroll
    for (int q = 0; q < L::W_INSTR; q++) {
        const int p = (q * NW + wave) * 64 + l, row = p / F::PIECES, piece = p - row * F::PIECES;
        o.w[q] = (uint32_t)row * wrb + 16u * (uint32_t)(piece < F::WP ? piece : F::WP - 1);
    }
    o.xd = (uint32_t)(64 * wave + l) * xrb;
}

// x_instr: activation load instructions to issue (fewer when the tile has
// fewer rows; the rows left out keep stale bytes whose results are never
// stored, and their dx loads as zero).
template <class F, int BM, int NW>
__device__ __forceinline__ void kq_issue(uint8_t* stage, i32x4v xr, i32x4v wr, const KQOff<F, BM, NW>& o, int b,
                                         int wave, int x_instr = KQL<F, BM, NW>::X_INSTR_ALL) {
    using L = KQL<F, BM, NW>;
    const uint32_t xs = (uint32_t)b * Q8_K_BYTES, ws = F::soff(b);
    #pragma unroll
    for (int q = 0; q < L::X_INSTR; q++) {
        const int idx = q * NW + wave;
        if (idx < x_instr) lds_load16(xr, stage + L::XQ + 1024 * idx, o.x[q], xs);
    }
    #pragma unroll
    for (int q = 0; q < L::W_INSTR; q++) {
        const int idx = q * NW + wave;
        if (idx < L::W_INSTR_ALL) lds_load16(wr, stage + L::W + 1024 * idx, o.w[q], ws);
    }
    if (wave < L::XD_LOADS) lds_load4(xr, stage + L::XD + 256 * wave, o.xd, xs);
}

// dx of the lane's 16 output rows of tile t (32x32 C layout: lane (n, g2),
// register r -> row 8*(r/4) + 4*g2 + r%4)
template <int MT>
__device__ __forceinline__ void kq_dx(const uint8_t* xd, int mbase, int g2, float (&dx)[MT][16]) {
    #pragma unroll
    for (int t = 0; t < MT; t++)
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = *reinterpret_cast<const float4*>(xd + 4 * (mbase + 32 * t + 8 * q + 4 * g2));
            dx[t][4 * q] = v.x; dx[t][4 * q + 1] = v.y; dx[t][4 * q + 2] = v.z; dx[t][4 * q + 3] = v.w;
        }
}

// ---- Q4_K super-block --------------------------------------------------------
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Eight signed 16-bit values as f16 (exact: |bsum| <= 16 * 128)
__device__ __forceinline__ h8 i16x8_to_h8(uint4 w) {
    h8 r;
    r[0] = (_Float16)(short)(w.x & 0xFFFFu); r[1] = (_Float16)(short)(w.x >> 16);
    r[2] = (_Float16)(short)(w.y & 0xFFFFu); r[3] = (_Float16)(short)(w.y >> 16);
    r[4] = (_Float16)(short)(w.z & 0xFFFFu); r[5] = (_Float16)(short)(w.z >> 16);
    r[6] = (_Float16)(short)(w.w & 0xFFFFu); r[7] = (_Float16)(short)(w.w >> 16);
    return r;
}

// A Q4_K super-block between its MFMAs and its f32 epilogue: the two scale
// passes' integer sums, the mins sums and the block's d / dmin (this lane's
// weight row).
template <int MT>
struct KQ4Part {
    v16i ch[MT], cl[MT];
    f32x16 cm[MT];
    float d, dmin;
};

template <int MT>
__device__ __forceinline__ void kq4_mma(const uint8_t* wrow, const uint8_t* xrow, int g2, KQ4Part<MT>& p) {
    constexpr int XRS = KQ4::XRS;
    const uint4 hdr = *reinterpret_cast<const uint4*>(wrow);
    p.d = f16_bits_to_f32(hdr.x & 0xFFFFu);
    p.dmin = f16_bits_to_f32(hdr.x >> 16);
    // kept as an f32 register: folded into the epilogue's 32 FMAs the
    // conversion becomes v_fma_mix_f32, which issues slower than v_fma_f32
    asm volatile("" : "+v"(p.dmin));
    // get_scale_min_k4 (gguf.rs:825-837) for the eight sub-blocks, bytewise
    const uint32_t scA = hdr.y & 0x3F3F3F3Fu;
    const uint32_t scB = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
    const uint32_t mA = hdr.z & 0x3F3F3F3Fu;
    const uint32_t mB = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
    const uint32_t s1A = (scA >> 3) & 0x07070707u, s0A = scA & 0x07070707u;
    const uint32_t s1B = (scB >> 3) & 0x07070707u, s0B = scB & 0x07070707u;
    // Mins: sum_j m_j * (sum of x over sub-block j) as one f16 MFMA with
    // K = the 16 bsums: lane group g2 holds bsums 8 g2 .. 8 g2 + 7, i.e. both
    // halves of sub-blocks 4 g2 .. 4 g2 + 3, against m of those sub-blocks.
    // Every value and partial sum is an integer below 2^24: exact in f32.
    const uint32_t mm = g2 ? mB : mA;
    h8 bmin;
    #pragma unroll
    for (int q = 0; q < 4; q++) {
        const _Float16 m = (_Float16)(float)((mm >> (8 * q)) & 0xFFu);
        bmin[2 * q] = m;
        bmin[2 * q + 1] = m;
    }
    #pragma unroll
    for (int t = 0; t < MT; t++) {
        const h8 amin = i16x8_to_h8(*reinterpret_cast<const uint4*>(xrow + 32 * t * XRS + 256));
        const f32x16 z = {};
        p.cm[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(amin, bmin, z, 0, 0, 0);
    }
    #pragma unroll
    for (int pr = 0; pr < 4; pr++) {
        // sub-blocks 2pr (low nibbles) and 2pr+1 (high nibbles) share qs[32pr + 16g2 .. +16)
        const uint4 qs = *reinterpret_cast<const uint4*>(wrow + 16 + 32 * pr + 16 * g2);
        #pragma unroll
        for (int h = 0; h < 2; h++) {
            const int j = 2 * pr + h;
            const uint32_t bsel = (uint32_t)(j & 3);
            const uint32_t s1 = __builtin_amdgcn_perm(0u, j < 4 ? s1A : s1B, 0x0c000c00u | (bsel << 16) | bsel);
            const uint32_t s0 = __builtin_amdgcn_perm(0u, j < 4 ? s0A : s0B, 0x0c000c00u | (bsel << 16) | bsel);
            const uint32_t n0 = (qs.x >> (4 * h)) & 0x0F0F0F0Fu, n1 = (qs.y >> (4 * h)) & 0x0F0F0F0Fu;
            const uint32_t n2 = (qs.z >> (4 * h)) & 0x0F0F0F0Fu, n3 = (qs.w >> (4 * h)) & 0x0F0F0F0Fu;
            const v4i bh = {(int)mul_u16x2(n0, s1), (int)mul_u16x2(n1, s1), (int)mul_u16x2(n2, s1), (int)mul_u16x2(n3, s1)};
            const v4i bl = {(int)mul_u16x2(n0, s0), (int)mul_u16x2(n1, s0), (int)mul_u16x2(n2, s0), (int)mul_u16x2(n3, s0)};
            #pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i a = *reinterpret_cast<const v4i*>(xrow + 32 * t * XRS + 32 * j);
                const v16i z = {};
                p.ch[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bh, j ? p.ch[t] : z, 0, 0, 0);
                p.cl[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bl, j ? p.cl[t] : z, 0, 0, 0);
            }
        }
    }
}

template <int MT>
__device__ __forceinline__ void kq4_epilogue(const KQ4Part<MT>& p, const float (&dx)[MT][16], float (&acc)[MT][16]) {
    #pragma unroll
    for (int t = 0; t < MT; t++)
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            const int c = (p.ch[t][r] << 3) + p.cl[t][r];
            const float v = __builtin_fmaf(-p.dmin, p.cm[t][r], p.d * (float)c);
            acc[t][r] = __builtin_fmaf(dx[t][r], v, acc[t][r]);
        }
}

template <int MT>
__device__ __forceinline__ void kq4_compute(const uint8_t* wrow, const uint8_t* xrow, const uint8_t* xd, int mbase,
                                            int g2, float (&acc)[MT][16]) {
    KQ4Part<MT> p;
    kq4_mma<MT>(wrow, xrow, g2, p);
    float dx[MT][16];
    kq_dx<MT>(xd, mbase, g2, dx);
    kq4_epilogue<MT>(p, dx, acc);
}

// ---- Q6_K super-block --------------------------------------------------------
// 16 bytes at p + sh (p 16-byte aligned, sh in {0, 2}) from an aligned 16-byte
// read and the following dword
__device__ __forceinline__ uint4 lds16_sh(const uint8_t* p, uint32_t sh) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(p + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                      __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh));
}

// Four 6-bit quants q (bytes of q4) -> bytes of h and l with s*(q-32) = 256*h + l.
// Each 16-bit lane holds w' = s*(q-32) + 128 (off = 128 - 32 s; |w'| < 2^15, so
// the packed multiply-add's low 16 bits are exact): h is its high byte (w' >> 8),
// l its low byte less 128 (the byte with the top bit flipped, read as int8).
__device__ __forceinline__ void q6_split4(uint32_t q4, uint32_t scv, uint32_t off, int& h, int& l) {
    const uint32_t a = mul_u16x2(__builtin_amdgcn_perm(0u, q4, 0x0c010c00u), scv);
    const uint32_t c = mul_u16x2(__builtin_amdgcn_perm(0u, q4, 0x0c030c02u), scv);
    const uint32_t wa = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, a) + __builtin_bit_cast(s16x2, off));
    const uint32_t wc = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, c) + __builtin_bit_cast(s16x2, off));
    h = (int)__builtin_amdgcn_perm(wc, wa, 0x07050301u);
    l = (int)(__builtin_amdgcn_perm(wc, wa, 0x06040200u) ^ 0x80808080u);
}

template <int MT>
__device__ __forceinline__ void kq6_compute(const uint8_t* wrow, const uint8_t* xrow, const uint8_t* xd, int mbase,
                                            int g2, int b, float (&acc)[MT][16]) {
    // the block starts sh bytes into the copied window (gguf.rs:839-914 layout:
    // ql[128] @0, qh[64] @128, scales[16] @192, d @208)
    const uint32_t sh = 2u * (uint32_t)(b & 1);
    const uint32_t dw = *reinterpret_cast<const uint32_t*>(wrow + 208);
    const float d = f16_bits_to_f32(sh ? dw >> 16 : dw & 0xFFFFu);
    v16i ch[MT], cl[MT];
    #pragma unroll
    for (int half = 0; half < 2; half++) {
        // element 32j + 16g2 + i: half = j/4, quarter qd = j%4, position l = 16g2 + i
        const uint4 qh = lds16_sh(wrow + 128 + 32 * half + 16 * g2, sh);
        #pragma unroll
        for (int odd = 0; odd < 2; odd++) {
            const uint4 ql = lds16_sh(wrow + 64 * half + 32 * odd + 16 * g2, sh);
            #pragma unroll
            for (int hi = 0; hi < 2; hi++) {
                const int qd = 2 * hi + odd, j = 4 * half + qd;
                const int sc = (int)(int8_t)wrow[sh + 192 + 8 * half + g2 + 2 * qd];
                const uint32_t scv = ((uint32_t)sc & 0xFFFFu) * 0x00010001u;
                const uint32_t off = ((uint32_t)(128 - 32 * sc) & 0xFFFFu) * 0x00010001u;
                const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w}, qhw[4] = {qh.x, qh.y, qh.z, qh.w};
                int hv[4], lv[4];
                #pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t q4 = ((qlw[i] >> (4 * hi)) & 0x0F0F0F0Fu) | (((qhw[i] >> (2 * qd)) & 0x03030303u) << 4);
                    q6_split4(q4, scv, off, hv[i], lv[i]);
                }
                const v4i bh = {hv[0], hv[1], hv[2], hv[3]}, bl = {lv[0], lv[1], lv[2], lv[3]};
                #pragma unroll
                for (int t = 0; t < MT; t++) {
                    const v4i a = *reinterpret_cast<const v4i*>(xrow + 32 * t * KQ6::XRS + 32 * j);
                    const v16i z = {};
                    ch[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bh, j ? ch[t] : z, 0, 0, 0);
                    cl[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bl, j ? cl[t] : z, 0, 0, 0);
                }
            }
        }
    }
    float dx[MT][16];
    kq_dx<MT>(xd, mbase, g2, dx);
    #pragma unroll
    for (int t = 0; t < MT; t++)
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            const int c = (ch[t][r] << 8) + cl[t][r];
            acc[t][r] = __builtin_fmaf(dx[t][r], d * (float)c, acc[t][r]);
        }
}

// ---- 16-row tiles (v_mfma_i32_16x16x64_i8) ------------------------------------
// For expert groups of a few tokens: a wave covers 16 rows x 32 columns as two
// 16x16 column blocks.  16x16x64 layout: lane (row/column l % 16, k group
// g4 = l / 16: k = 16 g4 .. 16 g4 + 15 of each 64); C: rows 4 g4 + r, column
// l % 16.  A lane's 16 k-values lie in one Q4_K sub-block (32) or one Q6_K
// sub-block (16), so the scales still fold into its B operand.
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void kq16_dx(const uint8_t* xd, int g4, float (&dx)[4]) {
    const float4 v = *reinterpret_cast<const float4*>(xd + 16 * g4);
    dx[0] = v.x; dx[1] = v.y; dx[2] = v.z; dx[3] = v.w;
}

// acc[0][4 cb + r]: column block cb, row 4 g4 + r
__device__ __forceinline__ void kq4_compute16(const uint8_t* st, int wave, int l, float (&acc)[1][16]) {
    using L = KQL<KQ4, 16, 4>;
    const int n = l & 15, g4 = l >> 4;
    const uint8_t* xrow = st + L::XQ + n * KQ4::XRS + 16 * g4;
    // A fragments for the four k-steps and the bsums (mins)
    v4i a[4];
    #pragma unroll
    for (int t = 0; t < 4; t++) a[t] = *reinterpret_cast<const v4i*>(xrow + 64 * t);
    h8v amin;
    {
        const uint4 bs = *reinterpret_cast<const uint4*>(st + L::XQ + n * KQ4::XRS + 256 + 16 * (g4 & 1));
        amin = i16x8_to_h8(bs);
        if (g4 >= 2) amin = h8v{};
    }
    float dx[4];
    kq16_dx(st + L::XD, g4, dx);
    #pragma unroll
    for (int cb = 0; cb < 2; cb++) {
        const uint8_t* wrow = st + L::W + (32 * wave + 16 * cb + n) * KQ4::RS;
        const uint4 hdr = *reinterpret_cast<const uint4*>(wrow);
        const float d = f16_bits_to_f32(hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(hdr.x >> 16);
        const uint32_t scA = hdr.y & 0x3F3F3F3Fu;
        const uint32_t scB = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        const uint32_t mA = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mB = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        // mins: k = bsum index for g4 < 2 (sub-block k / 2), zero above
        h8v bmin = {};
        if (g4 < 2) {
            const uint32_t mm = g4 ? mB : mA;
            #pragma unroll
            for (int q = 0; q < 4; q++) {
                const _Float16 m = (_Float16)(float)((mm >> (8 * q)) & 0xFFu);
                bmin[2 * q] = m;
                bmin[2 * q + 1] = m;
            }
        }
        const f32x4 zf = {};
        const f32x4 cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin, bmin, zf, 0, 0, 0);
        v4i ch = {}, cl = {};
        #pragma unroll
        for (int t = 0; t < 4; t++) {
            // k-step t: sub-block j = 2t + g4 / 2 from qs[32t + 16 (g4 & 1) ..], nibble g4 / 2
            const uint4 qs = *reinterpret_cast<const uint4*>(wrow + 16 + 32 * t + 16 * (g4 & 1));
            const int hsh = 4 * (g4 >> 1);
            const uint32_t bsel = (uint32_t)(2 * t + (g4 >> 1)) & 3u;
            const uint32_t scw = t < 2 ? scA : scB;
            const uint32_t s1 = __builtin_amdgcn_perm(0u, (scw >> 3) & 0x07070707u, 0x0c000c00u | (bsel << 16) | bsel);
            const uint32_t s0 = __builtin_amdgcn_perm(0u, scw & 0x07070707u, 0x0c000c00u | (bsel << 16) | bsel);
            const uint32_t n0 = (qs.x >> hsh) & 0x0F0F0F0Fu, n1 = (qs.y >> hsh) & 0x0F0F0F0Fu;
            const uint32_t n2 = (qs.z >> hsh) & 0x0F0F0F0Fu, n3 = (qs.w >> hsh) & 0x0F0F0F0Fu;
            const v4i bh = {(int)mul_u16x2(n0, s1), (int)mul_u16x2(n1, s1), (int)mul_u16x2(n2, s1), (int)mul_u16x2(n3, s1)};
            const v4i bl = {(int)mul_u16x2(n0, s0), (int)mul_u16x2(n1, s0), (int)mul_u16x2(n2, s0), (int)mul_u16x2(n3, s0)};
            ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], bh, ch, 0, 0, 0);
            cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], bl, cl, 0, 0, 0);
        }
        #pragma unroll
        for (int r = 0; r < 4; r++) {
            const int c = (ch[r] << 3) + cl[r];
            const float v = __builtin_fmaf(-dmin, cm[r], d * (float)c);
            acc[0][4 * cb + r] = __builtin_fmaf(dx[r], v, acc[0][4 * cb + r]);
        }
    }
}

__device__ __forceinline__ void kq6_compute16(const uint8_t* st, int wave, int l, int b, float (&acc)[1][16]) {
    using L = KQL<KQ6, 16, 4>;
    const int n = l & 15, g4 = l >> 4;
    const uint8_t* xrow = st + L::XQ + n * KQ6::XRS + 16 * g4;
    v4i a[4];
    #pragma unroll
    for (int t = 0; t < 4; t++) a[t] = *reinterpret_cast<const v4i*>(xrow + 64 * t);
    float dx[4];
    kq16_dx(st + L::XD, g4, dx);
    const uint32_t sh = 2u * (uint32_t)(b & 1);
    #pragma unroll
    for (int cb = 0; cb < 2; cb++) {
        const uint8_t* wrow = st + L::W + (32 * wave + 16 * cb + n) * KQ6::RS;
        const uint32_t dw = *reinterpret_cast<const uint32_t*>(wrow + 208);
        const float d = f16_bits_to_f32(sh ? dw >> 16 : dw & 0xFFFFu);
        v4i ch = {}, cl = {};
        #pragma unroll
        for (int t = 0; t < 4; t++) {
            // element 64t + 16 g4 + i = 128 half + 32 qd + l: half = t / 2,
            // qd = 2 (t & 1) + g4 / 2, l = 16 (g4 & 1) + i
            const int half = t >> 1, qd = 2 * (t & 1) + (g4 >> 1);
            const uint4 ql = lds16_sh(wrow + 64 * half + 32 * (g4 >> 1) + 16 * (g4 & 1), sh);
            const uint4 qh = lds16_sh(wrow + 128 + 32 * half + 16 * (g4 & 1), sh);
            const int sc = (int)(int8_t)wrow[sh + 192 + 8 * half + (g4 & 1) + 2 * qd];
            const uint32_t scv = ((uint32_t)sc & 0xFFFFu) * 0x00010001u;
            const uint32_t off = ((uint32_t)(128 - 32 * sc) & 0xFFFFu) * 0x00010001u;
            const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w}, qhw[4] = {qh.x, qh.y, qh.z, qh.w};
            const int lsh = 4 * (t & 1), hsh = 2 * qd;
            int hv[4], lv[4];
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t q4 = ((qlw[i] >> lsh) & 0x0F0F0F0Fu) | (((qhw[i] >> hsh) & 0x03030303u) << 4);
                q6_split4(q4, scv, off, hv[i], lv[i]);
            }
            const v4i bh = {hv[0], hv[1], hv[2], hv[3]}, bl = {lv[0], lv[1], lv[2], lv[3]};
            ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], bh, ch, 0, 0, 0);
            cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], bl, cl, 0, 0, 0);
        }
        #pragma unroll
        for (int r = 0; r < 4; r++) {
            const int c = (ch[r] << 8) + cl[r];
            acc[0][4 * cb + r] = __builtin_fmaf(dx[r], d * (float)c, acc[0][4 * cb + r]);
        }
    }
}

// ---- pipeline ----------------------------------------------------------------
// Super-block b (32-row MFMA tiles) from its weight rows ws, activation rows
// xs and activation scales xd in LDS into the accumulators (b's parity places
// the Q6_K windows).
template <class F, int BM, int NW>
__device__ __forceinline__ void kq_compute_parts(const uint8_t* ws, const uint8_t* xs, const uint8_t* xd, int b,
                                                 int wave, int l, float (&acc)[KQL<F, BM, NW>::MTW][16]) {
    constexpr int MT = KQL<F, BM, NW>::MTW;
    const int n = l & 31, g2 = l >> 5;
    const int slice = wave & 3, mbase = 32 * MT * (wave >> 2);   // eight waves: two per column slice
    const uint8_t* wrow = ws + (32 * slice + n) * F::RS;
    const uint8_t* xrow = xs + (mbase + n) * F::XRS + 16 * g2;
    if constexpr (F::TYPE == TYPE_Q4_K) kq4_compute<MT>(wrow, xrow, xd, mbase, g2, acc);
    else kq6_compute<MT>(wrow, xrow, xd, mbase, g2, b, acc);
}

// Super-block b of the tile from one LDS stage into the accumulators.
template <class F, int BM, int NW>
__device__ __forceinline__ void kq_compute(const uint8_t* st, int b, int wave, int l,
                                           float (&acc)[KQL<F, BM, NW>::MTW][16]) {
    using L = KQL<F, BM, NW>;
    if constexpr (BM == 16) {
        if constexpr (F::TYPE == TYPE_Q4_K) kq4_compute16(st, wave, l, acc);
        else kq6_compute16(st, wave, l, b, acc);
    } else {
        kq_compute_parts<F, BM, NW>(st + L::W, st + L::XQ, st + L::XD, b, wave, l, acc);
    }
}

// One step: super-block b computed from stage S (= b % NS) while the loads of
// b+NS-1 go to stage (S-1) % NS.  Each stage is its own LDS array; the raw
// s_barrier (no memory fence) does not drain the in-flight stages.
constexpr int KQ_MAX_NS = 6;

// With KG K-groups a stage holds KG consecutive super-blocks, one per group:
// group kg (its own NW waves, `wave` counted within the group) loads and
// computes super-block KG * b + kg of step b.
template <class F, int BM, int NW, int NS, int KG, int S>
__device__ __forceinline__ void kq_step(uint8_t* const (&stages)[KQ_MAX_NS], int b, int nst, i32x4v xr, i32x4v wr,
                                        const KQOff<F, BM, NW>& off, int kg, int wave, int l,
                                        float (&acc)[KQL<F, BM, NW>::MTW][16]) {
    using L = KQL<F, BM, NW>;
    if (b >= nst) return;
    // this thread's loads of step b are done once at most the later
    // stages' loads are outstanding; every thread's are after the barrier
    if (b + NS - 2 < nst) wait_vmcnt<(NS - 2) * L::LOADS_MIN>();
    else wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int sub = kg * L::STAGE;
    if (b + NS - 1 < nst)
        kq_issue<F, BM, NW>(stages[(S + NS - 1) % NS] + sub, xr, wr, off, KG * (b + NS - 1) + kg, wave);
    kq_compute<F, BM, NW>(stages[S] + sub, KG * b + kg, wave, l, acc);
}

// The Q4_K two-K-group step with group 1's epilogue deferred: group 0 runs
// MFMAs then its epilogue, group 1 first the epilogue of its previous
// super-block (kept in registers with its activation scales) and then its
// MFMAs, so on each SIMD one group's f32 epilogue runs beside the other
// group's MFMAs.  The dx reads of every wave have landed before the barrier
// (lgkmcnt 0), because the next loads into the stage are issued after it.
template <int BM, int NW, int NS, int S>
__device__ __forceinline__ void kq4_step_defer(uint8_t* const (&stages)[KQ_MAX_NS], int b, int nst, i32x4v xr,
                                               i32x4v wr, const KQOff<KQ4, BM, NW>& off, int kg, int wave, int l,
                                               KQ4Part<KQL<KQ4, BM, NW>::MTW>& part,
                                               float (&dxs)[KQL<KQ4, BM, NW>::MTW][16],
                                               float (&acc)[KQL<KQ4, BM, NW>::MTW][16]) {
    using L = KQL<KQ4, BM, NW>;
    constexpr int MT = L::MTW;
    if (b >= nst) return;
    if (b + NS - 2 < nst) wait_vmcnt<(NS - 2) * L::LOADS_MIN>();
    else wait_vmcnt<0>();
    wait_lgkmcnt0();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int sub = kg * L::STAGE;
    const int n = l & 31, g2 = l >> 5;
    const int slice = wave & 3, mbase = 32 * MT * (wave >> 2);
    const uint8_t* st = stages[S] + sub;
    if (kg == 1 && b > 0) kq4_epilogue<MT>(part, dxs, acc);
    if (b + NS - 1 < nst) kq_issue<KQ4, BM, NW>(stages[(S + NS - 1) % NS] + sub, xr, wr, off, 2 * (b + NS - 1) + kg, wave);
    kq4_mma<MT>(st + L::W + (32 * slice + n) * KQ4::RS, st + L::XQ + (mbase + n) * KQ4::XRS + 16 * g2, g2, part);
    kq_dx<MT>(st + L::XD, mbase, g2, dxs);
    if (kg == 0) kq4_epilogue<MT>(part, dxs, acc);
}

template <int BM, int NW, int NS, int... S>
__device__ __forceinline__ void kq4_round_defer(std::integer_sequence<int, S...>, uint8_t* const (&stages)[KQ_MAX_NS],
                                                int b, int nst, i32x4v xr, i32x4v wr, const KQOff<KQ4, BM, NW>& off,
                                                int kg, int wave, int l, KQ4Part<KQL<KQ4, BM, NW>::MTW>& part,
                                                float (&dxs)[KQL<KQ4, BM, NW>::MTW][16],
                                                float (&acc)[KQL<KQ4, BM, NW>::MTW][16]) {
    (kq4_step_defer<BM, NW, NS, S>(stages, b + S, nst, xr, wr, off, kg, wave, l, part, dxs, acc), ...);
}

// One BM x 128 output tile: rows [m0, m0 + BM) of the `count` activation rows
// at X (row bytes xrb) against weight rows [n0, n0 + 128) of W; results to
// Y[row * N + col].  All waves of the workgroup call it with the same values.
// NS consecutive steps (one per stage), unrolled so that stage indices are constants
template <class F, int BM, int NW, int NS, int KG, int... S>
__device__ __forceinline__ void kq_round(std::integer_sequence<int, S...>, uint8_t* const (&stages)[KQ_MAX_NS], int b,
                                         int nst, i32x4v xr, i32x4v wr, const KQOff<F, BM, NW>& off, int kg, int wave,
                                         int l, float (&acc)[KQL<F, BM, NW>::MTW][16]) {
    (kq_step<F, BM, NW, NS, KG, S>(stages, b + S, nst, xr, wr, off, kg, wave, l, acc), ...);
}

// Tile results to Y[row * N + col] for rows < count and columns < N, with
// non-temporal stores: lines the next kernel reads from memory anyway are
// not left dirty in L2 (measured: C4 25.6-26.8 against 27.2-28.1 us, the
// prefill layer 452-454 against 461-463 us, C5 231 against 234-237 us).
template <class F, int BM, int NW>
__device__ __forceinline__ void kq_store(const float (&acc)[KQL<F, BM, NW>::MTW][16], float* Y, int count, int N,
                                         int m0, int n0, int wave, int l) {
    constexpr int MT = KQL<F, BM, NW>::MTW;
    if constexpr (BM == 16) {
        #pragma unroll
        for (int cb = 0; cb < 2; cb++) {
            const int col = n0 + 32 * wave + 16 * cb + (l & 15);
            if (col < N) {
                #pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = m0 + 4 * (l >> 4) + r;
                    if (row < count) __builtin_nontemporal_store(acc[0][4 * cb + r], &Y[(size_t)row * N + col]);
                }
            }
        }
        return;
    }
    const int col = n0 + 32 * (wave & 3) + (l & 31), g2 = l >> 5, mb = 32 * MT * (wave >> 2);
    if (col < N) {
        #pragma unroll
        for (int t = 0; t < MT; t++)
            #pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + mb + 32 * t + 8 * (r >> 2) + 4 * g2 + (r & 3);
                if (row < count) __builtin_nontemporal_store(acc[t][r], &Y[(size_t)row * N + col]);
            }
    }
}

// K-group kg > 0 hands its partial sums to group 0 through LDS (stage 0,
// free once every wave has passed the first barrier); group 0 adds them in
// group order.
template <class F, int BM, int NW, int KG>
__device__ __forceinline__ void kq_reduce_groups(uint8_t* lds, float (&acc)[KQL<F, BM, NW>::MTW][16], int kg, int wave,
                                                 int l) {
    constexpr int MT = KQL<F, BM, NW>::MTW, LANES = 64 * NW;
    static_assert((KG - 1) * MT * 16 * LANES * 4 <= KG * KQL<F, BM, NW>::STAGE, "reduction fits stage 0");
    float* red = reinterpret_cast<float*>(lds);
    const int lane = 64 * wave + l;
    __syncthreads();
    if (kg > 0) {
        #pragma unroll
        for (int t = 0; t < MT; t++)
            #pragma unroll
            for (int r = 0; r < 16; r++) red[((kg - 1) * MT * 16 + 16 * t + r) * LANES + lane] = acc[t][r];
    }
    __syncthreads();
    if (kg == 0) {
        #pragma unroll
        for (int g = 1; g < KG; g++)
            #pragma unroll
            for (int t = 0; t < MT; t++)
                #pragma unroll
                for (int r = 0; r < 16; r++) acc[t][r] += red[((g - 1) * MT * 16 + 16 * t + r) * LANES + lane];
    }
}

template <class F, int BM, int NS, int NW, int KG, bool DEFER = false>
__device__ __forceinline__ void kq_tile(uint8_t* const (&stages)[KQ_MAX_NS], const uint8_t* W, uint32_t wrb, const uint8_t* X,
                                        uint32_t xrb, float* Y, int count, int N, int nsb, int m0, int n0, int kg,
                                        int wave, int l, int kb0 = 0) {
    using L = KQL<F, BM, NW>;
    constexpr int MT = L::MTW;
    const int nst = nsb / KG;   // steps (nsb is a multiple of KG)
    // super-blocks [kb0, kb0 + nsb) of each row (kb0 even: Q6_K windows keep their parity)
    const uint32_t xk = (uint32_t)kb0 * Q8_K_BYTES, wk = (uint32_t)kb0 * F::BB;
    const i32x4v xr = make_rsrc4(X + (size_t)m0 * xrb + xk, (uint32_t)((size_t)(count - m0) * xrb) - xk);
    const i32x4v wr = make_rsrc4(W + (size_t)n0 * wrb + wk, (uint32_t)((size_t)(N - n0) * wrb) - wk);

    float acc[MT][16];
    #pragma unroll
    for (int t = 0; t < MT; t++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    KQOff<F, BM, NW> off;
    kq_offsets<F, BM, NW>(off, xrb, wrb, wave, l);
    #pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < nst) kq_issue<F, BM, NW>(stages[s] + kg * L::STAGE, xr, wr, off, KG * s + kg, wave);
    if constexpr (DEFER) {
        static_assert(F::TYPE == TYPE_Q4_K && KG == 2 && BM >= 32, "deferred epilogue: Q4_K, two K-groups");
        KQ4Part<MT> part;
        float dxs[MT][16];
        for (int b = 0; b < nst; b += NS)
            kq4_round_defer<BM, NW, NS>(std::make_integer_sequence<int, NS>{}, stages, b, nst, xr, wr, off, kg, wave,
                                        l, part, dxs, acc);
        if (kg == 1 && nst > 0) kq4_epilogue<MT>(part, dxs, acc);
    } else {
        for (int b = 0; b < nst; b += NS)
            kq_round<F, BM, NW, NS, KG>(std::make_integer_sequence<int, NS>{}, stages, b, nst, xr, wr, off, kg, wave,
                                        l, acc);
    }

    if constexpr (KG > 1) kq_reduce_groups<F, BM, NW, KG>(stages[0], acc, kg, wave, l);
    if (kg == 0) kq_store<F, BM, NW>(acc, Y, count, N, m0, n0, wave, l);
}

// ---- Q4_K, 64 x 128 tiles, two K-groups, weight pairs ---------------------------
// A step's two super-blocks (one per K-group) are adjacent in each weight
// row, so the stage takes them as one 288-byte run per row (plus a pad piece:
// 304-byte rows keep a fragment read's 16 lanes on distinct LDS banks), loaded
// by all eight waves and read by both groups; each group's activation rows
// and scales keep their own part of the stage.  Per load instruction the
// weight lanes then touch ~11 cache lines instead of ~15 for 144-byte runs
// (measured on MI355X: the load pipeline of the C4 GEMM alone, arithmetic
// removed in a timing copy, took 20.5 us with the 144-byte weight runs and
// 13.3 us with fully contiguous weight runs).
struct KQ4P {
    using L = KQL<KQ4, 64, 4>;
    static constexpr int X_INSTR_ALL = L::X_INSTR_ALL;           // 19
    static constexpr int X_INSTR = L::X_INSTR;                   // per wave of a group
    static constexpr int XD = X_INSTR_ALL * 1024;                // a group's activation scales
    static constexpr int GROUP = XD + 256;
    static constexpr int W = 2 * GROUP;
    static constexpr int WRS = 304, WPIECES = 19;
    static constexpr int W_INSTR_ALL = KQ_BN * WPIECES / 64;     // 38
    static constexpr int W_INSTR = (W_INSTR_ALL + 7) / 8;        // per wave of the workgroup
    static constexpr int STAGE = W + KQ_BN * WRS;
    static_assert(KQ_BN * WPIECES % 64 == 0, "weight pairs are whole load instructions");
    static_assert(2 * STAGE <= 163840, "two stages fit the LDS");
};

struct KQ4POff {
    uint32_t x[KQ4P::X_INSTR];
    uint32_t w[KQ4P::W_INSTR];
    uint32_t xd;
};

__device__ __forceinline__ void kq4p_offsets(KQ4POff& o, uint32_t xrb, uint32_t wrb, int kg, int wave, int l) {
    #pragma unroll
    for (int q = 0; q < KQ4P::X_INSTR; q++) {
        const int p = (q * 4 + wave) * 64 + l, r = p / KQ4::XC, c = p - r * KQ4::XC;
        o.x[q] = (uint32_t)r * xrb + 4u + 16u * (uint32_t)(c < KQ4::XC - 1 ? c : 0);
    }
    #pragma unroll
    for (int q = 0; q < KQ4P::W_INSTR; q++) {
        const int p = (q * 8 + 4 * kg + wave) * 64 + l, row = p / KQ4P::WPIECES, piece = p - row * KQ4P::WPIECES;
        o.w[q] = (uint32_t)row * wrb + 16u * (uint32_t)(piece < KQ4P::WPIECES - 1 ? piece : 0);
    }
    o.xd = (uint32_t)l * xrb;
}

// the loads of step b (super-blocks 2b and 2b + 1) into one stage
__device__ __forceinline__ void kq4p_issue(uint8_t* stage, i32x4v xr, i32x4v wr, const KQ4POff& o, int b, int kg,
                                           int wave) {
    const uint32_t xs = (uint32_t)(2 * b + kg) * Q8_K_BYTES, ws = (uint32_t)(2 * b) * Q4_K_BYTES;
    uint8_t* gx = stage + kg * KQ4P::GROUP;
    #pragma unroll
    for (int q = 0; q < KQ4P::X_INSTR; q++) {
        const int idx = q * 4 + wave;
        if (idx < KQ4P::X_INSTR_ALL) lds_load16(xr, gx + 1024 * idx, o.x[q], xs);
    }
    #pragma unroll
    for (int q = 0; q < KQ4P::W_INSTR; q++) {
        const int idx = q * 8 + 4 * kg + wave;
        if (idx < KQ4P::W_INSTR_ALL) lds_load16(wr, stage + KQ4P::W + 1024 * idx, o.w[q], ws);
    }
    if (wave == 0) lds_load4(xr, gx + KQ4P::XD, o.xd, xs);
}

template <bool DEFER, int S>
__device__ __forceinline__ void kq4p_step(uint8_t* const (&stages)[KQ_MAX_NS], int b, int nst, i32x4v xr, i32x4v wr,
                                          const KQ4POff& off, int kg, int wave, int l, KQ4Part<2>& part,
                                          float (&dxs)[2][16], float (&acc)[2][16]) {
    if (b >= nst) return;
    wait_vmcnt<0>();
    if constexpr (DEFER) wait_lgkmcnt0();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int n = l & 31, g2 = l >> 5;
    const uint8_t* st = stages[S];
    const uint8_t* gx = st + kg * KQ4P::GROUP;
    if (DEFER && kg == 1 && b > 0) kq4_epilogue<2>(part, dxs, acc);
    if (b + 1 < nst) kq4p_issue(stages[S ^ 1], xr, wr, off, b + 1, kg, wave);
    kq4_mma<2>(st + KQ4P::W + (32 * wave + n) * KQ4P::WRS + KQ4::BB * kg, gx + n * KQ4::XRS + 16 * g2, g2, part);
    kq_dx<2>(gx + KQ4P::XD, 0, g2, dxs);
    if (!DEFER || kg == 0) kq4_epilogue<2>(part, dxs, acc);
}

template <bool DEFER>
__device__ __forceinline__ void kq4p_tile(uint8_t* const (&stages)[KQ_MAX_NS], const uint8_t* W, uint32_t wrb,
                                          const uint8_t* X, uint32_t xrb, float* Y, int count, int N, int nsb, int m0,
                                          int n0, int kg, int wave, int l, int kb0) {
    const int nst = nsb / 2;
    const uint32_t xk = (uint32_t)kb0 * Q8_K_BYTES, wk = (uint32_t)kb0 * Q4_K_BYTES;
    const i32x4v xr = make_rsrc4(X + (size_t)m0 * xrb + xk, (uint32_t)((size_t)(count - m0) * xrb) - xk);
    const i32x4v wr = make_rsrc4(W + (size_t)n0 * wrb + wk, (uint32_t)((size_t)(N - n0) * wrb) - wk);
    float acc[2][16];
    #pragma unroll
    for (int t = 0; t < 2; t++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    KQ4POff off;
    kq4p_offsets(off, xrb, wrb, kg, wave, l);
    if (nst > 0) kq4p_issue(stages[0], xr, wr, off, 0, kg, wave);
    KQ4Part<2> part;
    float dxs[2][16];
    for (int b = 0; b < nst; b += 2) {
        kq4p_step<DEFER, 0>(stages, b, nst, xr, wr, off, kg, wave, l, part, dxs, acc);
        kq4p_step<DEFER, 1>(stages, b + 1, nst, xr, wr, off, kg, wave, l, part, dxs, acc);
    }
    if (DEFER && kg == 1 && nst > 0) kq4_epilogue<2>(part, dxs, acc);
    kq_reduce_groups<KQ4, 64, 4, 2>(stages[0], acc, kg, wave, l);
    if (kg == 0) kq_store<KQ4, 64, 4>(acc, Y, count, N, m0, n0, wave, l);
}

// ---- grouped: one pipeline across the workgroup's tiles ------------------------
// A grouped workgroup runs several tiles; its loads run NS-1 super-blocks
// ahead across tile boundaries, so a new tile does not start with an empty
// pipeline.  Each step is still one stage: wait for this thread's loads of
// the stage, barrier, issue the stage NS-1 steps ahead (into the stage every
// wave finished before the barrier), compute.
struct KQTile {
    const uint8_t* W;
    const uint8_t* X;
    float* Y;
    int count, m0, n0, kb0;
};

template <class F>
__device__ __forceinline__ void kq_tile_rsrc(const KQTile& t, uint32_t xrb, uint32_t wrb, int N, i32x4v& xr, i32x4v& wr) {
    const uint32_t xk = (uint32_t)t.kb0 * Q8_K_BYTES, wk = (uint32_t)t.kb0 * F::BB;
    xr = make_rsrc4(t.X + (size_t)t.m0 * xrb + xk, (uint32_t)((size_t)(t.count - t.m0) * xrb) - xk);
    wr = make_rsrc4(t.W + (size_t)t.n0 * wrb + wk, (uint32_t)((size_t)(N - t.n0) * wrb) - wk);
}

template <class F, int BM, int NW, class Dec>
struct KQStream {
    const Dec& decode;
    int total, grid, nsb, N;
    uint32_t xrb, wrb;
    KQOff<F, BM, NW> off;
    int wave, l;
    // load cursor
    int lt, lb, lxi;
    i32x4v lxr, lwr;
    // compute cursor
    int ct, cb;
    KQTile cT;

    __device__ __forceinline__ void set_load_tile(const KQTile& t) {
        kq_tile_rsrc<F>(t, xrb, wrb, N, lxr, lwr);
        const int rows = t.count - t.m0 < BM ? t.count - t.m0 : BM;
        const int xi = (rows * F::XC + 63) / 64;
        lxi = xi < KQL<F, BM, NW>::X_INSTR_ALL ? xi : KQL<F, BM, NW>::X_INSTR_ALL;
    }
    __device__ __forceinline__ void issue_next(uint8_t* stage) {
        kq_issue<F, BM, NW>(stage, lxr, lwr, off, lb, wave, lxi);
        if (++lb == nsb) {
            lb = 0;
            lt += grid;
            if (lt < total) set_load_tile(decode(lt));
        }
    }
};

template <class F, int BM, int NW, int NS, int S, class Dec>
__device__ __forceinline__ void kq_stream_step(KQStream<F, BM, NW, Dec>& st, uint8_t* const (&stages)[KQ_MAX_NS],
                                               int h, int G, float (&acc)[KQL<F, BM, NW>::MTW][16]) {
    using L = KQL<F, BM, NW>;
    constexpr int MT = L::MTW;
    if (h >= G) return;
    // stages may skip activation loads: count only the weight loads
    if (h + NS - 2 < G) wait_vmcnt<(NS - 2) * L::LOADS_MIN_W>();
    else wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (h + NS - 1 < G) st.issue_next(stages[(S + NS - 1) % NS]);
    kq_compute<F, BM, NW>(stages[S], st.cb, st.wave, st.l, acc);
    if (++st.cb == st.nsb) {
        kq_store<F, BM, NW>(acc, st.cT.Y, st.cT.count, st.N, st.cT.m0, st.cT.n0, st.wave, st.l);
        #pragma unroll
        for (int t = 0; t < MT; t++)
            #pragma unroll
            for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
        st.cb = 0;
        st.ct += st.grid;
        if (st.ct < st.total) st.cT = st.decode(st.ct);
    }
}

template <class F, int BM, int NW, int NS, class Dec, int... S>
__device__ __forceinline__ void kq_stream_round(std::integer_sequence<int, S...>, KQStream<F, BM, NW, Dec>& st,
                                                uint8_t* const (&stages)[KQ_MAX_NS], int g, int G,
                                                float (&acc)[KQL<F, BM, NW>::MTW][16]) {
    (kq_stream_step<F, BM, NW, NS, S>(st, stages, g + S, G, acc), ...);
}

template <class F, int BM, int NS, int NW, class Dec>
__device__ __forceinline__ void kq_grouped_stream(uint8_t* const (&stages)[KQ_MAX_NS], const Dec& decode, int total,
                                                  int nsb, uint32_t xrb, uint32_t wrb, int N, int wave, int l) {
    using L = KQL<F, BM, NW>;
    constexpr int MT = L::MTW;
    const int t0 = blockIdx.x, grid = gridDim.x;
    if (t0 >= total) return;
    const int G = ((total - 1 - t0) / grid + 1) * nsb;   // this workgroup's steps
    KQStream<F, BM, NW, Dec> st{decode, total, grid, nsb, N, xrb, wrb, {}, wave, l, t0, 0, 0, {}, {}, t0, 0, {}};
    kq_offsets<F, BM, NW>(st.off, xrb, wrb, wave, l);
    st.cT = decode(t0);
    st.set_load_tile(st.cT);
    #pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < G) st.issue_next(stages[s]);
    float acc[MT][16];
    #pragma unroll
    for (int t = 0; t < MT; t++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    for (int g = 0; g < G; g += NS)
        kq_stream_round<F, BM, NW, NS>(std::make_integer_sequence<int, NS>{}, st, stages, g, G, acc);
}

// The flattened (expert, m-tile, mat, K slice, n-tile) list of a grouped
// launch: every wave builds the per-expert m-tile prefix from the device
// offsets (lane e holds expert e); operator() maps a list index to its tile.
template <int BM>
struct KQExperts {
    const KQWeights& wt;
    const uint8_t* X;
    uint32_t xrb;
    float* Y;
    int N, tiles_n, ne, nmat, ks, nsb_k, total;
    size_t ymat, ykstride;
    int r0, cnt, nt, inc;

    __device__ __forceinline__ KQExperts(const KQWeights& wt_, const uint8_t* X_, uint32_t xrb_, float* Y_, int N_,
                                         int nsb, int tiles_n_, const int32_t* __restrict__ offsets, int ne_,
                                         int nmat_, size_t ymat_, int ks_, size_t ykstride_, int l)
        : wt(wt_), X(X_), xrb(xrb_), Y(Y_), N(N_), tiles_n(tiles_n_), ne(ne_), nmat(nmat_), ks(ks_),
          nsb_k(nsb / ks_), total(0), ymat(ymat_), ykstride(ykstride_), r0(0), cnt(0) {
        if (l < ne) {
            r0 = offsets[l];
            cnt = offsets[l + 1] - r0;
        }
        nt = (cnt + BM - 1) / BM;
        inc = nt;   // inclusive prefix of m-tiles over experts
        #pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(inc, o);
            if (l >= o) inc += v;
        }
        total = __builtin_amdgcn_readlane(inc, 63) * nmat * ks * tiles_n;
    }

    __device__ __forceinline__ KQTile operator()(int t) const {
        const int ntile = t % tiles_n, rk = t / tiles_n, ksl = rk % ks, r = rk / ks, mat = r % nmat, s = r / nmat;
        // expert of m-slot s: the number of experts whose tiles all lie before it
        const int e = __builtin_amdgcn_readfirstlane(__popcll(__ballot(inc <= s)));
        const int mt = s - __builtin_amdgcn_readlane(inc - nt, e);
        const int row0 = __builtin_amdgcn_readlane(r0, e);
        KQTile T;
        T.W = wt.w[mat * ne + e];
        T.X = X + (size_t)row0 * xrb;
        T.Y = Y + (size_t)mat * ymat + (size_t)ksl * ykstride + (size_t)row0 * N;
        T.count = __builtin_amdgcn_readlane(cnt, e);
        T.m0 = mt * BM;
        T.n0 = ntile * KQ_BN;
        T.kb0 = ksl * nsb_k;
        return T;
    }
};

// Ungrouped: one tile per workgroup of the M x N product with weights wt.w[0].
// GROUPED: nmat weight sets of ne experts each; expert e's activation and
// output rows are [offsets[e], offsets[e+1]) of X and of Y + mat * ymat, and
// its weights are wt.w[mat * ne + e].  Tiles exist only for rows that are
// there: every workgroup builds the per-expert tile prefix from the device
// offsets (lane e holds expert e) and strides over the flattened
// (expert, m-tile, mat, n-tile) list, so no host round trip is needed.
template <class F, int BM, int NS, int NW, int KG, bool GROUPED, bool DEFER = false, bool PAIR = false>
__global__ __launch_bounds__(64 * NW * KG, 1)
void kq_kernel(KQWeights wt, uint32_t wrb, const uint8_t* __restrict__ X, uint32_t xrb, float* __restrict__ Y, int M,
               int N, int nsb, int tiles_m, int tiles_n, const int32_t* __restrict__ offsets, int ne, int nmat,
               size_t ymat, int ks, size_t ykstride, int xcd_order) {
    static_assert(NS >= 2 && NS <= KQ_MAX_NS, "stage count");
    static_assert(KG == 1 || !GROUPED, "K-groups split one tile's super-blocks (ungrouped launches)");
    using L = KQL<F, BM, NW>;
    static_assert(!PAIR || (F::TYPE == TYPE_Q4_K && BM == 64 && NW == 4 && KG == 2 && NS == 2 && !GROUPED),
                  "weight pairs: Q4_K 64 x 128 tiles, two K-groups, two stages");
    constexpr int SB = PAIR ? KQ4P::STAGE : KG * L::STAGE;
    // one array per stage (stages beyond NS are unused 16-byte stubs)
    __shared__ __align__(16) uint8_t st0[SB];
    __shared__ __align__(16) uint8_t st1[SB];
    __shared__ __align__(16) uint8_t st2[NS > 2 ? SB : 16];
    __shared__ __align__(16) uint8_t st3[NS > 3 ? SB : 16];
    __shared__ __align__(16) uint8_t st4[NS > 4 ? SB : 16];
    __shared__ __align__(16) uint8_t st5[NS > 5 ? SB : 16];
    uint8_t* const stages[KQ_MAX_NS] = {st0, st1, st2, st3, st4, st5};
    const int l = threadIdx.x & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kg = wave_all / NW, wave = wave_all - kg * NW;

    if constexpr (!GROUPED) {
        // workgroup i runs on XCD i % 8: give each XCD a contiguous run of
        // tiles so neighbouring weight tiles share its L2
        // with ks K slices, slice i of a tile takes super-blocks
        // [i, i + 1) * nsb / ks and writes its partial product to Y + i M N
        const int n_tiles = tiles_m * tiles_n;
        const int slice = blockIdx.x / n_tiles, nsb_k = nsb / ks;
        int tile = blockIdx.x - slice * n_tiles;
        if (xcd_order && (n_tiles & 7) == 0) tile = (tile & 7) * (n_tiles >> 3) + (tile >> 3);
        const int mt = tile % tiles_m, ntile = tile / tiles_m;
        if constexpr (PAIR)
            kq4p_tile<DEFER>(stages, wt.w[0], wrb, X, xrb, Y + (size_t)slice * M * N, M, N, nsb_k, mt * BM,
                             ntile * KQ_BN, kg, wave, l, slice * nsb_k);
        else
            kq_tile<F, BM, NS, NW, KG, DEFER>(stages, wt.w[0], wrb, X, xrb, Y + (size_t)slice * M * N, M, N, nsb_k,
                                              mt * BM, ntile * KQ_BN, kg, wave, l, slice * nsb_k);
    } else {
        const KQExperts<BM> ex(wt, X, xrb, Y, N, nsb, tiles_n, offsets, ne, nmat, ymat, ks, ykstride, l);
        kq_grouped_stream<F, BM, NS, NW>(stages, ex, ex.total, ex.nsb_k, xrb, wrb, N, wave, l);
    }
}

// ---- launch ------------------------------------------------------------------

static int cu_count() {
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

struct KQArgs {
    KQWeights wt;
    uint32_t wrb, xrb;
    const uint8_t* X;
    float* Y;
    int M, N, nsb;
    const int32_t* offsets;
    int ne, nmat;        // grouped: experts per weight set, weight sets
    size_t total_rows;   // grouped: rows over all experts
    size_t ymat;
    int ks;              // K slices, each writing its partial product
    size_t ykstride;
};

template <class F, int BM, int NS, int NW, bool GROUPED, int KG = 1, bool DEFER = false, bool PAIR = false>
static hipError_t kq_launch_t(const KQArgs& a, hipStream_t s) {
    const int tiles_n = (a.N + KQ_BN - 1) / KQ_BN;
    int tiles_m = (a.M + BM - 1) / BM;
    unsigned grid = (unsigned)(tiles_m * tiles_n * a.ks);
    if constexpr (GROUPED) {
        // m-tiles over all experts: sum of ceil(c_e / BM) <= (total + ne (BM - 1)) / BM
        const size_t slots = (a.total_rows + (size_t)a.ne * (BM - 1)) / BM;
        const size_t tiles = slots * (size_t)a.nmat * (size_t)a.ks * (size_t)tiles_n;
        const size_t per_cu = 163840 / (NS * (size_t)KQL<F, BM, NW>::STAGE);
        const size_t cap = (size_t)cu_count() * (per_cu ? per_cu : 1);
        grid = (unsigned)(tiles < cap ? tiles : cap);
        tiles_m = 0;
    }
    // ungrouped K slices: whole K-group steps, even first super-blocks
    if (!GROUPED && (a.nsb % a.ks != 0 || (a.ks > 1 && (a.nsb / a.ks) % 2 != 0))) return hipErrorInvalidValue;
    if ((GROUPED ? a.nsb : a.nsb / a.ks) % KG != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((kq_kernel<F, BM, NS, NW, KG, GROUPED, DEFER, PAIR>), dim3(grid), dim3(64 * NW * KG), 0, s, a.wt, a.wrb, a.X, a.xrb,
                       a.Y, a.M, a.N, a.nsb, tiles_m, tiles_n, a.offsets, a.ne, a.nmat, a.ymat, a.ks, a.ykstride,
                       tuning_env(TUNE_GEMM_XCD, 1));   // XCD-aware tile order (ungrouped)
    return hipGetLastError();
}

// The Q6_K prompt GEMM on 128 x 128 tiles: four waves of 128 x 32, so each
// weight slice is decoded once for four MFMA row tiles (gemm_kq6_tall.hip).
hipError_t kq6_tall_launch(const KQArgs& a, hipStream_t s);

}  // namespace barq
