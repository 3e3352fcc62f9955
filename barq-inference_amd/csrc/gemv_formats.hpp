// Per-format lane slices for the batch-1 GEMV kernels.
//
// Every GEMV wave walks rows; inside a row, lane L owns the same 64 weights
// of each 4096-element K chunk ("iteration"), so its activation slice is
// loaded once per iteration (straight from global memory: the whole vector is
// a few KB and stays in L1/L2) and reused for every row the wave handles.
//
//   Q4_K  (144 B / 256): lane -> super-block L/4, sub-block pair p = L%4:
//         header (d, dmin, 12 scale bytes) + qs[32p .. 32p+32).
//   Q6_K  (210 B / 256): lane -> block L/4, half h, 16-lane run lr:
//         ql[64h+lr..+16], ql[64h+32+lr..+16], qh[32h+lr..+16], 4 scales, d.
//   Q4_0  (18 B / 32), Q8_0 (34 B / 32), Q4_0_BARQ (20 B / 32):
//         lane -> two consecutive blocks (64 elements).
//
// Each format provides, for the integer (Q8 activation) path:
//   X, Wt, Lane     activation slice, weight bytes, per-lane constants
//   load_x / load_w / dot
// and for the literal f32 path:
//   deq4(w, lane, g, v)  the 4 weights of group g (g = 0..15), bit-identical
//                        to the reference decoders; xoff(lane, g) is their K
//                        offset inside the iteration.
#pragma once
#include "common.hpp"

namespace barq {

constexpr uint32_t M4 = 0x0F0F0F0Fu;
constexpr uint32_t M30 = 0x30303030u;
typedef short s16x2q __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t u4get(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ int sext16(uint32_t v, uint32_t off) { return __builtin_amdgcn_sbfe((int)v, off, 16); }

// Sum of the 16 signed bytes of a uint4 (v_dot4 against 0x01010101).
__device__ __forceinline__ int bytesum16(const uint4& v) {
    int s = sdot4(v.x, 0x01010101u, 0);
    s = sdot4(v.y, 0x01010101u, s);
    s = sdot4(v.z, 0x01010101u, s);
    return sdot4(v.w, 0x01010101u, s);
}

// ---------------------------------------------------------------------------
// Q4_K x Q8_K  (gguf.rs:730-837 decode; llama.cpp vec_dot_q4_K_q8_K math)
// ---------------------------------------------------------------------------
struct FmtQ4K {
    static constexpr int ROW_BLOCK_ELEMS = 256;
    static constexpr int ROW_BLOCK_BYTES = 144;

    struct X { uint4 v[4]; int sa, sb; float dx; };
    struct Wt { uint4 hdr, q0, q1; };
    // get_scale_min_k4 (gguf.rs:825-837) for sub-blocks 2p and 2p+1 as bit
    // field extracts: p < 2 reads 6-bit fields of q[2p..2p+1] / q[2p+4..];
    // p >= 2 takes the low/high nibble of q[2p+4..] plus 2 bits of q[2p-4..].
    // sel: the byte-permute selector that gathers those bytes (scales4).
    struct Lane { int sbl, p; uint32_t o, n1, n2, ob, sel; bool hi; };

    static __device__ __forceinline__ Lane lane(int l) {
        Lane c;
        c.sbl = l >> 2;
        c.p = l & 3;
        c.hi = c.p >= 2;
        c.o = 16u * (uint32_t)(c.p & 1);
        c.n1 = c.hi ? 4u : 6u;
        c.n2 = c.hi ? 2u : 0u;
        c.ob = c.hi ? c.o + 4 : c.o;
        const uint32_t pp = 2u * (uint32_t)(c.p & 1);
        c.sel = pp | ((pp + 1) << 8) | ((pp + 4) << 16) | ((pp + 5) << 24);
        return c;
    }
    static __device__ __forceinline__ int blk(int it, const Lane& c) { return it * 16 + c.sbl; }
    static __device__ __forceinline__ bool active(int it, const Lane& c, int nblk) { return blk(it, c) < nblk; }

    // Q8_K block: f32 d, i8 qs[256] at +4, i16 bsums[16] at +260
    static __device__ __forceinline__ void load_x(X& x, const uint8_t* __restrict__ xq, int it, const Lane& c, int) {
        const uint8_t* b = xq + (size_t)blk(it, c) * 292;
        x.dx = *reinterpret_cast<const float*>(b);
        #pragma unroll
        for (int i = 0; i < 4; i++) x.v[i] = ld16_a4(b + 4 + 64 * c.p + 16 * i);
        const uint32_t* bs = reinterpret_cast<const uint32_t*>(b + 260 + 8 * c.p);
        const uint32_t b0 = bs[0], b1 = bs[1];
        x.sa = sext16(b0, 0) + sext16(b0, 16);
        x.sb = sext16(b1, 0) + sext16(b1, 16);
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, const Lane& c, int) {
        const uint8_t* b = row + (size_t)blk(it, c) * 144;
        w.hdr = *reinterpret_cast<const uint4*>(b);
        w.q0 = *reinterpret_cast<const uint4*>(b + 16 + 32 * c.p);
        w.q1 = *reinterpret_cast<const uint4*>(b + 32 + 32 * c.p);
    }

    static __device__ __forceinline__ void scales(const uint4& hdr, const Lane& c, int& sca, int& ma, int& scb, int& mb) {
        const uint32_t A = c.hi ? hdr.w : hdr.y, B = c.hi ? hdr.w : hdr.z;
        sca = (int)(__builtin_amdgcn_ubfe(A, c.o, c.n1) | (__builtin_amdgcn_ubfe(hdr.y, c.o + 6, c.n2) << 4));
        scb = (int)(__builtin_amdgcn_ubfe(A, c.o + 8, c.n1) | (__builtin_amdgcn_ubfe(hdr.y, c.o + 14, c.n2) << 4));
        ma = (int)(__builtin_amdgcn_ubfe(B, c.ob, c.n1) | (__builtin_amdgcn_ubfe(hdr.z, c.o + 6, c.n2) << 4));
        mb = (int)(__builtin_amdgcn_ubfe(B, c.ob + 8, c.n1) | (__builtin_amdgcn_ubfe(hdr.z, c.o + 14, c.n2) << 4));
    }

    // The same four values as bytes [sc_a, sc_b, m_a, m_b] of one dword, by
    // byte permutes: P gathers q[2p'], q[2p'+1], q[2p'+4], q[2p'+5] (p' = p
    // mod 2), Q the bytes q[8+2p'], q[9+2p'] and the high nibbles of the
    // same two bytes.  p < 2: P's 6-bit fields; p >= 2: Q's nibbles with
    // P's top two bits above them.
    static __device__ __forceinline__ uint32_t scales4(const uint4& hdr, const Lane& c) {
        const uint32_t P = __builtin_amdgcn_perm(hdr.z, hdr.y, c.sel);
        const uint32_t Q = __builtin_amdgcn_perm(hdr.w >> 4, hdr.w, c.sel);
        return c.hi ? (((P >> 2) & M30) | (Q & M4)) : (P & 0x3F3F3F3Fu);
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, const Lane& c) {
        int ia = 0, ib = 0;
        ia = sdot4(w.q0.x & M4, x.v[0].x, ia); ia = sdot4(w.q0.y & M4, x.v[0].y, ia);
        ia = sdot4(w.q0.z & M4, x.v[0].z, ia); ia = sdot4(w.q0.w & M4, x.v[0].w, ia);
        ia = sdot4(w.q1.x & M4, x.v[1].x, ia); ia = sdot4(w.q1.y & M4, x.v[1].y, ia);
        ia = sdot4(w.q1.z & M4, x.v[1].z, ia); ia = sdot4(w.q1.w & M4, x.v[1].w, ia);
        ib = sdot4((w.q0.x >> 4) & M4, x.v[2].x, ib); ib = sdot4((w.q0.y >> 4) & M4, x.v[2].y, ib);
        ib = sdot4((w.q0.z >> 4) & M4, x.v[2].z, ib); ib = sdot4((w.q0.w >> 4) & M4, x.v[2].w, ib);
        ib = sdot4((w.q1.x >> 4) & M4, x.v[3].x, ib); ib = sdot4((w.q1.y >> 4) & M4, x.v[3].y, ib);
        ib = sdot4((w.q1.z >> 4) & M4, x.v[3].z, ib); ib = sdot4((w.q1.w >> 4) & M4, x.v[3].w, ib);
        const uint32_t sm = scales4(w.hdr, c);
        // |ia|, |ib| <= 32*15*128 and the scales are 6-bit: 24-bit products suffice
        const int im = __mul24((int)(sm & 0xFFu), ia) + __mul24((int)__builtin_amdgcn_ubfe(sm, 8, 8), ib);
        // the mins against the two bsum pairs (|sa|, |sb| <= 32*128) as one i16 dot2
        const uint32_t mm = __builtin_amdgcn_perm(0u, sm, 0x0c030c02u);   // u16 pair (m_a, m_b)
        const uint32_t sab = ((uint32_t)x.sa & 0xFFFFu) | ((uint32_t)x.sb << 16);
        const int in = __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2q, mm), __builtin_bit_cast(s16x2q, sab), 0, false);
        const float d = f16_bits_to_f32(w.hdr.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(w.hdr.x >> 16);
        return x.dx * __builtin_fmaf(d, (float)im, -(dmin * (float)in));
    }

    // literal path: group g covers elements 64p + 4g .. +4 of super-block sb
    static __device__ __forceinline__ int xoff(int l, int g) { return (l >> 2) * 256 + 64 * (l & 3) + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, const Lane& c, int g, float v[4]) {
        int sca, ma, scb, mb;
        scales(w.hdr, c, sca, ma, scb, mb);
        const float d = f16_bits_to_f32(w.hdr.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(w.hdr.x >> 16);
        const bool hi = g >= 8;
        const float d1 = d * (float)(hi ? scb : sca);
        const float m1 = dmin * (float)(hi ? mb : ma);
        const int gg = g & 7;
        uint32_t q = u4get(gg < 4 ? w.q0 : w.q1, gg & 3);
        if (hi) q >>= 4;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = d1 * (float)((q >> (8 * i)) & 15u);
            v[i] = p - m1;
        }
    }
};

// ---------------------------------------------------------------------------
// Q6_K x Q8_K  (gguf.rs:839-914 decode; llama.cpp vec_dot_q6_K_q8_K math)
// ---------------------------------------------------------------------------
struct FmtQ6K {
    static constexpr int ROW_BLOCK_ELEMS = 256;
    static constexpr int ROW_BLOCK_BYTES = 210;

    struct X { uint4 v[4]; int bs32[4]; float dx; };
    struct Wt { uint4 a, b, h; uint2 sc; uint32_t d; };
    struct Lane { int bl, h, lr, s0; };

    static __device__ __forceinline__ Lane lane(int l) {
        Lane c;
        c.bl = l >> 2;
        c.h = (l >> 1) & 1;
        c.s0 = l & 1;
        c.lr = 16 * c.s0;
        return c;
    }
    static __device__ __forceinline__ int blk(int it, const Lane& c) { return it * 16 + c.bl; }
    static __device__ __forceinline__ bool active(int it, const Lane& c, int nblk) { return blk(it, c) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const uint8_t* __restrict__ xq, int it, const Lane& c, int) {
        const uint8_t* b = xq + (size_t)blk(it, c) * 292;
        x.dx = *reinterpret_cast<const float*>(b);
        #pragma unroll
        for (int qd = 0; qd < 4; qd++) x.v[qd] = ld16_a4(b + 4 + 128 * c.h + c.lr + 32 * qd);
        // bsums[8h + 2qd + s0], qd = 0..3: the int16 at half s0 of dword qd
        const uint4 bs = ld16_a4(b + 260 + 16 * c.h);
        const uint32_t off = 16u * (uint32_t)c.s0;
        x.bs32[0] = 32 * sext16(bs.x, off);
        x.bs32[1] = 32 * sext16(bs.y, off);
        x.bs32[2] = 32 * sext16(bs.z, off);
        x.bs32[3] = 32 * sext16(bs.w, off);
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, const Lane& c, int) {
        const uint8_t* b = row + (size_t)blk(it, c) * 210;
        w.a = ld16_a2(b + 64 * c.h + c.lr);
        w.b = ld16_a2(b + 64 * c.h + 32 + c.lr);
        w.h = ld16_a2(b + 128 + 32 * c.h + c.lr);
        w.sc = ld8_a2(b + 192 + 8 * c.h);
        w.d = ld_u16(b + 208);
    }

    // the lane's four i8 scales sc[8h + lr/16 + 2qd], qd = 0..3
    static __device__ __forceinline__ void scales(const Wt& w, const Lane& c, int s[4]) {
        const uint32_t o = 8u * (uint32_t)c.s0;
        s[0] = __builtin_amdgcn_sbfe((int)w.sc.x, o, 8);
        s[1] = __builtin_amdgcn_sbfe((int)w.sc.x, o + 16, 8);
        s[2] = __builtin_amdgcn_sbfe((int)w.sc.y, o, 8);
        s[3] = __builtin_amdgcn_sbfe((int)w.sc.y, o + 16, 8);
    }

    static __device__ __forceinline__ void unpack(uint32_t A, uint32_t B, uint32_t H, uint32_t q[4]) {
        q[0] = (A & M4) | ((H << 4) & M30);
        q[1] = (B & M4) | ((H << 2) & M30);
        q[2] = ((A >> 4) & M4) | (H & M30);
        q[3] = ((B >> 4) & M4) | ((H >> 2) & M30);
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, const Lane& c) {
        int i[4] = {0, 0, 0, 0};
        #pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t q[4];
            unpack(u4get(w.a, t), u4get(w.b, t), u4get(w.h, t), q);
            #pragma unroll
            for (int qd = 0; qd < 4; qd++) i[qd] = sdot4(q[qd], u4get(x.v[qd], t), i[qd]);
        }
        int s[4];
        scales(w, c, s);
        // q6 in [0,63]: sum (q6-32) x = i - 32*bsum; |i - 32 bs| < 2^18, |s| <= 128
        const int tot = __mul24(s[0], i[0] - x.bs32[0]) + __mul24(s[1], i[1] - x.bs32[1]) +
                        __mul24(s[2], i[2] - x.bs32[2]) + __mul24(s[3], i[3] - x.bs32[3]);
        return (f16_bits_to_f32(w.d) * x.dx) * (float)tot;
    }

    // literal path: group g = 4*qd + t -> elements 128h + 32qd + lr + 4t
    static __device__ __forceinline__ int xoff(int l, int g) {
        return (l >> 2) * 256 + 128 * ((l >> 1) & 1) + 32 * (g >> 2) + 16 * (l & 1) + 4 * (g & 3);
    }
    static __device__ __forceinline__ void deq4(const Wt& w, const Lane& c, int g, float v[4]) {
        const int qd = g >> 2, t = g & 3;
        uint32_t q[4];
        unpack(u4get(w.a, t), u4get(w.b, t), u4get(w.h, t), q);
        int s[4];
        scales(w, c, s);
        const float dd = f16_bits_to_f32(w.d) * (float)s[qd];
        const uint32_t qq = q[qd];
        #pragma unroll
        for (int e = 0; e < 4; e++) v[e] = dd * (float)((int)((qq >> (8 * e)) & 63u) - 32);
    }
};

// ---------------------------------------------------------------------------
// Two 32-element blocks per lane: Q4_0 (GGUF), Q8_0, Q4_0_BARQ, all against
// Q8_0 activations (f16 d + 32 x i8, 34 B).
// ---------------------------------------------------------------------------
struct Pair32Lane { int l; };

struct XQ80 { uint4 v[4]; int s[2]; float dx[2]; };

__device__ __forceinline__ void load_x_q8_0(XQ80& x, const uint8_t* __restrict__ xq, int b, int nblk) {
    #pragma unroll
    for (int j = 0; j < 2; j++) {
        if (b + j < nblk) {
            const uint8_t* p = xq + (size_t)(b + j) * 34;
            x.dx[j] = f16_bits_to_f32(ld_u16(p));
            x.v[2 * j] = ld16_a2(p + 2);
            x.v[2 * j + 1] = ld16_a2(p + 18);
        } else {
            x.dx[j] = 0.0f;
            x.v[2 * j] = make_uint4(0, 0, 0, 0);
            x.v[2 * j + 1] = make_uint4(0, 0, 0, 0);
        }
        x.s[j] = bytesum16(x.v[2 * j]) + bytesum16(x.v[2 * j + 1]);
    }
}

// Q4_0 (GGUF) x Q8_0  (llama.cpp block_q4_0; parity with gguf.rs:521-578 via
// the byte adapter: both decode to (nib - 8) * d)
struct FmtQ40 {
    static constexpr int ROW_BLOCK_ELEMS = 32;
    static constexpr int ROW_BLOCK_BYTES = 18;
    using X = XQ80;
    using Lane = Pair32Lane;
    struct Wt { uint4 q[2]; uint32_t d[2]; };

    static __device__ __forceinline__ Lane lane(int l) { return {l}; }
    static __device__ __forceinline__ int blk(int it, const Lane& c) { return it * 128 + 2 * c.l; }
    static __device__ __forceinline__ bool active(int it, const Lane& c, int nblk) { return blk(it, c) < nblk; }
    static __device__ __forceinline__ void load_x(X& x, const uint8_t* __restrict__ xq, int it, const Lane& c, int nblk) {
        load_x_q8_0(x, xq, blk(it, c), nblk);
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, const Lane& c, int nblk) {
        const int b = blk(it, c);
        const uint8_t* p = row + (size_t)b * 18;
        w.d[0] = ld_u16(p);
        w.q[0] = ld16_a2(p + 2);
        if (b + 1 < nblk) {
            w.d[1] = ld_u16(p + 18);
            w.q[1] = ld16_a2(p + 20);
        } else {
            w.d[1] = 0; w.q[1] = make_uint4(0, 0, 0, 0);
        }
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, const Lane&) {
        float r = 0.0f;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            int s = 0;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = u4get(w.q[j], t);
                s = sdot4(q & M4, u4get(x.v[2 * j], t), s);
                s = sdot4((q >> 4) & M4, u4get(x.v[2 * j + 1], t), s);
            }
            const float dw = f16_bits_to_f32(w.d[j]);
            r = __builtin_fmaf(dw * x.dx[j], (float)(s - 8 * x.s[j]), r);
        }
        return r;
    }

    // literal: g<8 block 0, else block 1; gg<4 low nibbles of dword gg
    // (elements 4gg..), else high nibbles of dword gg-4 (elements 16+4(gg-4)..)
    static __device__ __forceinline__ int xoff(int l, int g) { return 64 * l + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, const Lane&, int g, float v[4]) {
        const int j = g >> 3, gg = g & 7;
        uint32_t q = u4get(w.q[j], gg & 3);
        if (gg >= 4) q >>= 4;
        const float d = f16_bits_to_f32(w.d[j]);
        #pragma unroll
        for (int e = 0; e < 4; e++) v[e] = (float)((int)((q >> (8 * e)) & 15u) - 8) * d;
    }
};

// Q8_0 x Q8_0  (gguf.rs:634-681 decode; llama.cpp vec_dot_q8_0_q8_0 math)
struct FmtQ80 {
    static constexpr int ROW_BLOCK_ELEMS = 32;
    static constexpr int ROW_BLOCK_BYTES = 34;
    using X = XQ80;
    using Lane = Pair32Lane;
    struct Wt { uint4 q[4]; uint32_t d[2]; };

    static __device__ __forceinline__ Lane lane(int l) { return {l}; }
    static __device__ __forceinline__ int blk(int it, const Lane& c) { return it * 128 + 2 * c.l; }
    static __device__ __forceinline__ bool active(int it, const Lane& c, int nblk) { return blk(it, c) < nblk; }
    static __device__ __forceinline__ void load_x(X& x, const uint8_t* __restrict__ xq, int it, const Lane& c, int nblk) {
        load_x_q8_0(x, xq, blk(it, c), nblk);
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, const Lane& c, int nblk) {
        const int b = blk(it, c);
        const uint8_t* p = row + (size_t)b * 34;
        w.d[0] = ld_u16(p);
        w.q[0] = ld16_a2(p + 2);
        w.q[1] = ld16_a2(p + 18);
        if (b + 1 < nblk) {
            w.d[1] = ld_u16(p + 34);
            w.q[2] = ld16_a2(p + 36);
            w.q[3] = ld16_a2(p + 52);
        } else {
            w.d[1] = 0; w.q[2] = make_uint4(0, 0, 0, 0); w.q[3] = make_uint4(0, 0, 0, 0);
        }
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, const Lane&) {
        float r = 0.0f;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            int s = 0;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                s = sdot4(u4get(w.q[2 * j], t), u4get(x.v[2 * j], t), s);
                s = sdot4(u4get(w.q[2 * j + 1], t), u4get(x.v[2 * j + 1], t), s);
            }
            const float dw = f16_bits_to_f32(w.d[j]);
            r = __builtin_fmaf(dw * x.dx[j], (float)s, r);
        }
        return r;
    }

    static __device__ __forceinline__ int xoff(int l, int g) { return 64 * l + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, const Lane&, int g, float v[4]) {
        const int j = g >> 3;
        const uint32_t q = u4get(w.q[g >> 2], g & 3);
        const float d = f16_bits_to_f32(w.d[j]);
        #pragma unroll
        for (int e = 0; e < 4; e++) v[e] = (float)(int8_t)((q >> (8 * e)) & 0xFFu) * d;
    }
};

// Q4_0_BARQ x Q8_0: the reference's own 20-byte layout (gguf.rs:521-578,
// quant/src/q4_0.rs:69-115): f32 scale, element 2i low / 2i+1 high nibble of
// byte i, sign-extended.
struct FmtQ40Barq {
    static constexpr int ROW_BLOCK_ELEMS = 32;
    static constexpr int ROW_BLOCK_BYTES = 20;
    using Lane = Pair32Lane;
    // activation bytes deinterleaved into even / odd elements per block
    struct X { uint32_t e[2][4], o[2][4]; int s[2]; float dx[2]; };
    struct Wt { uint4 q[2]; float sc[2]; };

    static __device__ __forceinline__ Lane lane(int l) { return {l}; }
    static __device__ __forceinline__ int blk(int it, const Lane& c) { return it * 128 + 2 * c.l; }
    static __device__ __forceinline__ bool active(int it, const Lane& c, int nblk) { return blk(it, c) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const uint8_t* __restrict__ xq, int it, const Lane& c, int nblk) {
        XQ80 r;
        load_x_q8_0(r, xq, blk(it, c), nblk);
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint4 lo = r.v[2 * j], hi = r.v[2 * j + 1];
            const uint32_t X8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                x.e[j][t] = __builtin_amdgcn_perm(X8[2 * t + 1], X8[2 * t], 0x06040200u);
                x.o[j][t] = __builtin_amdgcn_perm(X8[2 * t + 1], X8[2 * t], 0x07050301u);
            }
            x.s[j] = r.s[j];
            x.dx[j] = r.dx[j];
        }
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, const Lane& c, int nblk) {
        const int b = blk(it, c);
        const uint8_t* p = row + (size_t)b * 20;
        w.sc[0] = *reinterpret_cast<const float*>(p);
        w.q[0] = ld16_a4(p + 4);
        if (b + 1 < nblk) {
            w.sc[1] = *reinterpret_cast<const float*>(p + 20);
            w.q[1] = ld16_a4(p + 24);
        } else {
            w.sc[1] = 0.0f; w.q[1] = make_uint4(0, 0, 0, 0);
        }
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, const Lane&) {
        float r = 0.0f;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            int s = 0;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = u4get(w.q[j], t);
                // nibble n encodes q = sext(n); n ^ 8 = q + 8 in [0, 15]
                s = sdot4((q & M4) ^ 0x08080808u, x.e[j][t], s);
                s = sdot4(((q >> 4) & M4) ^ 0x08080808u, x.o[j][t], s);
            }
            r = __builtin_fmaf(w.sc[j] * x.dx[j], (float)(s - 8 * x.s[j]), r);
        }
        return r;
    }

    // literal: group g -> block g/8, dword (g%8)/2, bytes 2*(g%2), +1
    static __device__ __forceinline__ int xoff(int l, int g) { return 64 * l + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, const Lane&, int g, float v[4]) {
        const int j = g >> 3, gg = g & 7;
        const uint32_t q = u4get(w.q[j], gg >> 1) >> (16 * (gg & 1));
        const float sc = w.sc[j];
        #pragma unroll
        for (int e = 0; e < 4; e++) {
            const int n = (q >> (4 * e)) & 15;
            const int qs = n >= 8 ? n - 16 : n;
            v[e] = (float)qs * sc;
        }
    }
};

}  // namespace barq
