// Per-format lane slices for the batch-1 GEMV kernels.
//
// Every GEMV wave walks rows; inside a row, lane L owns the same 64 weights
// of each 4096-element K chunk ("iteration"), so its activation slice is
// loaded once per iteration and reused for all rows the wave handles.
//
//   Q4_K  (144 B / 256): lane -> super-block L/4, sub-block pair p = L%4:
//         header (d, dmin, 12 scale bytes) + qs[32p .. 32p+32).
//   Q6_K  (210 B / 256): lane -> block L/4, half h, 16-lane run lr:
//         ql[64h+lr..+16], ql[64h+32+lr..+16], qh[32h+lr..+16], 4 scales, d.
//   Q4_0  (18 B / 32), Q8_0 (34 B / 32), Q4_0_BARQ (20 B / 32):
//         lane -> two consecutive blocks (64 elements).
//
// Each format provides, for the integer (Q8 activation) path:
//   X              activation slice in registers
//   Wt             weight bytes in registers
//   load_x / load_w / dot
// and for the literal f32 path:
//   deq4(w, g, v)  the 4 weights of group g (g = 0..15), bit-identical to
//                  the reference decoders; xoff(lane, g) is their K offset
//                  inside the iteration.
#pragma once
#include "act_stage.hpp"

namespace barq {

constexpr uint32_t M4 = 0x0F0F0F0Fu;
constexpr uint32_t M30 = 0x30303030u;

__device__ __forceinline__ uint32_t u4get(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// ---------------------------------------------------------------------------
// Q4_K x Q8_K  (gguf.rs:730-837 decode; llama.cpp vec_dot_q4_K_q8_K math)
// ---------------------------------------------------------------------------
struct FmtQ4K {
    static constexpr int ACT_BLOCK = 256;
    static constexpr int ROW_BLOCK_ELEMS = 256;
    static constexpr int ROW_BLOCK_BYTES = 144;
    static constexpr int LANES_PER_BLOCK = 4;

    struct X { uint4 v[4]; int sa, sb; float dx; };
    struct Wt { uint4 hdr, q0, q1; };

    static __device__ __forceinline__ int blk(int it, int lane) { return it * 16 + (lane >> 2); }
    static __device__ __forceinline__ bool active(int it, int lane, int nblk) { return blk(it, lane) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const ActLds& a, int it, int lane) {
        int sb = blk(it, lane), p = lane & 3;
        const uint4* q = reinterpret_cast<const uint4*>(a.qs + sb * 256 + 64 * p);
        x.v[0] = q[0]; x.v[1] = q[1]; x.v[2] = q[2]; x.v[3] = q[3];
        const int* s = a.s16 + sb * 16 + 4 * p;
        x.sa = s[0] + s[1];
        x.sb = s[2] + s[3];
        x.dx = a.d[sb];
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, int lane) {
        const uint8_t* b = row + (size_t)blk(it, lane) * 144;
        int p = lane & 3;
        w.hdr = *reinterpret_cast<const uint4*>(b);
        w.q0 = *reinterpret_cast<const uint4*>(b + 16 + 32 * p);
        w.q1 = *reinterpret_cast<const uint4*>(b + 32 + 32 * p);
    }

    // (sc, m) of sub-blocks 2p and 2p+1: get_scale_min_k4 (gguf.rs:825-837)
    // with the 12 scale bytes in hdr.y (q[0..3]), hdr.z (q[4..7]), hdr.w (q[8..11]).
    static __device__ __forceinline__ void scales(const uint4& hdr, int p, int& sca, int& ma, int& scb, int& mb) {
        uint32_t s = 16u * (uint32_t)(p & 1);
        uint32_t t1 = hdr.y >> s, t2 = hdr.z >> s, t3 = hdr.w >> s;
        if (p < 2) {
            sca = t1 & 63; scb = (t1 >> 8) & 63;
            ma = t2 & 63; mb = (t2 >> 8) & 63;
        } else {
            sca = (t3 & 15) | ((t1 >> 2) & 48);
            scb = ((t3 >> 8) & 15) | ((t1 >> 10) & 48);
            ma = ((t3 >> 4) & 15) | ((t2 >> 2) & 48);
            mb = ((t3 >> 12) & 15) | ((t2 >> 10) & 48);
        }
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, int lane) {
        int sca, ma, scb, mb;
        scales(w.hdr, lane & 3, sca, ma, scb, mb);
        int ia = 0, ib = 0;
        ia = sdot4(w.q0.x & M4, x.v[0].x, ia); ia = sdot4(w.q0.y & M4, x.v[0].y, ia);
        ia = sdot4(w.q0.z & M4, x.v[0].z, ia); ia = sdot4(w.q0.w & M4, x.v[0].w, ia);
        ia = sdot4(w.q1.x & M4, x.v[1].x, ia); ia = sdot4(w.q1.y & M4, x.v[1].y, ia);
        ia = sdot4(w.q1.z & M4, x.v[1].z, ia); ia = sdot4(w.q1.w & M4, x.v[1].w, ia);
        ib = sdot4((w.q0.x >> 4) & M4, x.v[2].x, ib); ib = sdot4((w.q0.y >> 4) & M4, x.v[2].y, ib);
        ib = sdot4((w.q0.z >> 4) & M4, x.v[2].z, ib); ib = sdot4((w.q0.w >> 4) & M4, x.v[2].w, ib);
        ib = sdot4((w.q1.x >> 4) & M4, x.v[3].x, ib); ib = sdot4((w.q1.y >> 4) & M4, x.v[3].y, ib);
        ib = sdot4((w.q1.z >> 4) & M4, x.v[3].z, ib); ib = sdot4((w.q1.w >> 4) & M4, x.v[3].w, ib);
        int im = sca * ia + scb * ib;
        int in = ma * x.sa + mb * x.sb;
        float d = f16_bits_to_f32(w.hdr.x & 0xFFFFu);
        float dmin = f16_bits_to_f32(w.hdr.x >> 16);
        return x.dx * __builtin_fmaf(d, (float)im, -(dmin * (float)in));
    }

    // literal path: group g covers elements 64p + 4g .. +4 of super-block sb
    static __device__ __forceinline__ int xoff(int lane, int g) { return (lane >> 2) * 256 + 64 * (lane & 3) + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, int lane, int g, float v[4]) {
        int sca, ma, scb, mb;
        scales(w.hdr, lane & 3, sca, ma, scb, mb);
        float d = f16_bits_to_f32(w.hdr.x & 0xFFFFu);
        float dmin = f16_bits_to_f32(w.hdr.x >> 16);
        bool hi = g >= 8;
        float d1 = d * (float)(hi ? scb : sca);
        float m1 = dmin * (float)(hi ? mb : ma);
        int gg = g & 7;
        uint32_t q = u4get(gg < 4 ? w.q0 : w.q1, gg & 3);
        if (hi) q >>= 4;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            float p = d1 * (float)((q >> (8 * i)) & 15u);
            v[i] = p - m1;
        }
    }
};

// ---------------------------------------------------------------------------
// Q6_K x Q8_K  (gguf.rs:839-914 decode; llama.cpp vec_dot_q6_K_q8_K math)
// ---------------------------------------------------------------------------
struct FmtQ6K {
    static constexpr int ACT_BLOCK = 256;
    static constexpr int ROW_BLOCK_ELEMS = 256;
    static constexpr int ROW_BLOCK_BYTES = 210;
    static constexpr int LANES_PER_BLOCK = 4;

    struct X { uint4 v[4]; int bs32[4]; float dx; };
    struct Wt { uint4 a, b, h; uint2 sc; uint32_t d; };

    static __device__ __forceinline__ int blk(int it, int lane) { return it * 16 + (lane >> 2); }
    static __device__ __forceinline__ bool active(int it, int lane, int nblk) { return blk(it, lane) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const ActLds& a, int it, int lane) {
        int b = blk(it, lane), h = (lane >> 1) & 1, lr = 16 * (lane & 1);
        const int8_t* q = a.qs + b * 256 + 128 * h + lr;
        #pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            x.v[qd] = *reinterpret_cast<const uint4*>(q + 32 * qd);
            x.bs32[qd] = 32 * a.s16[b * 16 + 8 * h + 2 * qd + (lane & 1)];
        }
        x.dx = a.d[b];
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, int lane) {
        const uint8_t* b = row + (size_t)blk(it, lane) * 210;
        int h = (lane >> 1) & 1, lr = 16 * (lane & 1);
        w.a = ld16_a2(b + 64 * h + lr);
        w.b = ld16_a2(b + 64 * h + 32 + lr);
        w.h = ld16_a2(b + 128 + 32 * h + lr);
        w.sc = ld8_a2(b + 192 + 8 * h);
        w.d = ld_u16(b + 208);
    }

    // the lane's four i8 scales sc[8h + lr/16 + 2qd], qd = 0..3
    static __device__ __forceinline__ void scales(const Wt& w, int lane, int s[4]) {
        uint32_t o = 8u * (uint32_t)(lane & 1);
        s[0] = __builtin_amdgcn_sbfe(w.sc.x, o, 8);
        s[1] = __builtin_amdgcn_sbfe(w.sc.x, o + 16, 8);
        s[2] = __builtin_amdgcn_sbfe(w.sc.y, o, 8);
        s[3] = __builtin_amdgcn_sbfe(w.sc.y, o + 16, 8);
    }

    static __device__ __forceinline__ void unpack(uint32_t A, uint32_t B, uint32_t H, uint32_t q[4]) {
        q[0] = (A & M4) | ((H << 4) & M30);
        q[1] = (B & M4) | ((H << 2) & M30);
        q[2] = ((A >> 4) & M4) | (H & M30);
        q[3] = ((B >> 4) & M4) | ((H >> 2) & M30);
    }

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, int lane) {
        int i[4] = {0, 0, 0, 0};
        #pragma unroll
        for (int t = 0; t < 4; t++) {
            uint32_t q[4];
            unpack(u4get(w.a, t), u4get(w.b, t), u4get(w.h, t), q);
            #pragma unroll
            for (int qd = 0; qd < 4; qd++) i[qd] = sdot4(q[qd], u4get(x.v[qd], t), i[qd]);
        }
        int s[4];
        scales(w, lane, s);
        int tot = s[0] * (i[0] - x.bs32[0]) + s[1] * (i[1] - x.bs32[1]) +
                  s[2] * (i[2] - x.bs32[2]) + s[3] * (i[3] - x.bs32[3]);
        float d = f16_bits_to_f32(w.d);
        return (d * x.dx) * (float)tot;
    }

    // literal path: group g = 4*qd + t -> elements 128h + 32qd + lr + 4t
    static __device__ __forceinline__ int xoff(int lane, int g) {
        return (lane >> 2) * 256 + 128 * ((lane >> 1) & 1) + 32 * (g >> 2) + 16 * (lane & 1) + 4 * (g & 3);
    }
    static __device__ __forceinline__ void deq4(const Wt& w, int lane, int g, float v[4]) {
        int qd = g >> 2, t = g & 3;
        uint32_t q[4];
        unpack(u4get(w.a, t), u4get(w.b, t), u4get(w.h, t), q);
        int s[4];
        scales(w, lane, s);
        float d = f16_bits_to_f32(w.d);
        float dd = d * (float)s[qd];
        uint32_t qq = q[qd];
        #pragma unroll
        for (int e = 0; e < 4; e++) v[e] = dd * (float)((int)((qq >> (8 * e)) & 63u) - 32);
    }
};

// ---------------------------------------------------------------------------
// Q4_0 (GGUF) x Q8_0  (llama.cpp block_q4_0; parity with gguf.rs:521-578 via
// the byte adapter: both decode to (nib - 8) * d)
// ---------------------------------------------------------------------------
struct FmtQ40 {
    static constexpr int ACT_BLOCK = 32;
    static constexpr int ROW_BLOCK_ELEMS = 32;
    static constexpr int ROW_BLOCK_BYTES = 18;
    static constexpr int LANES_PER_BLOCK = 0;  // two blocks per lane

    struct X { uint4 v[4]; int s[2]; float dx[2]; };
    struct Wt { uint4 q[2]; uint32_t d[2]; };

    static __device__ __forceinline__ int blk(int it, int lane) { return it * 128 + 2 * lane; }
    static __device__ __forceinline__ bool active(int it, int lane, int nblk) { return blk(it, lane) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const ActLds& a, int it, int lane, int nblk) {
        int b = blk(it, lane);
        const uint4* q = reinterpret_cast<const uint4*>(a.qs + b * 32);
        bool two = b + 1 < nblk;
        x.v[0] = q[0]; x.v[1] = q[1];
        x.v[2] = two ? q[2] : make_uint4(0, 0, 0, 0);
        x.v[3] = two ? q[3] : make_uint4(0, 0, 0, 0);
        x.s[0] = a.s16[2 * b] + a.s16[2 * b + 1];
        x.s[1] = two ? a.s16[2 * b + 2] + a.s16[2 * b + 3] : 0;
        x.dx[0] = a.d[b];
        x.dx[1] = two ? a.d[b + 1] : 0.0f;
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, int lane, int nblk) {
        int b = blk(it, lane);
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

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, int) {
        float r = 0.0f;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            int s = 0;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                uint32_t q = u4get(w.q[j], t);
                s = sdot4(q & M4, u4get(x.v[2 * j], t), s);
                s = sdot4((q >> 4) & M4, u4get(x.v[2 * j + 1], t), s);
            }
            float dw = f16_bits_to_f32(w.d[j]);
            r = __builtin_fmaf(dw * x.dx[j], (float)(s - 8 * x.s[j]), r);
        }
        return r;
    }

    // literal: g<8 block 0, else block 1; gg<4 low nibbles of dword gg
    // (elements 4gg..), else high nibbles of dword gg-4 (elements 16+4(gg-4)..)
    static __device__ __forceinline__ int xoff(int lane, int g) { return 64 * lane + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, int, int g, float v[4]) {
        int j = g >> 3, gg = g & 7;
        uint32_t q = u4get(w.q[j], gg & 3);
        if (gg >= 4) q >>= 4;
        float d = f16_bits_to_f32(w.d[j]);
        #pragma unroll
        for (int e = 0; e < 4; e++) v[e] = (float)((int)((q >> (8 * e)) & 15u) - 8) * d;
    }
};

// ---------------------------------------------------------------------------
// Q8_0 x Q8_0  (gguf.rs:634-681 decode; llama.cpp vec_dot_q8_0_q8_0 math)
// ---------------------------------------------------------------------------
struct FmtQ80 {
    static constexpr int ACT_BLOCK = 32;
    static constexpr int ROW_BLOCK_ELEMS = 32;
    static constexpr int ROW_BLOCK_BYTES = 34;
    static constexpr int LANES_PER_BLOCK = 0;

    struct X { uint4 v[4]; float dx[2]; };
    struct Wt { uint4 q[4]; uint32_t d[2]; };

    static __device__ __forceinline__ int blk(int it, int lane) { return it * 128 + 2 * lane; }
    static __device__ __forceinline__ bool active(int it, int lane, int nblk) { return blk(it, lane) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const ActLds& a, int it, int lane, int nblk) {
        int b = blk(it, lane);
        const uint4* q = reinterpret_cast<const uint4*>(a.qs + b * 32);
        bool two = b + 1 < nblk;
        x.v[0] = q[0]; x.v[1] = q[1];
        x.v[2] = two ? q[2] : make_uint4(0, 0, 0, 0);
        x.v[3] = two ? q[3] : make_uint4(0, 0, 0, 0);
        x.dx[0] = a.d[b];
        x.dx[1] = two ? a.d[b + 1] : 0.0f;
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, int lane, int nblk) {
        int b = blk(it, lane);
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

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, int) {
        float r = 0.0f;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            int s = 0;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                s = sdot4(u4get(w.q[2 * j], t), u4get(x.v[2 * j], t), s);
                s = sdot4(u4get(w.q[2 * j + 1], t), u4get(x.v[2 * j + 1], t), s);
            }
            float dw = f16_bits_to_f32(w.d[j]);
            r = __builtin_fmaf(dw * x.dx[j], (float)s, r);
        }
        return r;
    }

    static __device__ __forceinline__ int xoff(int lane, int g) { return 64 * lane + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, int, int g, float v[4]) {
        int j = g >> 3;
        uint32_t q = u4get(w.q[g >> 2], g & 3);
        float d = f16_bits_to_f32(w.d[j]);
        #pragma unroll
        for (int e = 0; e < 4; e++) v[e] = (float)(int8_t)((q >> (8 * e)) & 0xFFu) * d;
    }
};

// ---------------------------------------------------------------------------
// Q4_0_BARQ x Q8_0: the reference's own 20-byte layout (gguf.rs:521-578,
// quant/src/q4_0.rs:69-115): f32 scale, element 2i low / 2i+1 high nibble of
// byte i, sign-extended.
// ---------------------------------------------------------------------------
struct FmtQ40Barq {
    static constexpr int ACT_BLOCK = 32;
    static constexpr int ROW_BLOCK_ELEMS = 32;
    static constexpr int ROW_BLOCK_BYTES = 20;
    static constexpr int LANES_PER_BLOCK = 0;

    // activation bytes deinterleaved into even / odd elements per block
    struct X { uint32_t e[2][4], o[2][4]; int s[2]; float dx[2]; };
    struct Wt { uint4 q[2]; float sc[2]; };

    static __device__ __forceinline__ int blk(int it, int lane) { return it * 128 + 2 * lane; }
    static __device__ __forceinline__ bool active(int it, int lane, int nblk) { return blk(it, lane) < nblk; }

    static __device__ __forceinline__ void load_x(X& x, const ActLds& a, int it, int lane, int nblk) {
        int b = blk(it, lane);
        const uint4* q = reinterpret_cast<const uint4*>(a.qs + b * 32);
        bool two = b + 1 < nblk;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            uint4 lo = (j == 0 || two) ? q[2 * j] : make_uint4(0, 0, 0, 0);
            uint4 hi = (j == 0 || two) ? q[2 * j + 1] : make_uint4(0, 0, 0, 0);
            uint32_t X8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                x.e[j][t] = __builtin_amdgcn_perm(X8[2 * t + 1], X8[2 * t], 0x06040200u);
                x.o[j][t] = __builtin_amdgcn_perm(X8[2 * t + 1], X8[2 * t], 0x07050301u);
            }
        }
        x.s[0] = a.s16[2 * b] + a.s16[2 * b + 1];
        x.s[1] = two ? a.s16[2 * b + 2] + a.s16[2 * b + 3] : 0;
        x.dx[0] = a.d[b];
        x.dx[1] = two ? a.d[b + 1] : 0.0f;
    }

    static __device__ __forceinline__ void load_w(Wt& w, const uint8_t* row, int it, int lane, int nblk) {
        int b = blk(it, lane);
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

    static __device__ __forceinline__ float dot(const Wt& w, const X& x, int) {
        float r = 0.0f;
        #pragma unroll
        for (int j = 0; j < 2; j++) {
            int s = 0;
            #pragma unroll
            for (int t = 0; t < 4; t++) {
                uint32_t q = u4get(w.q[j], t);
                // nibble n encodes q = sext(n); n ^ 8 = q + 8 in [0, 15]
                s = sdot4((q & M4) ^ 0x08080808u, x.e[j][t], s);
                s = sdot4(((q >> 4) & M4) ^ 0x08080808u, x.o[j][t], s);
            }
            r = __builtin_fmaf(w.sc[j] * x.dx[j], (float)(s - 8 * x.s[j]), r);
        }
        return r;
    }

    // literal: group g -> block g/8, dword (g%8)/2, bytes 2*(g%2), +1
    static __device__ __forceinline__ int xoff(int lane, int g) { return 64 * lane + 4 * g; }
    static __device__ __forceinline__ void deq4(const Wt& w, int, int g, float v[4]) {
        int j = g >> 3, gg = g & 7;
        uint32_t q = u4get(w.q[j], gg >> 1) >> (16 * (gg & 1));
        float sc = w.sc[j];
        #pragma unroll
        for (int e = 0; e < 4; e++) {
            int n = (q >> (4 * e)) & 15;
            int qs = n >= 8 ? n - 16 : n;
            v[e] = (float)qs * sc;
        }
    }
};

}  // namespace barq
