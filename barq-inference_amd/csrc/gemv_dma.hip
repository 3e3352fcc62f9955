// Batch-1 quantized GEMV with coalesced weight streaming (gfx950).
//
// GGUF blocks are 18, 20, 34, 144 or 210 bytes, so the per-lane loads of a
// register-direct GEMV are often only 2-byte aligned and every row costs
// many partially overlapping memory instructions.  Here each wave copies
// whole 4096-element row slices into its own LDS buffers with buffer->LDS
// direct loads (every lane 16 contiguous bytes per instruction), D slices
// ahead of the arithmetic, and the lanes then read their part of the blocks
// from LDS with aligned loads (plus a funnel shift where a block starts 2
// bytes past a dword).  Q6_K slices are copied as one 27-chunk window per
// block pair (420 bytes), so every block starts 0 or 2 bytes past a 16-byte
// LDS boundary.  The activation vector is staged in LDS once per workgroup
// (Q8_K blocks with quants, bsums and scale on 16-byte boundaries; Q8_0 as
// is).
//
// The per-lane arithmetic is the register GEMV's (FmtQ4K::dot etc.): the
// same integer dot products, scale handling and reduction.
#include "gemv_formats.hpp"
#include "launch.hpp"
#include "mfma_common.hpp"

namespace barq {

// 16 bytes at p + sh, p 16-byte aligned, sh in {0, 2}
__device__ __forceinline__ uint4 lds_rd16(const uint8_t* p, uint32_t sh) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t e = *reinterpret_cast<const uint32_t*>(p + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                      __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh));
}

typedef uint32_t u32a4 __attribute__((aligned(4)));

// N dwords from a 4-byte aligned LDS address
template <int N>
__device__ __forceinline__ void lds_dwords(const uint8_t* p, uint32_t (&w)[N]) {
    #pragma unroll
    for (int i = 0; i < N; i++) w[i] = reinterpret_cast<const u32a4*>(p)[i];
}

__device__ __forceinline__ uint4 shift2(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t e) {
    return make_uint4(__builtin_amdgcn_alignbyte(b, a, 2), __builtin_amdgcn_alignbyte(c, b, 2),
                      __builtin_amdgcn_alignbyte(d, c, 2), __builtin_amdgcn_alignbyte(e, d, 2));
}

constexpr uint32_t DMA_SKIP = 0x80000000u;   // per-lane offset past every descriptor's range: loads zeros

// ---- staged activation layouts ---------------------------------------------
// Q8_K: each 292-byte block as 19 chunks: quants 0..15 (16-byte aligned),
// bsums in chunks 16-17, the f32 scale at byte 288.
struct XStageQ8K {
    static constexpr int BLK_ELEMS = 256;
    static __device__ __forceinline__ int chunks(int nblk) { return nblk * 19; }
    static __device__ __forceinline__ uint32_t src(int j, int nblk) {
        const int b = j / 19, c = j - b * 19;
        if (b >= nblk) return DMA_SKIP;
        return (uint32_t)b * Q8_K_BYTES + (c < 16 ? 4u + 16u * c : c < 18 ? 260u + 16u * (c - 16) : 0u);
    }
    static __device__ __forceinline__ const uint8_t* blk(const uint8_t* xs, int b) { return xs + 304 * b; }
};
// Q8_0: the 34-byte blocks copied as they are (pairs of blocks are 4-byte aligned)
struct XStageQ80 {
    static constexpr int BLK_ELEMS = 32;
    static __device__ __forceinline__ int chunks(int nblk) { return (nblk * Q8_0_BYTES + 15) / 16; }
    static __device__ __forceinline__ uint32_t src(int j, int nblk) {
        return j < chunks(nblk) ? 16u * (uint32_t)j : DMA_SKIP;
    }
};

// Q8_0 activation of a block pair (2b, 2b + 1) from its 17 dwords (68 bytes
// at 68 b)
__device__ __forceinline__ void q8_0_pair_from_dwords(XQ80& x, const uint32_t (&w)[17]) {
    x.dx[0] = f16_bits_to_f32(w[0] & 0xFFFFu);
    x.v[0] = shift2(w[0], w[1], w[2], w[3], w[4]);
    x.v[1] = shift2(w[4], w[5], w[6], w[7], w[8]);
    x.dx[1] = f16_bits_to_f32(w[8] >> 16);
    x.v[2] = make_uint4(w[9], w[10], w[11], w[12]);
    x.v[3] = make_uint4(w[13], w[14], w[15], w[16]);
    x.s[0] = bytesum16(x.v[0]) + bytesum16(x.v[1]);
    x.s[1] = bytesum16(x.v[2]) + bytesum16(x.v[3]);
}

// Q8_0 activation of lane l's block pair (2b, 2b + 1) from the staged copy
__device__ __forceinline__ void stage_x_q8_0(XQ80& x, const uint8_t* xs, int b) {
    uint32_t w[17];
    lds_dwords<17>(xs + 34 * b, w);
    q8_0_pair_from_dwords(x, w);
}

// ---- weight slice layouts (4096 elements of one row per slice) ------------
// Q6_K: eight 27-chunk windows, one per block pair, so each block starts 0 or
// 2 bytes past a 16-byte boundary of the LDS copy.
struct DQ6K {
    using F = FmtQ6K;
    using XS = XStageQ8K;
    static constexpr int SLICE_BLOCKS = 16, SLICE_BYTES = 16 * Q6_K_BYTES, SLICE_INSTR = 4;
    static __device__ __forceinline__ uint32_t slice_src(int i) {
        const int p = i / 27, c = i - p * 27;
        return p < 8 ? (uint32_t)(420 * p + 16 * c) : DMA_SKIP;
    }
    static __device__ __forceinline__ void load_w(F::Wt& w, const uint8_t* sl, const F::Lane& c) {
        const uint32_t sh = 2u * (uint32_t)(c.bl & 1);
        const uint8_t* blk = sl + 432 * (c.bl >> 1) + 208 * (c.bl & 1);
        w.a = lds_rd16(blk + 64 * c.h + c.lr, sh);
        w.b = lds_rd16(blk + 64 * c.h + 32 + c.lr, sh);
        w.h = lds_rd16(blk + 128 + 32 * c.h + c.lr, sh);
        const uint2 s2 = *reinterpret_cast<const uint2*>(blk + 192 + 8 * c.h);
        const uint32_t e = *reinterpret_cast<const uint32_t*>(blk + 200 + 8 * c.h);
        w.sc = make_uint2(__builtin_amdgcn_alignbyte(s2.y, s2.x, sh), __builtin_amdgcn_alignbyte(e, s2.y, sh));
        const uint32_t dw = *reinterpret_cast<const uint32_t*>(blk + 208);
        w.d = sh ? dw >> 16 : dw & 0xFFFFu;
    }
    static __device__ __forceinline__ void load_x(F::X& x, const uint8_t* xs, int it, const F::Lane& c, int nblk) {
        const int b = it * 16 + c.bl;
        const uint8_t* xb = XS::blk(xs, b < nblk ? b : 0);
        x.dx = *reinterpret_cast<const float*>(xb + 288);
        #pragma unroll
        for (int qd = 0; qd < 4; qd++) x.v[qd] = *reinterpret_cast<const uint4*>(xb + 16 * (8 * c.h + c.s0 + 2 * qd));
        const uint4 bs = *reinterpret_cast<const uint4*>(xb + 16 * (16 + c.h));
        const uint32_t o = 16u * (uint32_t)c.s0;
        x.bs32[0] = 32 * sext16(bs.x, o);
        x.bs32[1] = 32 * sext16(bs.y, o);
        x.bs32[2] = 32 * sext16(bs.z, o);
        x.bs32[3] = 32 * sext16(bs.w, o);
    }
};

// Q4_K: the slice is 144 contiguous 16-byte aligned chunks
struct DQ4K {
    using F = FmtQ4K;
    using XS = XStageQ8K;
    static constexpr int SLICE_BLOCKS = 16, SLICE_BYTES = 16 * Q4_K_BYTES, SLICE_INSTR = 3;
    static __device__ __forceinline__ uint32_t slice_src(int i) { return i < 144 ? 16u * (uint32_t)i : DMA_SKIP; }
    static __device__ __forceinline__ void load_w(F::Wt& w, const uint8_t* sl, const F::Lane& c) {
        const uint8_t* b = sl + 144 * c.sbl;
        w.hdr = *reinterpret_cast<const uint4*>(b);
        w.q0 = *reinterpret_cast<const uint4*>(b + 16 + 32 * c.p);
        w.q1 = *reinterpret_cast<const uint4*>(b + 32 + 32 * c.p);
    }
    static __device__ __forceinline__ void load_x(F::X& x, const uint8_t* xs, int it, const F::Lane& c, int nblk) {
        const int b = it * 16 + c.sbl;
        const uint8_t* xb = XS::blk(xs, b < nblk ? b : 0);
        x.dx = *reinterpret_cast<const float*>(xb + 288);
        #pragma unroll
        for (int i = 0; i < 4; i++) x.v[i] = *reinterpret_cast<const uint4*>(xb + 16 * (4 * c.p + i));
        const uint2 bs = *reinterpret_cast<const uint2*>(xb + 16 * (16 + (c.p >> 1)) + 8 * (c.p & 1));
        x.sa = sext16(bs.x, 0) + sext16(bs.x, 16);
        x.sb = sext16(bs.y, 0) + sext16(bs.y, 16);
    }
};

// Q4_0 (18-byte blocks): lane l's block pair is 36 bytes at 36 l
struct DQ40 {
    using F = FmtQ40;
    using XS = XStageQ80;
    static constexpr int SLICE_BLOCKS = 128, SLICE_BYTES = 128 * Q4_0_BYTES, SLICE_INSTR = 3;
    static __device__ __forceinline__ uint32_t slice_src(int i) { return i < 144 ? 16u * (uint32_t)i : DMA_SKIP; }
    static __device__ __forceinline__ void load_w(F::Wt& w, const uint8_t* sl, const F::Lane& c) {
        uint32_t v[9];
        lds_dwords<9>(sl + 36 * c.l, v);
        w.d[0] = v[0] & 0xFFFFu;
        w.q[0] = shift2(v[0], v[1], v[2], v[3], v[4]);
        w.d[1] = v[4] >> 16;
        w.q[1] = make_uint4(v[5], v[6], v[7], v[8]);
    }
    static __device__ __forceinline__ void load_x(F::X& x, const uint8_t* xs, int it, const F::Lane& c, int nblk) {
        const int b = it * 128 + 2 * c.l;
        stage_x_q8_0(x, xs, b < nblk ? b : 0);
    }
    static __device__ __forceinline__ void x_from_pair(F::X& x, const XQ80& r) { x = r; }
};

// Q8_0 weights (34-byte blocks): lane l's block pair is 68 bytes at 68 l
struct DQ80 {
    using F = FmtQ80;
    using XS = XStageQ80;
    static constexpr int SLICE_BLOCKS = 128, SLICE_BYTES = 128 * Q8_0_BYTES, SLICE_INSTR = 5;
    static __device__ __forceinline__ uint32_t slice_src(int i) { return i < 272 ? 16u * (uint32_t)i : DMA_SKIP; }
    static __device__ __forceinline__ void load_w(F::Wt& w, const uint8_t* sl, const F::Lane& c) {
        uint32_t v[17];
        lds_dwords<17>(sl + 68 * c.l, v);
        w.d[0] = v[0] & 0xFFFFu;
        w.q[0] = shift2(v[0], v[1], v[2], v[3], v[4]);
        w.q[1] = shift2(v[4], v[5], v[6], v[7], v[8]);
        w.d[1] = v[8] >> 16;
        w.q[2] = make_uint4(v[9], v[10], v[11], v[12]);
        w.q[3] = make_uint4(v[13], v[14], v[15], v[16]);
    }
    static __device__ __forceinline__ void load_x(F::X& x, const uint8_t* xs, int it, const F::Lane& c, int nblk) {
        const int b = it * 128 + 2 * c.l;
        stage_x_q8_0(x, xs, b < nblk ? b : 0);
    }
    static __device__ __forceinline__ void x_from_pair(F::X& x, const XQ80& r) { x = r; }
};

// Q4_0_BARQ (20-byte blocks): lane l's block pair is 40 bytes at 40 l
struct DQ40B {
    using F = FmtQ40Barq;
    using XS = XStageQ80;
    static constexpr int SLICE_BLOCKS = 128, SLICE_BYTES = 128 * Q4_0_BARQ_BYTES, SLICE_INSTR = 3;
    static __device__ __forceinline__ uint32_t slice_src(int i) { return i < 160 ? 16u * (uint32_t)i : DMA_SKIP; }
    static __device__ __forceinline__ void load_w(F::Wt& w, const uint8_t* sl, const F::Lane& c) {
        uint32_t v[10];
        lds_dwords<10>(sl + 40 * c.l, v);
        w.sc[0] = __builtin_bit_cast(float, v[0]);
        w.q[0] = make_uint4(v[1], v[2], v[3], v[4]);
        w.sc[1] = __builtin_bit_cast(float, v[5]);
        w.q[1] = make_uint4(v[6], v[7], v[8], v[9]);
    }
    static __device__ __forceinline__ void load_x(F::X& x, const uint8_t* xs, int it, const F::Lane& c, int nblk) {
        const int b = it * 128 + 2 * c.l;
        XQ80 r;
        stage_x_q8_0(r, xs, b < nblk ? b : 0);
        x_from_pair(x, r);
    }
    // the even / odd activation bytes of the pair, for the split nibble layout
    static __device__ __forceinline__ void x_from_pair(F::X& x, const XQ80& r) {
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
};

// W waves per workgroup, R rows per wave, D slices in flight per wave; NX
// activation rows (tokens), each staged in its own x_region of LDS and dotted
// with every weight slice, so the weights are streamed once for all of them
// (y is [NX x n_rows]).
template <class P, int W, int R, int D, int NX = 1>
__global__ __launch_bounds__(W * 64)
void gemv_dma_kernel(const uint8_t* __restrict__ Wq, uint32_t rb, const uint8_t* __restrict__ xq, uint32_t x_bytes,
                     float* __restrict__ y, int n_rows, int nblk, uint32_t x_region) {
    using F = typename P::F;
    constexpr int SI = P::SLICE_INSTR, SL = 1024 * SI;
    static_assert(R % D == 0, "slice buffers rotate with the row index");
    extern __shared__ __align__(16) uint8_t smem[];
    const int l = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * W + wave) * R;
    const int n_it = (nblk + P::SLICE_BLOCKS - 1) / P::SLICE_BLOCKS;
    uint8_t* xs = smem;
    uint8_t* bufs = smem + NX * x_region + wave * (D * SL);

    // activation: every wave copies part of it (each token's row with its own
    // descriptor, so reads past a row return zeros as for one token)
    {
        const int n_instr = (P::XS::chunks(nblk) + 63) / 64;
        for (int q = wave; q < NX * n_instr; q += W) {
            const int j = q / n_instr, qq = q - j * n_instr;
            const i32x4v xr = make_rsrc4(xq + (size_t)j * x_bytes, x_bytes);
            lds_load16(xr, xs + (size_t)j * x_region + 1024 * qq, P::XS::src(64 * qq + l, nblk), 0);
        }
    }
    const bool live = row0 < n_rows;
    const int rows_here = live ? min(R, n_rows - row0) : 1;
    const i32x4v wr = make_rsrc4(Wq + (size_t)(live ? row0 : 0) * rb, (uint32_t)rows_here * rb);
    uint32_t voff[SI];
    #pragma unroll
    for (int q = 0; q < SI; q++) voff[q] = P::slice_src(64 * q + l);
    // the whole offset goes in the per-lane operand, which the descriptor's
    // range check covers: reads past this wave's rows return zeros
    auto issue = [&](int u) {
        const int it = u / R, r = u - it * R;
        const uint32_t so = (uint32_t)r * rb + (uint32_t)it * P::SLICE_BYTES;
        uint8_t* dst = bufs + (u % D) * SL;
        #pragma unroll
        for (int q = 0; q < SI; q++) lds_load16_nt(wr, dst + 1024 * q, voff[q] == DMA_SKIP ? DMA_SKIP : voff[q] + so, 0);
    };
    const int U = n_it * R;   // >= R >= D
    if (live) {
        #pragma unroll
        for (int u = 0; u < D; u++) issue(u);
        wait_vmcnt<SI * (D - 1)>();   // this wave's activation part and first slice
    } else {
        wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (!live) return;   // after the barrier: the other waves needed this wave's activation part

    const typename F::Lane c = F::lane(l);
    constexpr int NA = NX * R;   // token j, row r at j * R + r
    float acc[NA];
    #pragma unroll
    for (int i = 0; i < NA; i++) acc[i] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        const bool act = F::active(it, c, nblk);
        typename F::X x[NX];
        #pragma unroll
        for (int j = 0; j < NX; j++) P::load_x(x[j], xs + (size_t)j * x_region, it, c, nblk);
        #pragma unroll
        for (int r = 0; r < R; r++) {
            const int u = it * R + r;
            if (u > 0) {
                if (u + D - 1 < U) wait_vmcnt<SI * (D - 1)>();
                else wait_vmcnt<0>();
                asm volatile("" ::: "memory");
            }
            typename F::Wt w;
            P::load_w(w, bufs + (r % D) * SL, c);
            #pragma unroll
            for (int j = 0; j < NX; j++) {
                const float v = F::dot(w, x[j], c);
                if (act) acc[j * R + r] += v;
            }
            // the slice buffer is reused for unit u + D once its values are in registers
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (u + D < U) issue(u + D);
        }
    }

    #pragma unroll
    for (int g = 0; g < NA; g += 4) {
        const float v = reduce4(acc[g], g + 1 < NA ? acc[g + 1] : 0.0f, g + 2 < NA ? acc[g + 2] : 0.0f,
                                g + 3 < NA ? acc[g + 3] : 0.0f);
        if ((l & 15) == 0) {
            const int f = g + (l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3);
            const int j = f / R, rr = f - j * R;
            if (f < NA && row0 + rr < n_rows) y[(size_t)j * n_rows + row0 + rr] = v;
        }
    }
}

// ---- 32-element formats, two rows per wave (k <= 4096) ----------------------------
// The LDS-staged Q4_K rows' scheme (gemv.hip) for Q4_0, Q8_0 and Q4_0_BARQ:
// each wave copies its two rows (2 * rb contiguous bytes: 4608, 8704 and
// 5120 at k = 4096) into its own LDS buffer with whole-line non-temporal
// buffer->LDS loads; its lanes load their Q8_0 activation block pair (68
// bytes) into registers by inline-asm global loads issued before the copies
// (the compiler does not count them, so no wait of its own holds the copies
// back; nothing may touch these registers before the explicit wait, which
// the build's assembly check enforces), and row 0's arithmetic runs once its
// copies have landed.  No workgroup barrier.  The lane slicing, arithmetic
// and reduction are gemv_dma_kernel<P, W, 1, 1>'s: the outputs are
// bit-identical.
template <class P, int R = 2>
constexpr int pair32_buf = (R * 128 * P::F::ROW_BLOCK_BYTES + 1023) / 1024 * 1024;

struct Q80XRaw {
    i32x4v v[4];
    int e;
};

__device__ __forceinline__ void q80_x_issue(Q80XRaw& r, const uint8_t* __restrict__ xq, int pair) {
    const uint8_t* p = xq + (size_t)pair * 68;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r.v[0]) : "v"(p));
    asm volatile("global_load_dwordx4 %0, %1, off offset:16" : "=v"(r.v[1]) : "v"(p));
    asm volatile("global_load_dwordx4 %0, %1, off offset:32" : "=v"(r.v[2]) : "v"(p));
    asm volatile("global_load_dwordx4 %0, %1, off offset:48" : "=v"(r.v[3]) : "v"(p));
    asm volatile("global_load_dword %0, %1, off offset:64" : "=v"(r.e) : "v"(p));
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 4]
__device__ __forceinline__ void wait_vmcnt_upto4(uint32_t n) {
    switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    default: wait_vmcnt<4>(); break;
    }
}

// NX = 2-4 activation rows (x_row_bytes apart; y is [NX x n_rows]): every
// row's block pair is loaded ahead of the copies and each (token, row)
// product computed the same way, so y[j] equals the one-token GEMV of
// activation row j bit for bit.  R = 1: one weight row per wave (row 0's
// arithmetic and reduction unchanged, so the same bits).
template <class P, int WAVES, int NX = 1, int R = 2>
__global__ __launch_bounds__(WAVES * 64)
void gemv_pair32_kernel(const uint8_t* __restrict__ W, uint32_t w_bytes, const uint8_t* __restrict__ xq,
                        float* __restrict__ y, int n_rows, int nblk, uint32_t x_row_bytes) {
    using F = typename P::F;
    static_assert(R == 1 || R == 2, "one or two rows per wave");
    constexpr int BUF = pair32_buf<P, R>;
    __shared__ __align__(16) uint8_t lds[WAVES][BUF];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    uint8_t* buf = lds[wave];
    // every lane loads (lanes past the last pair re-read it and ignore it)
    Q80XRaw xr[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) q80_x_issue(xr[j], xq + (size_t)j * x_row_bytes, min(l, nblk / 2 - 1));
    const uint32_t rb = (uint32_t)nblk * F::ROW_BLOCK_BYTES, span = R * rb;
    const i32x4v rs = make_rsrc4(W, w_bytes);
    const uint32_t base = (uint32_t)row0 * rb;
    // every copy instruction is issued (a constant count; lanes past the
    // span read out of range)
    #pragma unroll
    for (int q = 0; q < BUF / 1024; q++) {
        const uint32_t off = 1024u * q + 16u * (uint32_t)l;
        lds_load16_nt(rs, buf + 1024 * q, off < span ? base + off : DMA_SKIP, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const typename F::Lane c = F::lane(l);
    const bool act = F::active(0, c, nblk);
    // copies issued after the last one row 0 needs (at most 4)
    wait_vmcnt_upto4(BUF / 1024 - (rb + 1023) / 1024);
    // the activation loads precede every copy (a constant wait the one above
    // implies, which the build's assembly check can verify on every path)
    wait_vmcnt<BUF / 1024>();
    asm volatile("" ::: "memory");
    typename F::X x[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) {
        Q80XRaw& q = xr[j];
        asm volatile("" : "+v"(q.v[0]), "+v"(q.v[1]), "+v"(q.v[2]), "+v"(q.v[3]), "+v"(q.e));
        const uint32_t w[17] = {(uint32_t)q.v[0].x, (uint32_t)q.v[0].y, (uint32_t)q.v[0].z, (uint32_t)q.v[0].w,
                                (uint32_t)q.v[1].x, (uint32_t)q.v[1].y, (uint32_t)q.v[1].z, (uint32_t)q.v[1].w,
                                (uint32_t)q.v[2].x, (uint32_t)q.v[2].y, (uint32_t)q.v[2].z, (uint32_t)q.v[2].w,
                                (uint32_t)q.v[3].x, (uint32_t)q.v[3].y, (uint32_t)q.v[3].z, (uint32_t)q.v[3].w,
                                (uint32_t)q.e};
        XQ80 r;
        q8_0_pair_from_dwords(r, w);
        P::x_from_pair(x[j], r);
    }
    float acc[2 * NX];   // token j, row r at 2 j + r
    #pragma unroll
    for (int i = 0; i < 2 * NX; i++) acc[i] = 0.0f;
    if (act) {
        typename F::Wt w;
        P::load_w(w, buf, c);
        #pragma unroll
        for (int j = 0; j < NX; j++) acc[2 * j] = F::dot(w, x[j], c);
    }
    if constexpr (R == 2) {
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        if (act) {
            typename F::Wt w;
            P::load_w(w, buf + rb, c);
            #pragma unroll
            for (int j = 0; j < NX; j++) acc[2 * j + 1] = F::dot(w, x[j], c);
        }
    }
    if constexpr (NX == 1) {
        const float v = reduce4(acc[0], acc[1], 0.0f, 0.0f);
        if ((l & 31) == 0) {
            const int rr = l >> 5;
            if (rr < R && row0 + rr < n_rows) y[row0 + rr] = v;
        }
    } else {
        constexpr int NA = 2 * NX;
        #pragma unroll
        for (int g = 0; g < NA; g += 4) {
            const float v = reduce4(acc[g], acc[g + 1], g + 2 < NA ? acc[g + 2] : 0.0f, g + 3 < NA ? acc[g + 3] : 0.0f);
            if ((l & 15) == 0) {
                const int f = g + (l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3);
                const int j = f >> 1, rr = f & 1;
                if (f < NA && rr < R && row0 + rr < n_rows) y[(size_t)j * n_rows + row0 + rr] = v;
            }
        }
    }
}

// ---- Q6_K, two rows per wave (k <= 4096) ------------------------------------------
// The same scheme for Q6_K: each of the wave's two rows is copied as
// gemv_dma_kernel's slice (eight 27-chunk windows, one per block pair, so
// every block starts 0 or 2 bytes past a 16-byte boundary), the rows 3456
// bytes apart in the wave's LDS buffer; the lane's Q8_K activation slice
// (FmtQ6K's lane slicing) comes from inline-asm global loads issued before
// the copies.  The outputs are gemv_dma_kernel<DQ6K, ...>'s, bit for bit.
constexpr int Q6P_ROW = 8 * 432, Q6P_BUF = 7 * 1024;

struct Q6XRaw {
    i32x4v v[4];
    i32x4v bs;
    int dx;
};

__device__ __forceinline__ void q6_x_issue(Q6XRaw& r, const uint8_t* __restrict__ xq, int blk, const FmtQ6K::Lane& c) {
    const uint8_t* b = xq + (size_t)blk * 292;
    const uint8_t* bq = b + 128 * c.h + c.lr;   // quants of this lane at +4 + 128 h + lr + 32 qd
    const uint8_t* bb = b + 16 * c.h;           // its bsums at +260 + 16 h
    asm volatile("global_load_dword %0, %1, off" : "=v"(r.dx) : "v"(b));
    asm volatile("global_load_dwordx4 %0, %1, off offset:4" : "=v"(r.v[0]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:36" : "=v"(r.v[1]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:68" : "=v"(r.v[2]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:100" : "=v"(r.v[3]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:260" : "=v"(r.bs) : "v"(bb));
}

// FmtQ6K::X from the loaded registers, after the wait that covers them (the
// empty asm keeps the compiler from reading them earlier)
__device__ __forceinline__ void q6_x_ready(Q6XRaw& xr, FmtQ6K::X& x, const FmtQ6K::Lane& c) {
    asm volatile("" : "+v"(xr.v[0]), "+v"(xr.v[1]), "+v"(xr.v[2]), "+v"(xr.v[3]), "+v"(xr.bs), "+v"(xr.dx));
    #pragma unroll
    for (int qd = 0; qd < 4; qd++)
        x.v[qd] = make_uint4((uint32_t)xr.v[qd].x, (uint32_t)xr.v[qd].y, (uint32_t)xr.v[qd].z, (uint32_t)xr.v[qd].w);
    x.dx = __builtin_bit_cast(float, xr.dx);
    const uint32_t off = 16u * (uint32_t)c.s0;
    x.bs32[0] = 32 * sext16((uint32_t)xr.bs.x, off);
    x.bs32[1] = 32 * sext16((uint32_t)xr.bs.y, off);
    x.bs32[2] = 32 * sext16((uint32_t)xr.bs.z, off);
    x.bs32[3] = 32 * sext16((uint32_t)xr.bs.w, off);
}

//
// NX = 2-4 activation rows (a small decode batch; x_row_bytes apart, y is
// [NX x n_rows]): the wave loads its lanes' slice of every activation row
// ahead of the copies and computes each (token, row) product the same way, so
// y[j] equals the one-token GEMV of activation row j bit for bit.
template <int WAVES, int NX = 1>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q6k_pair_kernel(const uint8_t* __restrict__ W, uint32_t w_bytes, const uint8_t* __restrict__ xq,
                          float* __restrict__ y, int n_rows, int nblk, uint32_t x_row_bytes) {
    using F = FmtQ6K;
    __shared__ __align__(16) uint8_t lds[WAVES][Q6P_BUF];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * 2;
    if (row0 >= n_rows) return;
    uint8_t* buf = lds[wave];
    const F::Lane c = F::lane(l);
    // every lane loads (lanes past the last block re-read it and ignore it)
    Q6XRaw xr[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) q6_x_issue(xr[j], xq + (size_t)j * x_row_bytes, min(c.bl, nblk - 1), c);
    const uint32_t rb = (uint32_t)nblk * Q6_K_BYTES, base = (uint32_t)row0 * rb;
    const int npair = nblk / 2;
    const i32x4v rs = make_rsrc4(W, w_bytes);
    #pragma unroll
    for (int q = 0; q < Q6P_BUF / 1024; q++) {
        const int i = 64 * q + l, r = i / 216, j = i - 216 * r, p = j / 27, ch = j - 27 * p;
        const uint32_t src = r < 2 && p < npair ? base + (uint32_t)r * rb + 420u * (uint32_t)p + 16u * (uint32_t)ch
                                                : DMA_SKIP;
        lds_load16_nt(rs, buf + 1024 * q, src, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const bool act = F::active(0, c, nblk);
    // row 0's windows end at byte 3456: copies 0-3; copies 4-6 are row 1's
    wait_vmcnt<3>();
    asm volatile("" ::: "memory");
    F::X x[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) q6_x_ready(xr[j], x[j], c);
    float acc[2 * NX];   // token j, row r at 2 j + r
    #pragma unroll
    for (int i = 0; i < 2 * NX; i++) acc[i] = 0.0f;
    if (act) {
        F::Wt w;
        DQ6K::load_w(w, buf, c);
        #pragma unroll
        for (int j = 0; j < NX; j++) acc[2 * j] = F::dot(w, x[j], c);
    }
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    if (act) {
        F::Wt w;
        DQ6K::load_w(w, buf + Q6P_ROW, c);
        #pragma unroll
        for (int j = 0; j < NX; j++) acc[2 * j + 1] = F::dot(w, x[j], c);
    }
    if constexpr (NX == 1) {
        const float v = reduce4(acc[0], acc[1], 0.0f, 0.0f);
        if ((l & 31) == 0) {
            const int rr = l >> 5;
            if (row0 + rr < n_rows) y[row0 + rr] = v;
        }
    } else {
        constexpr int NA = 2 * NX;
        #pragma unroll
        for (int g = 0; g < NA; g += 4) {
            const float v = reduce4(acc[g], acc[g + 1], g + 2 < NA ? acc[g + 2] : 0.0f, g + 3 < NA ? acc[g + 3] : 0.0f);
            if ((l & 15) == 0) {
                const int f = g + (l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3);
                const int j = f >> 1, rr = f & 1;
                if (f < NA && row0 + rr < n_rows) y[(size_t)j * n_rows + row0 + rr] = v;
            }
        }
    }
}

// Whether the Q6_K two-row kernel takes a one-token GEMV (k <= 4096;
// BARQ_GEMV_LDS=0 keeps gemv_dma_kernel).  Measured on one box, paired runs,
// us per call: C3 (128256 x 4096) 62.9-63.5 against 64.4-64.6, 14336 x 4096
// 9.9-10.0 against 11.3, 4096 x 4096 4.56-4.59 against 5.03.
static bool q6k_pair_path(size_t n_rows, size_t k) {
    return k > 0 && k <= 4096 && k % 512 == 0 && n_rows * (k / 256 * Q6_K_BYTES) < 0x80000000ull &&
           tuning_env(TUNE_GEMV_LDS, 1) != 0;
}

// Whether a two-row kernel of the 32-element formats takes a one-token GEMV
// (k <= 4096 and a multiple of 256, so rows are whole 16-byte chunks;
// BARQ_GEMV_LDS=0 keeps gemv_dma_kernel).  Measured at C1 (Q4_0 4096 x 4096,
// four paired runs on one box): 3.70-3.71 against 3.89-3.91 us.
static bool pair32_path(const void* W, size_t n_rows, size_t k, int blk_bytes) {
    return k > 0 && k <= 4096 && k % 256 == 0 && ((uintptr_t)W & 15) == 0 &&
           n_rows * (k / 32 * (size_t)blk_bytes) < 0x80000000ull && tuning_env(TUNE_GEMV_LDS, 1) != 0;
}

template <class P>
static hipError_t pair32_launch(const void* W, size_t n_rows, size_t k, const void* xq, float* y, hipStream_t s,
                                size_t m) {
    constexpr int WAVES = 4;
    const dim3 grid((unsigned)((n_rows + 2 * WAVES - 1) / (2 * WAVES))), block(WAVES * 64);
    const uint8_t* w8 = static_cast<const uint8_t*>(W);
    const uint8_t* x8 = static_cast<const uint8_t*>(xq);
    const uint32_t wb = (uint32_t)(n_rows * (k / 32 * P::F::ROW_BLOCK_BYTES)), xrb = (uint32_t)(k / 32 * Q8_0_BYTES);
    const int n = (int)n_rows, nb = (int)(k / 32);
    // one token: one weight row per wave up to 1024 rows (measured in one
    // process, us per call, one row against two: Q4_0 1024 x 4096 2.56 /
    // 2.68, 4096 x 4096 3.76 / 3.66, 6144 x 4096 4.62 / 4.30; Q8_0 and the
    // reference's Q4_0 at 4096 x 4096 4.77 / 4.53 and 3.92 / 3.84; outputs
    // bit-identical).  BARQ_GEMV_LDS = 2 / 3 force two / one.
    const int mode = tuning_env(TUNE_GEMV_LDS, 1);
    if (m == 1 && (mode == 3 || (mode == 1 && n_rows <= 1024))) {
        const dim3 grid1((unsigned)((n_rows + WAVES - 1) / WAVES));
        hipLaunchKernelGGL((gemv_pair32_kernel<P, WAVES, 1, 1>), grid1, block, 0, s, w8, wb, x8, y, n, nb, xrb);
        return hipGetLastError();
    }
    switch (m) {
    case 1: hipLaunchKernelGGL((gemv_pair32_kernel<P, WAVES, 1>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
    case 2: hipLaunchKernelGGL((gemv_pair32_kernel<P, WAVES, 2>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
    case 3: hipLaunchKernelGGL((gemv_pair32_kernel<P, WAVES, 3>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
    default: hipLaunchKernelGGL((gemv_pair32_kernel<P, WAVES, 4>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
    }
    return hipGetLastError();
}

// ---- launch ------------------------------------------------------------------
// tuning: BARQ_GEMV_DMA = W*100+R*10+D selects another launch shape (e.g. 842); -1 turns the path off

template <class P, int W, int R, int D, int NX = 1>
static hipError_t launch_dma(const uint8_t* Wq, uint32_t rb, size_t n_rows, int nblk, const uint8_t* xq,
                             uint32_t x_bytes, uint32_t x_region, float* y, hipStream_t s) {
    const size_t lds = (size_t)NX * x_region + (size_t)W * D * 1024 * P::SLICE_INSTR;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    // the whole 160 KiB enabled once per instance (thread-safe static init),
    // so concurrent callers never lower it below their own launch
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_dma_kernel<P, W, R, D, NX>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    const unsigned grid = (unsigned)((n_rows + (size_t)W * R - 1) / ((size_t)W * R));
    hipLaunchKernelGGL((gemv_dma_kernel<P, W, R, D, NX>), dim3(grid), dim3(W * 64), lds, s, Wq, rb, xq, x_bytes, y,
                       (int)n_rows, nblk, x_region);
    return hipGetLastError();
}

// The default launch shapes for NX tokens (several tokens: no tuning cases).
template <class P, int NX>
static hipError_t launch_dma_default(const uint8_t* w, uint32_t rb, size_t n_rows, int nblk, const uint8_t* x,
                                     uint32_t x_bytes, uint32_t x_region, float* y, hipStream_t s) {
    // measured on MI355X: four rows per wave for the 128256-row Q6_K head
    // (C3); eight waves of one row each for a few thousand rows (a 4096 x
    // 14336 down projection: 9.85-9.88 against 10.24-10.31 us, alternating
    // runs in one process; the token count of a multi-token call is not
    // tuned); for the 32-element formats one row per wave (more workgroups)
    // up to 8192 rows (C1: 3.82 against 3.94 us), two above
    if constexpr (P::SLICE_BLOCKS == 16) {
        if (NX == 1 && n_rows <= 8192) return launch_dma<P, 8, 1, 1, NX>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
        return launch_dma<P, 4, 4, 2, NX>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    } else if (n_rows <= 8192) {
        return launch_dma<P, 4, 1, 1, NX>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    } else {
        return launch_dma<P, 4, 2, 2, NX>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    }
}

template <class P>
static hipError_t dispatch_dma(const void* W, size_t n_rows, size_t k, const void* xq, float* y, hipStream_t s,
                               int blk_bytes, int x_blk_bytes, size_t m) {
    const int nblk = (int)(k / (P::SLICE_BLOCKS == 16 ? 256 : 32));
    const uint32_t rb = (uint32_t)(nblk * blk_bytes);
    const int xnb = P::XS::BLK_ELEMS == 256 ? (int)(k / 256) : nblk;
    const uint32_t x_bytes = (uint32_t)(xnb * x_blk_bytes);
    const int xch = P::SLICE_BLOCKS == 16 ? xnb * 19 : (xnb * x_blk_bytes + 15) / 16;
    const uint32_t x_region = (uint32_t)((xch + 63) / 64 * 1024);
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    switch (m) {
    case 1: break;
    case 2: return launch_dma_default<P, 2>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    case 3: return launch_dma_default<P, 3>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    case 4: return launch_dma_default<P, 4>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    default: return hipErrorInvalidValue;
    }
#define BARQ_DMA_CASE(WW, RR, DD) \
    case WW * 100 + RR * 10 + DD: return launch_dma<P, WW, RR, DD>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    switch (tuning_env(TUNE_GEMV_DMA)) {
    BARQ_DMA_CASE(4, 2, 2) BARQ_DMA_CASE(4, 4, 4) BARQ_DMA_CASE(4, 8, 2) BARQ_DMA_CASE(8, 2, 2)
    BARQ_DMA_CASE(8, 4, 2) BARQ_DMA_CASE(2, 2, 2) BARQ_DMA_CASE(2, 4, 2) BARQ_DMA_CASE(4, 1, 1)
    BARQ_DMA_CASE(8, 1, 1)
    default: return launch_dma_default<P, 1>(w, rb, n_rows, nblk, x, x_bytes, x_region, y, s);
    }
#undef BARQ_DMA_CASE
}

// Rows are streamed in 4096-element slices: weight rows and the activation
// must be 4-byte aligned, a Q6_K row must hold an even number of blocks (so
// block pairs start on 4-byte boundaries), the 32-element formats need whole
// block pairs per lane, offsets within one wave's rows stay below 2 GiB and
// the staged activation fits in LDS beside the slice buffers.
bool gemv_dma_supported(int w_type, const void* W, size_t n_rows, size_t k, const void* xq) {
    if (tuning_env(TUNE_GEMV_DMA) < 0 || k == 0 || n_rows > (size_t)INT32_MAX) return false;
    if (((uintptr_t)W & 3) || ((uintptr_t)xq & 3)) return false;
    size_t rb = 0, xch = 0;
    switch (w_type) {
    case TYPE_Q6_K: if (k % 512) return false; rb = k / 256 * Q6_K_BYTES; xch = k / 256 * 19; break;
    case TYPE_Q4_K: if (k % 256) return false; rb = k / 256 * Q4_K_BYTES; xch = k / 256 * 19; break;
    case TYPE_Q4_0: if (k % 64) return false; rb = k / 32 * Q4_0_BYTES; xch = (k / 32 * Q8_0_BYTES + 15) / 16; break;
    case TYPE_Q8_0: if (k % 64) return false; rb = k / 32 * Q8_0_BYTES; xch = (k / 32 * Q8_0_BYTES + 15) / 16; break;
    case TYPE_Q4_0_BARQ: if (k % 64) return false; rb = k / 32 * Q4_0_BARQ_BYTES; xch = (k / 32 * Q8_0_BYTES + 15) / 16; break;
    default: return false;
    }
    return rb * 8 < (1ull << 31) && (xch + 63) / 64 * 1024 <= 96 * 1024;
}

// m tokens (1-4); y is [m x n_rows]
hipError_t gemv_dma_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, float* y,
                           hipStream_t s, size_t m) {
    if (n_rows == 0) return hipSuccess;
    switch (w_type) {
    case TYPE_Q6_K:
        if (m <= 4 && q6k_pair_path(n_rows, k)) {
            constexpr int WAVES = 4;
            const dim3 grid((unsigned)((n_rows + 2 * WAVES - 1) / (2 * WAVES))), block(WAVES * 64);
            const uint32_t wb = (uint32_t)(n_rows * (k / 256 * Q6_K_BYTES)), xrb = (uint32_t)(k / 256 * Q8_K_BYTES);
            const uint8_t* w8 = static_cast<const uint8_t*>(W);
            const uint8_t* x8 = static_cast<const uint8_t*>(xq);
            const int n = (int)n_rows, nb = (int)(k / 256);
            switch (m) {
            case 1: hipLaunchKernelGGL((gemv_q6k_pair_kernel<WAVES, 1>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
            case 2: hipLaunchKernelGGL((gemv_q6k_pair_kernel<WAVES, 2>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
            case 3: hipLaunchKernelGGL((gemv_q6k_pair_kernel<WAVES, 3>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
            default: hipLaunchKernelGGL((gemv_q6k_pair_kernel<WAVES, 4>), grid, block, 0, s, w8, wb, x8, y, n, nb, xrb); break;
            }
            return hipGetLastError();
        }
        return dispatch_dma<DQ6K>(W, n_rows, k, xq, y, s, Q6_K_BYTES, Q8_K_BYTES, m);
    case TYPE_Q4_K: return dispatch_dma<DQ4K>(W, n_rows, k, xq, y, s, Q4_K_BYTES, Q8_K_BYTES, m);
    case TYPE_Q4_0:
        if (m <= 4 && pair32_path(W, n_rows, k, Q4_0_BYTES)) return pair32_launch<DQ40>(W, n_rows, k, xq, y, s, m);
        return dispatch_dma<DQ40>(W, n_rows, k, xq, y, s, Q4_0_BYTES, Q8_0_BYTES, m);
    case TYPE_Q8_0:
        if (m <= 4 && pair32_path(W, n_rows, k, Q8_0_BYTES)) return pair32_launch<DQ80>(W, n_rows, k, xq, y, s, m);
        return dispatch_dma<DQ80>(W, n_rows, k, xq, y, s, Q8_0_BYTES, Q8_0_BYTES, m);
    case TYPE_Q4_0_BARQ:
        if (m <= 4 && pair32_path(W, n_rows, k, Q4_0_BARQ_BYTES)) return pair32_launch<DQ40B>(W, n_rows, k, xq, y, s, m);
        return dispatch_dma<DQ40B>(W, n_rows, k, xq, y, s, Q4_0_BARQ_BYTES, Q8_0_BYTES, m);
    default: return hipErrorInvalidValue;
    }
}

// The staged rows of m tokens fit LDS beside the default slice buffers
// (gemv_dma_supported bounds one token's at 96 KiB).
bool gemv_dma_multi_fits(int w_type, size_t k, size_t m) {
    const size_t xch = w_type == TYPE_Q6_K || w_type == TYPE_Q4_K ? k / 256 * 19 : (k / 32 * Q8_0_BYTES + 15) / 16;
    return m * ((xch + 63) / 64 * 1024) <= 96 * 1024;
}

}  // namespace barq
