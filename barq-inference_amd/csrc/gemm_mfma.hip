// Batched K-quant x Q8_K GEMM on gfx950 int8 MFMA: Y[m, n] = sum_k X[m, k] W[n, k]
// for Q4_K and Q6_K weights (GGUF rows, blocks along k) and Q8_K activation
// rows with 16x16x64 tiles and register-staged loads.  gemm_kq.hip's
// 32x32x32 kernel takes every shape it supports; this one remains for Q6_K
// rows with an odd number of super-blocks (and for comparison runs with
// BARQ_GEMM_IMPL=0).
//
// Per workgroup: a tile of BM activation rows x 64 weight rows; per 256-element
// super-block, the Q8_K rows (int8 + scale + bsums) and the packed weight
// blocks are staged in LDS, each of the four waves unpacks the blocks of its
// 16 weight rows into int8 MFMA operands in registers and runs
// v_mfma_i32_16x16x64_i8 over the BM/16 activation tiles.
//
// Why two MFMA passes per super-block: a K-quant weight is d * s * q (minus a
// min term), where the per-sub-block integer scale s times the quant q is 10
// (Q4_K) or 13 (Q6_K) bits wide and so does not fit an int8 operand.
//   Q4_K: s = 8*s1 + s0 with s1, s0 in [0, 7]; s1*q and s0*q are <= 105 and
//         are formed four at a time by one packed 16-bit multiply (no carry
//         crosses a byte).  C = ((s1*q).x << 3) + (s0*q).x.
//   Q6_K: w' = s * (q - 32) in [-4064, 4096] is split as 128*h + l with
//         l in [0, 127] and h in [-32, 32].  C = ((h.x) << 7) + l.x.
// The Q4_K min term dmin * sum_k m_j(k) * x_k is one more int8 pass over the
// same activation fragments against the 6-bit mins broadcast over their
// 32-element sub-blocks (MFMA time is cheaper here than the VALU a separate
// bsum path would need).  The integer results are exact; the float epilogue
// per super-block is y += dx * (d * C - dmin * Cmin).
#include "common.hpp"
#include "launch.hpp"

#include <cstdio>
#include <cstdlib>

namespace barq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int GM_BN = 64;         // weight rows per workgroup: 4 waves x 16
constexpr int XQ_STRIDE = 272;    // LDS row stride of the int8 activation tile (256 + 16: no bank conflicts)

__device__ __forceinline__ uint32_t mul_u16x2(uint32_t a, uint32_t s) {
    const s16x2 r = __builtin_bit_cast(s16x2, a) * __builtin_bit_cast(s16x2, s);
    return __builtin_bit_cast(uint32_t, r);
}

// Raw buffer access: a 128-bit base/limit descriptor in SGPRs, a per-lane
// 32-bit offset and a wave-uniform offset.  Reads at or beyond the limit
// return zero, which pads ragged row tiles without per-row branches.
typedef __amdgpu_buffer_rsrc_t brsrc;
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ brsrc make_brsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(brsrc r, uint32_t voff, uint32_t soff) {
    const u32x4v v = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t bld4(brsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// ---------------------------------------------------------------------------
// Weight formats.  decode() produces, for lane (column n = l%16, k-group
// g = l/16) and MFMA step p (super-block elements 64p + 16g + [0, 16)), the
// high and low int8 operands of the two passes.
// ---------------------------------------------------------------------------
struct GQ4K {
    static constexpr int BB = Q4_K_BYTES;   // 144
    static constexpr int STRIDE = 144;      // LDS row stride
    static constexpr int CHUNKS = 9;        // 16-byte pieces per block
    static constexpr bool HAS_MIN = true;
    static constexpr int SHIFT = 3;

    // piece c of a block: 16-byte aligned (row bytes = 144 * k/256, base 16-aligned)
    static __device__ __forceinline__ uint4 chunk(brsrc r, uint32_t off, uint32_t soff, int) {
        return bld16(r, off, soff);
    }

    struct B {
        v4i h[4], l[4];
        int m[4];     // per step: the lane's sub-block min, broadcast to 4 bytes
        float d, dmin;
    };

    static __device__ __forceinline__ void decode(const uint8_t* wr, int g, B& b) {
        const uint4 hdr = *reinterpret_cast<const uint4*>(wr);
        b.d = f16_bits_to_f32(hdr.x & 0xFFFFu);
        b.dmin = f16_bits_to_f32(hdr.x >> 16);
        // get_scale_min_k4 (gguf.rs:825-837) for all eight sub-blocks, bytewise
        const uint32_t scA = hdr.y & 0x3F3F3F3Fu;
        const uint32_t scB = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
        const uint32_t mA = hdr.z & 0x3F3F3F3Fu;
        const uint32_t mB = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
        const int hi = g >> 1;
        const uint32_t nsh = 4u * (uint32_t)hi;
        #pragma unroll
        for (int p = 0; p < 4; p++) {
            // sub-block j = 2p + hi; sc byte (j & 3) of scA (j < 4) or scB
            const uint32_t sc = ((p < 2 ? scA : scB) >> (8 * ((2 * p + hi) & 3))) & 0xFFu;
            const uint32_t s1 = (sc >> 3) * 0x00010001u, s0 = (sc & 7u) * 0x00010001u;
            const uint4 qs = *reinterpret_cast<const uint4*>(wr + 16 + 32 * p + 16 * (g & 1));
            const uint32_t n0 = (qs.x >> nsh) & 0x0F0F0F0Fu, n1 = (qs.y >> nsh) & 0x0F0F0F0Fu;
            const uint32_t n2 = (qs.z >> nsh) & 0x0F0F0F0Fu, n3 = (qs.w >> nsh) & 0x0F0F0F0Fu;
            b.h[p] = v4i{(int)mul_u16x2(n0, s1), (int)mul_u16x2(n1, s1), (int)mul_u16x2(n2, s1), (int)mul_u16x2(n3, s1)};
            b.l[p] = v4i{(int)mul_u16x2(n0, s0), (int)mul_u16x2(n1, s0), (int)mul_u16x2(n2, s0), (int)mul_u16x2(n3, s0)};
            const uint32_t mj = ((p < 2 ? mA : mB) >> (8 * ((2 * p + hi) & 3))) & 0xFFu;
            b.m[p] = (int)(mj * 0x01010101u);
        }
    }
};

struct GQ6K {
    static constexpr int BB = Q6_K_BYTES;   // 210
    static constexpr int STRIDE = 224;
    static constexpr int CHUNKS = 14;       // 13 x 16 B + d
    static constexpr bool HAS_MIN = false;
    static constexpr int SHIFT = 7;

    // blocks are only 2-byte aligned: read the dword-aligned 20-byte window
    // and funnel-shift (pieces 0-12); piece 13 is the f16 d
    static __device__ __forceinline__ uint4 chunk(brsrc r, uint32_t off, uint32_t soff, int c) {
        const uint32_t o = off + soff, sh = o & 3u, a = o - sh;
        if (c == 13) {
            const uint32_t v = bld4(r, a, 0);
            return make_uint4(sh ? v >> 16 : v & 0xFFFFu, 0u, 0u, 0u);
        }
        const uint4 v = bld16(r, a, 0);
        const uint32_t e = bld4(r, a + 16u, 0);
        return make_uint4(__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                          __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh));
    }

    struct B {
        v4i h[4], l[4];
        int m[4];
        float d, dmin;
    };

    // w' = sc * (q - 32) as int16 pairs, split into h = w' >> 7 and l = w' & 127
    static __device__ __forceinline__ void split4(uint32_t q4, uint32_t scv, uint32_t off, int& h, int& l) {
        const uint32_t a = mul_u16x2(__builtin_amdgcn_perm(0u, q4, 0x0c010c00u), scv);
        const uint32_t c = mul_u16x2(__builtin_amdgcn_perm(0u, q4, 0x0c030c02u), scv);
        const s16x2 wa = __builtin_bit_cast(s16x2, a) + __builtin_bit_cast(s16x2, off);
        const s16x2 wc = __builtin_bit_cast(s16x2, c) + __builtin_bit_cast(s16x2, off);
        const s16x2 ha = wa >> (short)7, hc = wc >> (short)7;
        const s16x2 la = wa & (short)127, lc = wc & (short)127;
        h = (int)__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hc), __builtin_bit_cast(uint32_t, ha), 0x06040200u);
        l = (int)__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, lc), __builtin_bit_cast(uint32_t, la), 0x06040200u);
    }

    static __device__ __forceinline__ void decode(const uint8_t* wr, int g, B& b) {
        b.d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(wr + 208));
        b.dmin = 0.0f;
        const int g1 = g & 1;
        #pragma unroll
        for (int p = 0; p < 4; p++) {
            // element r = 64p + 16g + i: half h = p/2, quarter qd, position l = 16*g1 + i (gguf.rs:863-910)
            const int hh = p >> 1;
            const int qd = 2 * (p & 1) + (g >> 1);
            const uint4 ql = *reinterpret_cast<const uint4*>(wr + 64 * hh + 32 * (qd & 1) + 16 * g1);
            const uint4 qh = *reinterpret_cast<const uint4*>(wr + 128 + 32 * hh + 16 * g1);
            const int sc = (int)(int8_t)wr[192 + 8 * hh + g1 + 2 * qd];
            const uint32_t scv = ((uint32_t)sc & 0xFFFFu) * 0x00010001u;
            const uint32_t off = ((uint32_t)(-32 * sc) & 0xFFFFu) * 0x00010001u;
            const uint32_t nsh = qd >= 2 ? 4u : 0u, hsh = 2u * (uint32_t)qd;
            const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w}, qhw[4] = {qh.x, qh.y, qh.z, qh.w};
            int hv[4], lv[4];
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t q4 = ((qlw[i] >> nsh) & 0x0F0F0F0Fu) | (((qhw[i] >> hsh) & 0x03030303u) << 4);
                split4(q4, scv, off, hv[i], lv[i]);
            }
            b.h[p] = v4i{hv[0], hv[1], hv[2], hv[3]};
            b.l[p] = v4i{lv[0], lv[1], lv[2], lv[3]};
        }
    }
};

// ---------------------------------------------------------------------------
// One LDS stage holds super-block b of the tile: the int8 activation rows,
// their block scales, their split 32-element sums and the packed weight
// blocks.  Two stages alternate: while the waves run the MFMAs of stage b,
// the global loads of stage b+1 are in flight into registers; they are
// stored to the other stage afterwards, so one barrier per super-block
// separates the producers and consumers.
template <class F, int BM>
struct Stage {
    uint8_t xq[BM * XQ_STRIDE];
    float xd[BM];
    uint8_t w[GM_BN * F::STRIDE];
};

template <class F, int BM>
struct StageRegs {
    static constexpr int XQ_PER_T = BM / 16;                         // 16-byte activation pieces per thread
    static constexpr int W_PER_T = (GM_BN * F::CHUNKS + 255) / 256;  // 16-byte weight pieces per thread
    uint4 xq[XQ_PER_T];
    uint4 w[W_PER_T];
    float dx;         // block scale of the thread's row (threads < BM)
};

// Per-thread constant offsets of the stage loads (computed once per kernel).
template <class F, int BM>
struct StageAddr {
    uint32_t xq;                                  // activation piece (row t/16, 16 bytes at 16*(t%16))
    uint32_t xm;                                  // row t's block scale
    uint32_t w[StageRegs<F, BM>::W_PER_T];        // weight piece t + 256 i
};

template <class F, int BM>
__device__ __forceinline__ void stage_addr(StageAddr<F, BM>& a, size_t w_row_bytes, size_t x_row_bytes, int t) {
    a.xq = (uint32_t)(t >> 4) * (uint32_t)x_row_bytes + 4u + 16u * (uint32_t)(t & 15);
    a.xm = (uint32_t)t * (uint32_t)x_row_bytes;
    #pragma unroll
    for (int i = 0; i < StageRegs<F, BM>::W_PER_T; i++) {
        const int c = t + 256 * i, rr = c / F::CHUNKS, piece = c - rr * F::CHUNKS;
        a.w[i] = (uint32_t)rr * (uint32_t)w_row_bytes + 16u * (uint32_t)piece;
    }
}

// xr covers activation rows [m0, M) and wr weight rows [n0, N) of the tile;
// rows past the end read as zero.
template <class F, int BM>
__device__ __forceinline__ void stage_load(StageRegs<F, BM>& r, const StageAddr<F, BM>& a, brsrc wr, brsrc xr,
                                           uint32_t x_row_bytes, int b, int t) {
    const uint32_t xs = (uint32_t)b * Q8_K_BYTES;
    #pragma unroll
    for (int i = 0; i < StageRegs<F, BM>::XQ_PER_T; i++) r.xq[i] = bld16(xr, a.xq, xs + 16u * (uint32_t)i * x_row_bytes);
    if (t < BM) r.dx = __builtin_bit_cast(float, bld4(xr, a.xm, xs));
    const uint32_t ws = (uint32_t)b * F::BB;
    #pragma unroll
    for (int i = 0; i < StageRegs<F, BM>::W_PER_T; i++) {
        const int c = t + 256 * i;
        if (c < GM_BN * F::CHUNKS) r.w[i] = F::chunk(wr, a.w[i], ws, c % F::CHUNKS);
    }
}

template <class F, int BM>
__device__ __forceinline__ void stage_store(Stage<F, BM>& st, const StageRegs<F, BM>& r, int t) {
    #pragma unroll
    for (int i = 0; i < StageRegs<F, BM>::XQ_PER_T; i++)
        *reinterpret_cast<uint4*>(st.xq + ((t >> 4) + 16 * i) * XQ_STRIDE + 16 * (t & 15)) = r.xq[i];
    if (t < BM) st.xd[t] = r.dx;
    #pragma unroll
    for (int i = 0; i < StageRegs<F, BM>::W_PER_T; i++) {
        const int c = t + 256 * i;
        if (c < GM_BN * F::CHUNKS) {
            const int rr = c / F::CHUNKS, piece = c - rr * F::CHUNKS;
            *reinterpret_cast<uint4*>(st.w + rr * F::STRIDE + 16 * piece) = r.w[i];
        }
    }
}

// All BM/16 activation tiles' fragments are read first; the MFMAs then run
// step-major across tiles, so consecutive MFMAs are independent and the
// accumulation chains of different tiles hide each other's latency.
template <class F, int BM>
__device__ __forceinline__ void stage_compute(const Stage<F, BM>& st, float (&acc)[BM / 16][4], int wave, int g,
                                              int li) {
    constexpr int MT = BM / 16;
    typename F::B bw;
    F::decode(st.w + (16 * wave + li) * F::STRIDE, g, bw);
    v4i a[MT][4];
    #pragma unroll
    for (int i = 0; i < MT; i++) {
        const uint8_t* xr = st.xq + (16 * i + li) * XQ_STRIDE + 16 * g;
        #pragma unroll
        for (int p = 0; p < 4; p++) a[i][p] = *reinterpret_cast<const v4i*>(xr + 64 * p);
    }
    v4i c[MT];
    #pragma unroll
    for (int i = 0; i < MT; i++) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][0], bw.h[0], v4i{0, 0, 0, 0}, 0, 0, 0);
    #pragma unroll
    for (int p = 1; p < 4; p++) {
        #pragma unroll
        for (int i = 0; i < MT; i++) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][p], bw.h[p], c[i], 0, 0, 0);
    }
    #pragma unroll
    for (int i = 0; i < MT; i++) c[i] = c[i] << F::SHIFT;
    #pragma unroll
    for (int p = 0; p < 4; p++) {
        #pragma unroll
        for (int i = 0; i < MT; i++) c[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][p], bw.l[p], c[i], 0, 0, 0);
    }
    if (F::HAS_MIN) {
        v4i cm[MT];
        #pragma unroll
        for (int p = 0; p < 4; p++) {
            const v4i bm = {bw.m[p], bw.m[p], bw.m[p], bw.m[p]};
            #pragma unroll
            for (int i = 0; i < MT; i++)
                cm[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][p], bm, p ? cm[i] : v4i{0, 0, 0, 0}, 0, 0, 0);
        }
        #pragma unroll
        for (int i = 0; i < MT; i++) {
            const float4 dx = *reinterpret_cast<const float4*>(st.xd + 16 * i + 4 * g);
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const float v = __builtin_fmaf(-bw.dmin, (float)cm[i][r], bw.d * (float)c[i][r]);
                acc[i][r] = __builtin_fmaf(dxv[r], v, acc[i][r]);
            }
        }
    } else {
        #pragma unroll
        for (int i = 0; i < MT; i++) {
            const float4 dx = *reinterpret_cast<const float4*>(st.xd + 16 * i + 4 * g);
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
            #pragma unroll
            for (int r = 0; r < 4; r++) acc[i][r] = __builtin_fmaf(dxv[r], bw.d * (float)c[i][r], acc[i][r]);
        }
    }
}

template <class F, int BM>
__global__ __launch_bounds__(256, 1)
void gemm_kq_kernel(const uint8_t* __restrict__ W, size_t w_row_bytes, const uint8_t* __restrict__ X,
                    size_t x_row_bytes, float* __restrict__ Y, int M, int N, int nsb, int tiles_m, int n_tiles) {
    constexpr int MT = BM / 16;
    extern __shared__ __align__(16) uint8_t smem[];
    Stage<F, BM>* st = reinterpret_cast<Stage<F, BM>*>(smem);

    // XCD-aware order: workgroup i runs on XCD i % 8; give each XCD a
    // contiguous run of tiles so the activation rows of a weight tile's
    // neighbours share that XCD's L2.
    int tile = blockIdx.x;
    if ((n_tiles & 7) == 0) tile = (tile & 7) * (n_tiles >> 3) + (tile >> 3);
    const int mt = tile % tiles_m, ntile = tile / tiles_m;
    const int m0 = mt * BM, n0 = ntile * GM_BN;

    const int t = threadIdx.x, l = t & 63, wave = t >> 6, g = l >> 4, li = l & 15;

    float acc[MT][4];
    #pragma unroll
    for (int i = 0; i < MT; i++) acc[i][0] = acc[i][1] = acc[i][2] = acc[i][3] = 0.0f;

    // the tile's rows as buffers (the launcher keeps both limits below 2^32)
    const brsrc xr = make_brsrc(X + (size_t)m0 * x_row_bytes, (uint32_t)((size_t)(M - m0) * x_row_bytes));
    const brsrc wr = make_brsrc(W + (size_t)n0 * w_row_bytes, (uint32_t)((size_t)(N - n0) * w_row_bytes));
    StageAddr<F, BM> addr;
    stage_addr<F, BM>(addr, w_row_bytes, x_row_bytes, t);
    const uint32_t xrb = (uint32_t)x_row_bytes;

    // Super-block b+2's loads are issued while b is computed and b+1 waits
    // in the other register set, so each load has two iterations to land.
    StageRegs<F, BM> ra, rb;
    ra.dx = rb.dx = 0.0f;
    stage_load<F, BM>(ra, addr, wr, xr, xrb, 0, t);
    if (nsb > 1) stage_load<F, BM>(rb, addr, wr, xr, xrb, 1, t);
    stage_store<F, BM>(st[0], ra, t);
    __syncthreads();
    for (int b = 0; b < nsb; b += 2) {
        // even b: compute st[0]; rb holds b+1; reload ra with b+2
        if (b + 2 < nsb) stage_load<F, BM>(ra, addr, wr, xr, xrb, b + 2, t);
        stage_compute<F, BM>(st[0], acc, wave, g, li);
        if (b + 1 < nsb) stage_store<F, BM>(st[1], rb, t);
        __syncthreads();
        if (b + 1 >= nsb) break;
        // odd b+1: compute st[1]; ra holds b+2; reload rb with b+3
        if (b + 3 < nsb) stage_load<F, BM>(rb, addr, wr, xr, xrb, b + 3, t);
        stage_compute<F, BM>(st[1], acc, wave, g, li);
        if (b + 2 < nsb) stage_store<F, BM>(st[0], ra, t);
        __syncthreads();
    }

    // C layout of the 16x16 MFMA: lane (li, g) holds rows 4g + r of column li
    const int col = n0 + 16 * wave + li;
    if (col < N) {
        #pragma unroll
        for (int i = 0; i < MT; i++) {
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + 16 * i + 4 * g + r;
                if (row < M) __builtin_nontemporal_store(acc[i][r], &Y[(size_t)row * N + col]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K x Q8_K, v_mfma_i32_32x32x32_i8 (K = 32 = one Q4_K sub-block per MFMA).
//
// Workgroup tile BM activation rows x 128 weight rows; wave w owns weight
// rows [32w, 32w+32) and all BM activation rows (BM/32 MFMA tiles), so every
// weight sub-block is unpacked exactly once per workgroup.  NS LDS stages are
// filled by buffer->LDS direct loads (no VGPR staging), NS-1 super-blocks
// ahead of the MFMAs, with one barrier per super-block; rows past M or N read
// as zero from the range-checked buffers.  The activation tile is stored with
// its 16-byte chunks XOR-swizzled by row (chunk c of row r at c ^ (r & 15))
// so the fragment reads of 32 rows hit distinct banks.
//
// Per sub-block j and tile: Ch += x.(s1*q), Cl += x.(s0*q), Cm += x.m_j (three
// independent accumulation chains); per super-block C = 8*Ch + Cl and
// y += dx * (d*C - dmin*Cm).
// ---------------------------------------------------------------------------
// ---- launch ---------------------------------------------------------------

template <class F, int BM>
static hipError_t launch_kq(const uint8_t* W, size_t wrb, const uint8_t* X, size_t xrb, float* Y, int M, int N,
                            int nsb, hipStream_t s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + GM_BN - 1) / GM_BN;
    const int n_tiles = tiles_m * tiles_n;
    constexpr size_t lds = 2 * sizeof(Stage<F, BM>);
    // set once per template instance (thread-safe static init)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kq_kernel<F, BM>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((gemm_kq_kernel<F, BM>), dim3(n_tiles), dim3(256), lds, s, W, wrb, X, xrb, Y, M, N, nsb,
                       tiles_m, n_tiles);
    return hipGetLastError();
}

// Activation-tile height: the largest of 128/64/32/16 that still gives
// every CU two workgroups, never taller than M needs.
static int pick_bm(int M, int N) {
    if (const int o = tuning_env(TUNE_GEMM_BM)) return o;
    const int tiles_n = (N + GM_BN - 1) / GM_BN;
    int bm = 128;
    while (bm > 16 && (bm >= 2 * ((M + 15) / 16 * 16) || (long)tiles_n * ((M + bm - 1) / bm) < 512)) bm >>= 1;
    return bm;
}

// BARQ_GEMM_IMPL=0 selects this file's 16x16x64 kernel for every shape
// (comparison runs); by default gemm_kq.hip takes every shape it supports.

template <class F>
static hipError_t dispatch_kq(const void* W, size_t n_rows, size_t k, const void* xq, size_t m, float* y,
                              hipStream_t s) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const int nsb = (int)(k / 256);
    const size_t wrb = (size_t)nsb * F::BB, xrb = (size_t)nsb * Q8_K_BYTES;
    const int M = (int)m, N = (int)n_rows;
    switch (pick_bm(M, N)) {
    case 128: return launch_kq<F, 128>(w, wrb, x, xrb, y, M, N, nsb, s);
    case 64: return launch_kq<F, 64>(w, wrb, x, xrb, y, M, N, nsb, s);
    case 32: return launch_kq<F, 32>(w, wrb, x, xrb, y, M, N, nsb, s);
    default: return launch_kq<F, 16>(w, wrb, x, xrb, y, M, N, nsb, s);
    }
}

// The tile loads are raw buffer loads with 32-bit offsets: the weight matrix
// and the activation rows must each be below 2 GiB.
bool gemm_mfma_supported(int w_type, size_t n_rows, size_t k, size_t m) {
    if ((w_type != TYPE_Q4_K && w_type != TYPE_Q6_K) || k % 256 != 0 || n_rows == 0) return false;
    const size_t wbytes = n_rows * (k / 256) * (w_type == TYPE_Q4_K ? Q4_K_BYTES : Q6_K_BYTES);
    const size_t xbytes = m * (k / 256) * Q8_K_BYTES;
    return wbytes < (1ull << 31) && xbytes < (1ull << 31);
}

static bool use_kq(int w_type, size_t n_rows, size_t k, size_t m) {
    return tuning_env(TUNE_GEMM_IMPL, 2) != 0 && kq_supported(w_type, n_rows, k, m);
}

size_t gemm_mfma_workspace(int w_type, size_t n_rows, size_t k, size_t m) {
    return use_kq(w_type, n_rows, k, m) ? kq_workspace(w_type, m, n_rows, k) : 0;
}

hipError_t gemm_q8k_mfma_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m,
                                void* ws, float* y, hipStream_t s) {
    if (m == 0 || n_rows == 0) return hipSuccess;
    if (!gemm_mfma_supported(w_type, n_rows, k, m)) return hipErrorInvalidValue;
    if (use_kq(w_type, n_rows, k, m)) return kq_gemm_launch(w_type, W, n_rows, k, xq, m, ws, y, s);
    switch (w_type) {
    case TYPE_Q4_K: return dispatch_kq<GQ4K>(W, n_rows, k, xq, m, y, s);
    case TYPE_Q6_K: return dispatch_kq<GQ6K>(W, n_rows, k, xq, m, y, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace barq
