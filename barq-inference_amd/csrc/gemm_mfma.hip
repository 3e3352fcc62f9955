// Batched K-quant x Q8_K GEMM on gfx950 int8 MFMA: Y[m, n] = sum_k X[m, k] W[n, k]
// for Q4_K and Q6_K weights (GGUF rows, blocks along k) and Q8_K activation
// rows.  This is the prefill / MoE-expert-group path (M >= 16); it computes
// the same quantity as the batch-1 GEMV, row by row.
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
// The Q4_K min term dmin * sum_j m_j * sum_{i in sub-block j} x_i uses the
// activation's 32-element sums split the same way (s = 128*bh + bl) in a
// v_mfma_i32_16x16x32_i8 pair.  The integer results are exact; the float
// epilogue per super-block is y += dx * (d * C - dmin * Cmin).
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

    // global block rows are 16-byte aligned (row bytes = 144 * k/256, base 16-aligned)
    static __device__ __forceinline__ uint4 chunk(const uint8_t* blk, int c) {
        return *reinterpret_cast<const uint4*>(blk + 16 * c);
    }

    struct B {
        v4i h[4], l[4];
        long mn;      // mins m_0..m_7 (lanes of k-group 0), else 0
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
        }
        b.mn = g == 0 ? (long)(((uint64_t)mB << 32) | mA) : 0;
    }
};

struct GQ6K {
    static constexpr int BB = Q6_K_BYTES;   // 210
    static constexpr int STRIDE = 224;
    static constexpr int CHUNKS = 14;       // 13 x 16 B + d
    static constexpr bool HAS_MIN = false;
    static constexpr int SHIFT = 7;

    // block rows are only 2-byte aligned
    static __device__ __forceinline__ uint4 chunk(const uint8_t* blk, int c) {
        if (c < 13) return ld16_a2(blk + 16 * c);
        return make_uint4(ld_u16(blk + 208), 0u, 0u, 0u);
    }

    struct B {
        v4i h[4], l[4];
        long mn;
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
        b.mn = 0;
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
template <class F, int BM>
__global__ __launch_bounds__(256, 2)
void gemm_kq_kernel(const uint8_t* __restrict__ W, size_t w_row_bytes, const uint8_t* __restrict__ X,
                    size_t x_row_bytes, float* __restrict__ Y, int M, int N, int nsb, int tiles_m, int n_tiles) {
    constexpr int MT = BM / 16;
    __shared__ __align__(16) uint8_t s_xq[BM * XQ_STRIDE];
    __shared__ __align__(16) uint8_t s_xmin[BM * 16];
    __shared__ __align__(16) float s_xd[BM];
    __shared__ __align__(16) uint8_t s_w[GM_BN * F::STRIDE];

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

    for (int b = 0; b < nsb; b++) {
        if (b) __syncthreads();
        // ---- stage super-block b: activation rows ----
        #pragma unroll
        for (int i = 0; i < MT; i++) {
            const int r = (t >> 4) + 16 * i, row = m0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < M) v = ld16_a4(X + (size_t)row * x_row_bytes + (size_t)b * Q8_K_BYTES + 4 + 16 * (t & 15));
            *reinterpret_cast<uint4*>(s_xq + r * XQ_STRIDE + 16 * (t & 15)) = v;
        }
        for (int r = t; r < BM; r += 256) {
            const int row = m0 + r;
            float dx = 0.0f;
            uint4 mm = make_uint4(0, 0, 0, 0);
            if (row < M) {
                const uint8_t* blk = X + (size_t)row * x_row_bytes + (size_t)b * Q8_K_BYTES;
                dx = *reinterpret_cast<const float*>(blk);
                if (F::HAS_MIN) {
                    const uint4 s0 = ld16_a4(blk + 260), s1 = ld16_a4(blk + 276);
                    const uint32_t w[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
                    uint32_t bh[2] = {0, 0}, bl[2] = {0, 0};
                    #pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int s = __builtin_amdgcn_sbfe((int)w[j], 0, 16) + __builtin_amdgcn_sbfe((int)w[j], 16, 16);
                        bh[j >> 2] |= ((uint32_t)(s >> 7) & 0xFFu) << (8 * (j & 3));
                        bl[j >> 2] |= ((uint32_t)s & 0x7Fu) << (8 * (j & 3));
                    }
                    mm = make_uint4(bh[0], bh[1], bl[0], bl[1]);
                }
            }
            s_xd[r] = dx;
            *reinterpret_cast<uint4*>(s_xmin + 16 * r) = mm;
        }
        // ---- weight rows ----
        for (int c = t; c < GM_BN * F::CHUNKS; c += 256) {
            const int r = c / F::CHUNKS, piece = c - r * F::CHUNKS, row = n0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < N) v = F::chunk(W + (size_t)row * w_row_bytes + (size_t)b * F::BB, piece);
            *reinterpret_cast<uint4*>(s_w + r * F::STRIDE + 16 * piece) = v;
        }
        __syncthreads();

        // ---- compute ----
        typename F::B bw;
        F::decode(s_w + (16 * wave + li) * F::STRIDE, g, bw);
        #pragma unroll
        for (int i = 0; i < MT; i++) {
            const uint8_t* xr = s_xq + (16 * i + li) * XQ_STRIDE + 16 * g;
            v4i a[4];
            #pragma unroll
            for (int p = 0; p < 4; p++) a[p] = *reinterpret_cast<const v4i*>(xr + 64 * p);
            v4i c = {0, 0, 0, 0};
            #pragma unroll
            for (int p = 0; p < 4; p++) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[p], bw.h[p], c, 0, 0, 0);
            c = c << F::SHIFT;
            #pragma unroll
            for (int p = 0; p < 4; p++) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[p], bw.l[p], c, 0, 0, 0);
            const float4 dx = *reinterpret_cast<const float4*>(s_xd + 16 * i + 4 * g);
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
            if (F::HAS_MIN) {
                const uint4 mm = *reinterpret_cast<const uint4*>(s_xmin + 16 * (16 * i + li));
                const long ah = (long)(((uint64_t)mm.y << 32) | mm.x);
                const long al = (long)(((uint64_t)mm.w << 32) | mm.z);
                v4i cm = {0, 0, 0, 0};
                cm = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, bw.mn, cm, 0, 0, 0);
                cm = cm << 7;
                cm = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, bw.mn, cm, 0, 0, 0);
                #pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float v = __builtin_fmaf(-bw.dmin, (float)cm[r], bw.d * (float)c[r]);
                    acc[i][r] = __builtin_fmaf(dxv[r], v, acc[i][r]);
                }
            } else {
                #pragma unroll
                for (int r = 0; r < 4; r++) acc[i][r] = __builtin_fmaf(dxv[r], bw.d * (float)c[r], acc[i][r]);
            }
        }
    }

    // C layout of the 16x16 MFMA: lane (li, g) holds rows 4g + r of column li
    const int col = n0 + 16 * wave + li;
    if (col < N) {
        #pragma unroll
        for (int i = 0; i < MT; i++) {
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + 16 * i + 4 * g + r;
                if (row < M) Y[(size_t)row * N + col] = acc[i][r];
            }
        }
    }
}

// ---- launch ---------------------------------------------------------------
static int read_env_bm() {
    if (const char* e = getenv("BARQ_GEMM_BM")) return atoi(e);
    return 0;
}
static int g_bm_override = read_env_bm();

template <class F, int BM>
static hipError_t launch_kq(const uint8_t* W, size_t wrb, const uint8_t* X, size_t xrb, float* Y, int M, int N,
                            int nsb, hipStream_t s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + GM_BN - 1) / GM_BN;
    const int n_tiles = tiles_m * tiles_n;
    hipLaunchKernelGGL((gemm_kq_kernel<F, BM>), dim3(n_tiles), dim3(256), 0, s, W, wrb, X, xrb, Y, M, N, nsb,
                       tiles_m, n_tiles);
    return hipGetLastError();
}

// Activation-tile height: the largest of 128/64/32/16 that still gives
// every CU two workgroups, never taller than M needs.
static int pick_bm(int M, int N) {
    if (g_bm_override) return g_bm_override;
    const int tiles_n = (N + GM_BN - 1) / GM_BN;
    int bm = 128;
    while (bm > 16 && (bm >= 2 * ((M + 15) / 16 * 16) || (long)tiles_n * ((M + bm - 1) / bm) < 512)) bm >>= 1;
    return bm;
}

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

bool gemm_mfma_supported(int w_type, size_t n_rows, size_t k) {
    return (w_type == TYPE_Q4_K || w_type == TYPE_Q6_K) && k % 256 == 0 && n_rows > 0 &&
           n_rows <= (size_t)INT32_MAX;
}

hipError_t gemm_q8k_mfma_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m,
                                float* y, hipStream_t s) {
    if (m == 0 || n_rows == 0) return hipSuccess;
    switch (w_type) {
    case TYPE_Q4_K: return dispatch_kq<GQ4K>(W, n_rows, k, xq, m, y, s);
    case TYPE_Q6_K: return dispatch_kq<GQ6K>(W, n_rows, k, xq, m, y, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace barq
