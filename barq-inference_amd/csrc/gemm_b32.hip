// Batched GEMM for the 32-element block formats on gfx950 int8 MFMA:
// Y[m, n] = sum_b dx[m, b] * dw[n, b] * sum_{k in block b} xq[m, k] * wq[n, k]
// for GGUF Q4_0 (f16 d, (nibble - 8)), GGUF Q8_0 (f16 d, int8) and the quant
// crate's Q4_0 (f32 scale, signed nibbles in element order; q4_0.rs:69-115)
// weight rows against Q8_0 activation rows (the prefill path of models in
// these formats; gguf.rs:521-681, simd_quant.rs:272-317).
//
// v_mfma_i32_32x32x32_i8's K = 32 is exactly one block: each MFMA yields a
// 32x32 tile of one block's exact integer dot products, which the epilogue
// scales by dx * dw in f32.  Unlike the K-quant kernel (gemm_kq.hip), the
// per-block scales are floats, so they cannot be folded into the int8
// operands; the f32 epilogue (three vector instructions per output element
// per block) is what bounds this kernel.
//
// The Q8_0 activation rows are first repacked (q8_0_repack_kernel) into
// plain int8 rows (16-byte aligned blocks) and a table of the block scales
// as f32 in [block][row] order.  Per workgroup: BM activation rows x 128
// weight rows; four waves, each 32 weight rows and all BM activation rows.
// A step is four blocks (128 elements): NS LDS stages, each filled by
// buffer->LDS loads NS-1 steps ahead with one barrier per step (as in
// gemm_kq.hip).  A weight row's four blocks (72, 136 or 80 bytes) are copied
// as the 16-byte aligned window around them; with row bytes a multiple of
// 16 (k % 256 == 0) the window's offset is 0 or 8 for every row of a step.
#include "launch.hpp"
#include "mfma_common.hpp"

namespace barq {

// ---- activation repack ---------------------------------------------------------
// Q8_0 block b of row r -> 32 int8 at xr[r * k + 32 b], f32 scale at dx[b * m + r].
// A workgroup takes 16 rows x 16 blocks: thread t reads block t % 16 of row
// t / 16 (each row's blocks contiguous), and the scales go out through LDS as
// 16 runs of 16 consecutive rows.
__global__ __launch_bounds__(256) void q8_0_repack_kernel(const uint8_t* __restrict__ xq, size_t m, size_t nblk,
                                                          int8_t* __restrict__ xr, float* __restrict__ dx) {
    __shared__ float sd[16][17];
    const int t = threadIdx.x;
    const size_t r = (size_t)blockIdx.y * 16 + t / 16, b = (size_t)blockIdx.x * 16 + (t & 15);
    if (r < m && b < nblk) {
        const uint8_t* blk = xq + (r * nblk + b) * Q8_0_BYTES;
        sd[t & 15][t / 16] = f16_bits_to_f32(ld_u16(blk));
        uint4* dst = reinterpret_cast<uint4*>(xr + (r * nblk + b) * 32);
        dst[0] = ld16_a2(blk + 2);
        dst[1] = ld16_a2(blk + 18);
    }
    __syncthreads();
    const size_t r2 = (size_t)blockIdx.y * 16 + (t & 15), b2 = (size_t)blockIdx.x * 16 + t / 16;
    if (r2 < m && b2 < nblk) dx[b2 * m + r2] = sd[t / 16][t & 15];
}

// ---- formats -----------------------------------------------------------------
constexpr int B32_SB = 4;                 // blocks per step
constexpr int B32_BN = 128;               // weight rows per workgroup
constexpr int B32_XC = 9;                 // 16-byte chunks per staged activation row (8 + pad)
constexpr int B32_XRS = 16 * B32_XC;      // 144 bytes: 32-row fragment reads on distinct banks

// Four dwords from the 4- or 2-byte aligned LDS address p (a compile-time
// offset from a 4-byte aligned base: the funnel shift folds away when p is
// 4-byte aligned).
template <int OFF>
__device__ __forceinline__ uint4 lds_u4(const uint8_t* base) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(base + (OFF & ~3));
    if constexpr ((OFF & 3) == 0) {
        return make_uint4(q[0], q[1], q[2], q[3]);
    } else {
        const uint32_t a = q[0], b = q[1], c = q[2], d = q[3], e = q[4];
        return make_uint4(__builtin_amdgcn_alignbyte(b, a, OFF & 3), __builtin_amdgcn_alignbyte(c, b, OFF & 3),
                          __builtin_amdgcn_alignbyte(d, c, OFF & 3), __builtin_amdgcn_alignbyte(e, d, OFF & 3));
    }
}

template <int OFF>
__device__ __forceinline__ float lds_f16(const uint8_t* base) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(base + (OFF & ~3));
    return f16_bits_to_f32((OFF & 2) ? w >> 16 : w & 0xFFFFu);
}

// q - 8 for four nibbles q in [0, 15] (one per byte): no byte carries.
__device__ __forceinline__ uint32_t nib_minus8(uint32_t q) { return (q + 0x78787878u) ^ 0x80808080u; }

// GGUF Q4_0 (gguf.rs:521-578 with the 18-byte layout): element i < 16 is the
// low nibble of qs[i], element i + 16 the high nibble; value (q - 8) * d.
struct B40 {
    static constexpr int TYPE = TYPE_Q4_0, BB = Q4_0_BYTES, WP = 5, PIECES = 5, SHIFT = 8, NS = 3, KG_MAX = 4;
    template <int J>
    static __device__ __forceinline__ void block(const uint8_t* row, int g2, v4i& b, float& dw) {
        const uint4 qs = lds_u4<18 * J + 2>(row);
        const uint32_t sh = 4u * (uint32_t)g2;
        b = v4i{(int)nib_minus8((qs.x >> sh) & 0x0F0F0F0Fu), (int)nib_minus8((qs.y >> sh) & 0x0F0F0F0Fu),
                (int)nib_minus8((qs.z >> sh) & 0x0F0F0F0Fu), (int)nib_minus8((qs.w >> sh) & 0x0F0F0F0Fu)};
        dw = lds_f16<18 * J>(row);
    }
};

// GGUF Q8_0 (gguf.rs:634-681): f16 d + 32 int8.
struct B80 {
    static constexpr int TYPE = TYPE_Q8_0, BB = Q8_0_BYTES, WP = 9, PIECES = 9, SHIFT = 8, NS = 2, KG_MAX = 2;
    template <int J>
    static __device__ __forceinline__ void block(const uint8_t* row, int g2, v4i& b, float& dw) {
        const uint4 q = lds_u4<34 * J + 2>(row + 16 * g2);   // quants 16 g2 .. 16 g2 + 15
        b = v4i{(int)q.x, (int)q.y, (int)q.z, (int)q.w};
        dw = lds_f16<34 * J>(row);
    }
};

// The quant crate's Q4_0 (q4_0.rs:69-115): f32 scale, element i in byte i / 2
// (low nibble for even i), value (nib >= 8 ? nib - 16 : nib) * scale.
struct B40Barq {
    static constexpr int TYPE = TYPE_Q4_0_BARQ, BB = Q4_0_BARQ_BYTES, WP = 5, PIECES = 5, SHIFT = 0, NS = 3, KG_MAX = 4;
    // four nibbles (even or odd elements) -> signed bytes: (nib ^ 8) - 8
    static __device__ __forceinline__ uint32_t sext4(uint32_t v) {
        return ((v ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u;
    }
    template <int J>
    static __device__ __forceinline__ void block(const uint8_t* row, int g2, v4i& b, float& dw) {
        // elements 16 g2 .. 16 g2 + 15 are bytes 8 g2 .. 8 g2 + 7 of the 16 quant bytes
        const uint32_t* q = reinterpret_cast<const uint32_t*>(row + 20 * J + 4 + 8 * g2);
        const uint32_t d0 = q[0], d1 = q[1];
        const uint32_t lo0 = sext4(d0 & 0x0F0F0F0Fu), hi0 = sext4((d0 >> 4) & 0x0F0F0F0Fu);
        const uint32_t lo1 = sext4(d1 & 0x0F0F0F0Fu), hi1 = sext4((d1 >> 4) & 0x0F0F0F0Fu);
        // interleave even (lo) and odd (hi) elements back into element order
        b = v4i{(int)__builtin_amdgcn_perm(hi0, lo0, 0x05010400u), (int)__builtin_amdgcn_perm(hi0, lo0, 0x07030602u),
                (int)__builtin_amdgcn_perm(hi1, lo1, 0x05010400u), (int)__builtin_amdgcn_perm(hi1, lo1, 0x07030602u)};
        dw = *reinterpret_cast<const float*>(row + 20 * J);
    }
};

// LDS stage layout and per-wave load counts
template <class F, int BM>
struct B32L {
    static constexpr int RS = 16 * F::PIECES;                       // staged weight row stride
    static constexpr int X_INSTR_ALL = (BM * B32_XC + 63) / 64;
    static constexpr int W = 1024 * X_INSTR_ALL;                    // weight rows after the activation rows
    static constexpr int W_INSTR_ALL = B32_BN * F::PIECES / 64;
    static constexpr int DX = W + B32_BN * RS;                      // [block][row] f32 scales, one instruction
    static constexpr int STAGE = DX + 1024;
    static constexpr int X_INSTR = (X_INSTR_ALL + 3) / 4;
    static constexpr int W_INSTR = (W_INSTR_ALL + 3) / 4;
    static constexpr int LOADS_MIN = X_INSTR_ALL / 4 + W_INSTR_ALL / 4;
    static constexpr int MT = BM / 32;
    static_assert(B32_BN * F::PIECES % 64 == 0, "weight tile is whole load instructions");
    static_assert(B32_SB * BM * 4 <= 1024, "scales fit one instruction");
    static_assert(F::BB * B32_SB + F::SHIFT <= RS, "the 16-byte aligned window holds the step's blocks");
};

template <class F, int BM>
struct B32Off {
    uint32_t x[B32L<F, BM>::X_INSTR];
    uint32_t w[B32L<F, BM>::W_INSTR];
    uint32_t dx;
};

template <class F, int BM>
__device__ __forceinline__ void b32_offsets(B32Off<F, BM>& o, uint32_t k, uint32_t wrb, uint32_t m, int wave, int l) {
    using L = B32L<F, BM>;
    #pragma unroll
    for (int q = 0; q < L::X_INSTR; q++) {
        const int p = (q * 4 + wave) * 64 + l, r = p / B32_XC, c = p - r * B32_XC;
        o.x[q] = (uint32_t)r * k + 16u * (uint32_t)(c < B32_XC - 1 ? c : 0);   // the pad chunk reloads chunk 0
    }
    #pragma unroll
    for (int q = 0; q < L::W_INSTR; q++) {
        const int p = (q * 4 + wave) * 64 + l, row = p / F::PIECES, piece = p - row * F::PIECES;
        o.w[q] = (uint32_t)row * wrb + 16u * (uint32_t)(piece < F::WP ? piece : F::WP - 1);
    }
    // lane l: block l / (BM / 4) of the step, rows 4 (l % (BM / 4)) .. +3
    const int j = l / (BM / 4), rq = l - j * (BM / 4);
    o.dx = j < B32_SB ? ((uint32_t)j * m + 4u * (uint32_t)rq) * 4u : 0x80000000u;   // past the range: zeros
}

// step s: activation bytes 128 s of each row, weight window of blocks 4s..4s+3, scales of those blocks
template <class F, int BM>
__device__ __forceinline__ void b32_issue(uint8_t* stage, i32x4v xr, i32x4v wr, i32x4v dr, const B32Off<F, BM>& o,
                                          int s, uint32_t m, int wave) {
    using L = B32L<F, BM>;
    const uint32_t xs = 128u * (uint32_t)s, ws = (uint32_t)(F::BB * B32_SB) * (uint32_t)s & ~15u;
    #pragma unroll
    for (int q = 0; q < L::X_INSTR; q++) {
        const int idx = q * 4 + wave;
        if (idx < L::X_INSTR_ALL) lds_load16(xr, stage + 1024 * idx, o.x[q], xs);
    }
    #pragma unroll
    for (int q = 0; q < L::W_INSTR; q++) {
        const int idx = q * 4 + wave;
        if (idx < L::W_INSTR_ALL) lds_load16(wr, stage + L::W + 1024 * idx, o.w[q], ws);
    }
    if (wave == 0) lds_load16(dr, stage + L::DX, o.dx, (uint32_t)(B32_SB * 4) * m * (uint32_t)s);
}

// One step (four blocks) from a stage into the accumulators.
template <class F, int BM, int J>
__device__ __forceinline__ void b32_block(const uint8_t* st, const uint8_t* wrow, int mbase, int n, int g2,
                                          float (&acc)[BM / 32][16]) {
    using L = B32L<F, BM>;
    constexpr int MT = L::MT;
    v4i b;
    float dw;
    F::template block<J>(wrow, g2, b, dw);
    #pragma unroll
    for (int t = 0; t < MT; t++) {
        const v4i a = *reinterpret_cast<const v4i*>(st + (mbase + 32 * t + n) * B32_XRS + 32 * J + 16 * g2);
        const v16i z = {};
        const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
        #pragma unroll
        for (int q = 0; q < 4; q++) {
            // rows 32t + 8q + 4g2 .. +3 of the wave's rows (32x32 C layout)
            const float4 dx = *reinterpret_cast<const float4*>(st + L::DX + 4 * (J * BM + mbase + 32 * t + 8 * q + 4 * g2));
            acc[t][4 * q + 0] = __builtin_fmaf(dx.x * dw, (float)c[4 * q + 0], acc[t][4 * q + 0]);
            acc[t][4 * q + 1] = __builtin_fmaf(dx.y * dw, (float)c[4 * q + 1], acc[t][4 * q + 1]);
            acc[t][4 * q + 2] = __builtin_fmaf(dx.z * dw, (float)c[4 * q + 2], acc[t][4 * q + 2]);
            acc[t][4 * q + 3] = __builtin_fmaf(dx.w * dw, (float)c[4 * q + 3], acc[t][4 * q + 3]);
        }
    }
}

template <class F, int BM>
__device__ __forceinline__ void b32_compute(const uint8_t* st, int s, int wave, int l, float (&acc)[BM / 32][16]) {
    using L = B32L<F, BM>;
    const int n = l & 31, g2 = l >> 5;
    // the step's window starts 0 or 8 bytes before its first block
    const uint32_t sh = (uint32_t)(F::BB * B32_SB) * (uint32_t)s & 15u;
    const uint8_t* wrow = st + L::W + (32 * wave + n) * L::RS + sh;
    b32_block<F, BM, 0>(st, wrow, 0, n, g2, acc);
    b32_block<F, BM, 1>(st, wrow, 0, n, g2, acc);
    b32_block<F, BM, 2>(st, wrow, 0, n, g2, acc);
    b32_block<F, BM, 3>(st, wrow, 0, n, g2, acc);
}

// KG K-groups of four waves share a tile: group g computes steps g, g + KG,
// ... from its own part of each LDS stage (one barrier per KG steps), and the
// groups' partial sums are added through LDS at the end.  More waves per tile
// for the same LDS: small M has few tiles, and each tile's steps then run in
// parallel.  With KS > 1 K slices the grid has KS workgroups per tile, slice
// i taking steps [i, i + 1) * steps / KS and writing its partial product to
// Y + i * M * N (slice_sum_kernel adds the slices in order).
template <class F, int BM, int NS, int KG>
__global__ __launch_bounds__(256 * KG, 1)
void b32_gemm_kernel(const uint8_t* __restrict__ W, uint32_t wrb, const int8_t* __restrict__ X,
                     const float* __restrict__ DXT, float* __restrict__ Y, int M, int N, int K, int tiles_m,
                     int ks, int xcd_order) {
    using L = B32L<F, BM>;
    constexpr int MT = L::MT, SB = KG * L::STAGE;
    static_assert(NS >= 2 && NS <= 4, "stage count");
    static_assert(KG == 1 || MT * 16 * 256 * 4 <= SB, "one group's partial sums fit one stage");
    __shared__ __align__(16) uint8_t st0[SB];
    __shared__ __align__(16) uint8_t st1[SB];
    __shared__ __align__(16) uint8_t st2[NS > 2 ? SB : 16];
    __shared__ __align__(16) uint8_t st3[NS > 3 ? SB : 16];
    auto stage = [&](int i) -> uint8_t* { return i == 0 ? st0 : i == 1 ? st1 : i == 2 ? st2 : st3; };
    const int l = threadIdx.x & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kg = wave_all >> 2, wave = wave_all & 3;
    // workgroup i runs on XCD i % 8: each XCD takes a contiguous run of tiles
    const int n_tiles = tiles_m * ((N + B32_BN - 1) / B32_BN);
    const int slice = blockIdx.x / n_tiles;
    int tile = blockIdx.x - slice * n_tiles;
    if (xcd_order && (n_tiles & 7) == 0) tile = (tile & 7) * (n_tiles >> 3) + (tile >> 3);
    const int mt = tile % tiles_m, nt = tile / tiles_m;
    const int m0 = mt * BM, n0 = nt * B32_BN;
    const uint32_t k = (uint32_t)K, m = (uint32_t)M;
    const i32x4v xr = make_rsrc4(X + (size_t)m0 * K, (uint32_t)((size_t)(M - m0) * K));
    const i32x4v wr = make_rsrc4(W + (size_t)n0 * wrb, (uint32_t)((size_t)(N - n0) * wrb));
    const i32x4v dr = make_rsrc4(DXT + m0, (uint32_t)(((size_t)(K / 32) * M - m0) * 4));
    B32Off<F, BM> off;
    b32_offsets<F, BM>(off, k, wrb, m, wave, l);
    const int nst = K / (32 * B32_SB * KG * ks);   // steps per group (the host checks divisibility)
    const int s0 = slice * nst * KG;                // this slice's first step
    const int sub = kg * L::STAGE;

    float acc[MT][16];
    #pragma unroll
    for (int t = 0; t < MT; t++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;

    #pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < nst) b32_issue<F, BM>(stage(s) + sub, xr, wr, dr, off, s0 + KG * s + kg, m, wave);
    for (int s = 0; s < nst; s++) {
        // this thread's loads of step s are done once at most the later
        // steps' loads are outstanding; every thread's after the barrier
        if (s + NS - 2 < nst) {
            if constexpr (NS == 4) wait_vmcnt<2 * L::LOADS_MIN>();
            else if constexpr (NS == 3) wait_vmcnt<L::LOADS_MIN>();
            else wait_vmcnt<0>();
        } else {
            wait_vmcnt<0>();
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + NS - 1 < nst)
            b32_issue<F, BM>(stage((s + NS - 1) % NS) + sub, xr, wr, dr, off, s0 + KG * (s + NS - 1) + kg, m, wave);
        b32_compute<F, BM>(stage(s % NS) + sub, s0 + KG * s + kg, wave, l, acc);
    }

    if constexpr (KG > 1) {
        // groups 1.. hand their sums to group 0 through stage 0 (every wave
        // has passed its last read of it), one group at a time, which group 0
        // adds in group order
        float* red = reinterpret_cast<float*>(st0);
        const int lane = 64 * wave + l;
        #pragma unroll
        for (int g = 1; g < KG; g++) {
            __syncthreads();
            if (kg == g) {
                #pragma unroll
                for (int t = 0; t < MT; t++)
                    #pragma unroll
                    for (int r = 0; r < 16; r++) red[(16 * t + r) * 256 + lane] = acc[t][r];
            }
            __syncthreads();
            if (kg == 0) {
                #pragma unroll
                for (int t = 0; t < MT; t++)
                    #pragma unroll
                    for (int r = 0; r < 16; r++) acc[t][r] += red[(16 * t + r) * 256 + lane];
            }
        }
        if (kg > 0) return;
    }
    float* const out = Y + (size_t)slice * M * N;
    const int col = n0 + 32 * wave + (l & 31), g2 = l >> 5;
    if (col < N) {
        #pragma unroll
        for (int t = 0; t < MT; t++)
            #pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 32 * t + 8 * (r >> 2) + 4 * g2 + (r & 3);
                if (row < M) __builtin_nontemporal_store(acc[t][r], &out[(size_t)row * N + col]);
            }
    }
}

// Y[i] = sum over the ks slices of P[slice * n + i], in slice order
__global__ __launch_bounds__(256) void slice_sum_kernel(const float* __restrict__ P, int ks, size_t n,
                                                        float* __restrict__ Y) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float a = P[i];
    for (int sl = 1; sl < ks; sl++) a += P[(size_t)sl * n + i];
    __builtin_nontemporal_store(a, &Y[i]);
}

// ---- launch ------------------------------------------------------------------

template <class F, int BM, int NS, int KG>
static hipError_t b32_launch_t(const void* W, size_t n_rows, size_t k, const int8_t* xr, const float* dx, size_t m,
                               float* y, int ks, hipStream_t s) {
    const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)((n_rows + B32_BN - 1) / B32_BN);
    const uint32_t wrb = (uint32_t)(k / 32 * F::BB);
    if ((k / (32 * B32_SB)) % (KG * ks) != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((b32_gemm_kernel<F, BM, NS, KG>), dim3((unsigned)(tiles_m * tiles_n * ks)), dim3(256 * KG), 0, s,
                       static_cast<const uint8_t*>(W), wrb, xr, dx, y, (int)m, (int)n_rows, (int)k, tiles_m, ks,
                       tuning_env(TUNE_GEMM_XCD, 1));
    return hipGetLastError();
}

static int b32_bm(size_t m) {
    const int bm = tuning_env(TUNE_GEMM_BM, m > 32 ? 64 : 32);
    return bm == 32 ? 32 : 64;
}

// K slices across workgroups when the tiles alone would leave most CUs idle:
// doubled while the grid stays within 256 workgroups and every slice keeps
// an even number of steps.  BARQ_GEMM_KS overrides.
static int b32_k_slices(size_t m, size_t n_rows, size_t k) {
    const int bm = b32_bm(m);
    const size_t tiles = (m + bm - 1) / bm * ((n_rows + B32_BN - 1) / B32_BN), steps = k / (32 * B32_SB);
    int ks = 1;
    while (ks < 16 && tiles * ks * 2 <= 256 && steps % (size_t)(ks * 4) == 0) ks *= 2;
    const int ovr = tuning_env(TUNE_GEMM_KS);
    if (ovr > 0 && (ovr & (ovr - 1)) == 0 && ovr <= 16 && steps % (size_t)(2 * ovr) == 0) ks = ovr;
    return ks;
}

// Tile rows and K-groups: 64-row tiles above 32 rows; four K-groups when
// there are fewer tiles than CUs and the step count allows, else two (two
// with K slices).  BARQ_GEMM_BM (32, 64) and BARQ_GEMM_KG (1, 2, 4) override.
template <class F>
static hipError_t b32_dispatch(const void* W, size_t n_rows, size_t k, const int8_t* xr, const float* dx, size_t m,
                               float* y, int ks, hipStream_t s) {
    const int bm = b32_bm(m);
    const size_t tiles = (m + bm - 1) / bm * ((n_rows + B32_BN - 1) / B32_BN);
    const size_t steps = k / (32 * B32_SB) / ks;   // per slice
    int kg = tuning_env(TUNE_GEMM_KG, ks == 1 && tiles < 256 && steps % 4 == 0 ? 4 : 2);
    if (kg != 1 && kg != 2 && kg != 4) kg = 2;
    if (kg > F::KG_MAX) kg = F::KG_MAX;   // LDS: Q8_0 weight rows are twice as long
    if (steps % kg != 0) kg = steps % 2 == 0 ? 2 : 1;
#define B32_CASE(BMV, KGV) \
    if constexpr (KGV <= F::KG_MAX) \
        if (bm == BMV && kg == KGV) return b32_launch_t<F, BMV, (KGV == 4 ? 2 : F::NS), KGV>(W, n_rows, k, xr, dx, m, y, ks, s);
    B32_CASE(32, 1) B32_CASE(32, 2) B32_CASE(32, 4) B32_CASE(64, 1) B32_CASE(64, 2) B32_CASE(64, 4)
#undef B32_CASE
    return b32_launch_t<F, 64, F::NS, 2>(W, n_rows, k, xr, dx, m, y, ks, s);
}

// int8 rows, the scale table, then (with K slices) the partial products
static size_t b32_parts_offset(size_t m, size_t k) { return (m * k + m * (k / 32) * 4 + 255) / 256 * 256; }

size_t b32_workspace(size_t m, size_t n_rows, size_t k) {
    const int ks = b32_k_slices(m, n_rows, k);
    return b32_parts_offset(m, k) + (ks > 1 ? (size_t)ks * m * n_rows * 4 : 0);
}

bool b32_supported(int w_type, size_t n_rows, size_t k, size_t m) {
    if (w_type != TYPE_Q4_0 && w_type != TYPE_Q8_0 && w_type != TYPE_Q4_0_BARQ) return false;
    if (k == 0 || k % 256 != 0 || n_rows == 0 || m == 0 || n_rows > (size_t)INT32_MAX) return false;
    const size_t bb = w_type == TYPE_Q4_0 ? Q4_0_BYTES : w_type == TYPE_Q8_0 ? Q8_0_BYTES : Q4_0_BARQ_BYTES;
    // 32-bit buffer offsets
    return n_rows * (k / 32) * bb < (1ull << 31) && m * k < (1ull << 31) && m * (k / 32) * 4 < (1ull << 31);
}

hipError_t b32_gemm_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m, void* ws,
                           float* y, hipStream_t s) {
    if (!b32_supported(w_type, n_rows, k, m)) return hipErrorInvalidValue;
    const size_t nblk = k / 32;
    int8_t* xr = static_cast<int8_t*>(ws);
    float* dx = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + m * k);
    hipLaunchKernelGGL(q8_0_repack_kernel, dim3((unsigned)((nblk + 15) / 16), (unsigned)((m + 15) / 16)), dim3(256), 0, s,
                       static_cast<const uint8_t*>(xq), m, nblk, xr, dx);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int ks = b32_k_slices(m, n_rows, k);
    float* parts = ks > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + b32_parts_offset(m, k)) : y;
    switch (w_type) {
    case TYPE_Q4_0: e = b32_dispatch<B40>(W, n_rows, k, xr, dx, m, parts, ks, s); break;
    case TYPE_Q8_0: e = b32_dispatch<B80>(W, n_rows, k, xr, dx, m, parts, ks, s); break;
    default: e = b32_dispatch<B40Barq>(W, n_rows, k, xr, dx, m, parts, ks, s); break;
    }
    if (e != hipSuccess || ks == 1) return e;
    return slice_sum_launch(parts, ks, m * n_rows, y, s);
}

hipError_t slice_sum_launch(const float* parts, int ks, size_t n, float* y, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(slice_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, parts, ks, n, y);
    return hipGetLastError();
}

}  // namespace barq
