// Batch-1 quantized GEMV kernels for gfx950: y[n] = sum_k W[n,k] x[k].
//
// Integer path (x already quantized to Q8_0 / Q8_K): weight blocks stay packed
// in HBM and are read once with 16-byte loads; nibbles and 6-bit scales are
// unpacked in registers; the activation vector is staged into LDS once per
// workgroup; products run on v_dot4_i32_i8 and the per-lane partial sums are
// reduced across the wave with DPP.  Each wave owns R consecutive rows.
//
// Literal path (x in f32): the same lane slicing, weights dequantized in
// registers bit-identically to the reference decoders (barq_core/src/gguf.rs)
// and multiplied into f32 accumulators — the arithmetic of
// blas::gemv_f32(dequant(W), x) (blas.rs:292-303) up to summation order.
#include "gemv_formats.hpp"
#include "launch.hpp"
#include "mfma_common.hpp"

#include <cstdio>
#include <cstdlib>

namespace barq {

// Workgroup -> rows.  Workgroup i runs on XCD i % 8.  A workgroup covers
// RW = R * WAVES rows; LW = 32 / RW workgroups fill one 128-byte line of y.
// Workgroups on one XCD take whole lines of y and consecutive lines go to
// consecutive XCDs, so each output line is written from one L2 (no partial
// lines written back from several XCDs) while the weight reads still
// interleave across all XCDs at a 32-row granularity.
template <int RW>
__device__ __forceinline__ int wg_rows_remap(int id, int G) {
    if constexpr (RW >= 32 || (32 % RW) != 0) {
        return id;
    } else {
        constexpr int LW = 32 / RW;
        const int full = G / (8 * LW) * (8 * LW);
        if (id >= full) return id;
        const int x = id & 7, j = id >> 3;
        return ((j / LW) * 8 + x) * LW + (j % LW);
    }
}

// Integer path.  Per wave: the lane's activation slice is loaded first (it is
// shared by all rows), then the weight slices of all R rows are issued before
// any arithmetic (the scheduling barrier keeps the compiler from sinking them
// next to their uses), so each wave has R rows of HBM traffic in flight.
// ONE: k <= 4096, a single 4096-element chunk (no loop: fewer VGPRs, so more
// waves per SIMD; C2's 7168 waves of two rows are then all resident at once).
// R rows from row0 (of n_rows) of W by this wave.
template <class F, int R, bool ONE>
__device__ __forceinline__ void gemv_q8_rows(const uint8_t* __restrict__ W, size_t row_bytes,
                                             const uint8_t* __restrict__ xq, float* __restrict__ y, int row0,
                                             int n_rows, int k, int l) {
    const typename F::Lane c = F::lane(l);
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    const int n_it = ONE ? 1 : (k + 4095) / 4096;
    const int last = n_rows - 1 - row0;
    const uint8_t* wrow = W + (size_t)row0 * row_bytes;

    float acc[R];
    #pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        if (F::active(it, c, nblk)) {
            typename F::X xs;
            F::load_x(xs, xq, it, c, nblk);
            typename F::Wt w[R];
            #pragma unroll
            for (int r = 0; r < R; r++) F::load_w(w[r], wrow + (size_t)min(r, last) * row_bytes, it, c, nblk);
            __builtin_amdgcn_sched_barrier(0);
            #pragma unroll
            for (int r = 0; r < R; r++) acc[r] += F::dot(w[r], xs, c);
        }
    }

    #pragma unroll
    for (int g = 0; g < R; g += 4) {
        const float v = reduce4(acc[g], g + 1 < R ? acc[g + 1] : 0.0f, g + 2 < R ? acc[g + 2] : 0.0f,
                                g + 3 < R ? acc[g + 3] : 0.0f);
        if ((l & 15) == 0) {
            const int rr = g + (l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3);
            if (rr < R && rr <= last) y[row0 + rr] = v;
        }
    }
}

template <class F, int R, int WAVES, bool ONE>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q8_kernel(const uint8_t* __restrict__ W, size_t row_bytes, const uint8_t* __restrict__ xq,
                    float* __restrict__ y, int n_rows, int k) {
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (wg_rows_remap<R * WAVES>(blockIdx.x, gridDim.x) * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    gemv_q8_rows<F, R, ONE>(W, row_bytes, xq, y, row0, n_rows, k, l);
}

// Q4_K with k <= 4096, two rows per wave, staged through LDS.  The wave's
// two rows are 2 * 144 * k / 256 contiguous bytes (4608 at k = 4096); they
// are copied into the wave's own LDS buffer by buffer->LDS loads in which
// each lane takes 16 consecutive bytes, so every load instruction covers
// whole cache lines and the non-temporal hint pays (each line is fetched
// once; the register GEMV's per-lane loads cover half of each line they
// touch, so there the hint would fetch lines twice).  The lanes then read
// their FmtQ4K slices from LDS and run the register GEMV's arithmetic and
// reduction: outputs are bit-identical to gemv_q8_rows<FmtQ4K, 2, true>.
// Measured at C2 (14336 x 4096, one box, 11 rotating weight copies): 7.14
// against 7.29 us; the bare staging reaches the streaming-read floor.

// LDS per wave: R rows of 2304 bytes (k = 4096) rounded up to whole 1 KB load
// instructions
template <int R>
constexpr int q4k_lds_buf = (R * 16 * Q4_K_BYTES + 1023) / 1024 * 1024;
constexpr int Q4K_LDS_BUF = q4k_lds_buf<2>;

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 8]
__device__ __forceinline__ void wait_vmcnt_upto8(uint32_t n) {
    switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    default: wait_vmcnt<8>(); break;
    }
}

// The lane's Q8_K activation slice for the LDS-staged Q4_K rows (FmtQ4K's
// lane slicing), loaded by inline-asm global loads.  The compiler counts
// only the loads it emits itself, so with the buffer->LDS copies (also
// inline asm) issued after these it would wait for everything (vmcnt(0))
// before its first use of an activation register; loaded by asm, nothing
// waits until gemv_q4k_rows_finish's explicit waits, which can then let row
// 0's arithmetic run while row 1's copies are still in flight.  No code may
// read or write these registers before that wait: the build checks the
// device assembly for it (isa_check_asm_loads.py).
typedef int i32x2v __attribute__((ext_vector_type(2)));
struct Q4KXRaw {
    i32x4v v[4];
    i32x2v bs;
    int dx;
};

__device__ __forceinline__ void q4k_x_issue(Q4KXRaw& r, const uint8_t* __restrict__ xq, int blk, int p) {
    const uint8_t* b = xq + (size_t)blk * 292;
    const uint8_t* bq = b + 64 * p;   // quants of this lane at +4 + 64 p + 16 i
    const uint8_t* bs = b + 8 * p;    // its two bsum pairs at +260 + 8 p
    asm volatile("global_load_dword %0, %1, off" : "=v"(r.dx) : "v"(b));
    asm volatile("global_load_dwordx4 %0, %1, off offset:4" : "=v"(r.v[0]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:20" : "=v"(r.v[1]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:36" : "=v"(r.v[2]) : "v"(bq));
    asm volatile("global_load_dwordx4 %0, %1, off offset:52" : "=v"(r.v[3]) : "v"(bq));
    asm volatile("global_load_dwordx2 %0, %1, off offset:260" : "=v"(r.bs) : "v"(bs));
}

// After the wait for q4k_x_issue's loads: FmtQ4K::load_x's values.
__device__ __forceinline__ void q4k_x_ready(Q4KXRaw& r, FmtQ4K::X& x) {
    asm volatile("" : "+v"(r.v[0]), "+v"(r.v[1]), "+v"(r.v[2]), "+v"(r.v[3]), "+v"(r.bs), "+v"(r.dx));
    #pragma unroll
    for (int i = 0; i < 4; i++)
        x.v[i] = make_uint4((uint32_t)r.v[i].x, (uint32_t)r.v[i].y, (uint32_t)r.v[i].z, (uint32_t)r.v[i].w);
    x.dx = __builtin_bit_cast(float, r.dx);
    const uint32_t b0 = (uint32_t)r.bs.x, b1 = (uint32_t)r.bs.y;
    x.sa = sext16(b0, 0) + sext16(b0, 16);
    x.sb = sext16(b1, 0) + sext16(b1, 16);
}

// The lane's activation slice and the wave's buffer->LDS copies of rows
// row0 .. row0 + R - 1 (R * 144 * nblk contiguous bytes, in 1 KB
// instructions), issued in that order with nothing waiting in between: the
// activation is an L2 hit that lands ahead of the rows (loads return in
// order), and the copies start without waiting for it.  Issued after the
// copies instead, the activation's latency came after the rows' in every
// wave (C2 7.8 against 7.3 us); waited for before the copies, it delays each
// wave's stream by an L2 round trip (7.3 against 7.1 us).  w_bytes: bytes of
// the whole matrix (the buffer descriptor's range: rows past the end read as
// zeros).
template <int R>
__device__ __forceinline__ void gemv_q4k_rows_issue(const uint8_t* __restrict__ W, uint32_t w_bytes,
                                                    const uint8_t* __restrict__ xq, int row0, int nblk, int l,
                                                    uint8_t* buf, Q4KXRaw& xr) {
    // every lane loads (lanes past the last block re-read it and ignore it)
    q4k_x_issue(xr, xq, min(l >> 2, nblk - 1), l & 3);
    const uint32_t rb = (uint32_t)nblk * Q4_K_BYTES, span = R * rb;
    const i32x4v rs = make_rsrc4(W, w_bytes);
    const uint32_t base = (uint32_t)row0 * rb;
    // every copy instruction is issued, so their number is a constant: the
    // lanes past the span read out of range (zeros, no memory traffic)
    #pragma unroll
    for (int q = 0; q < q4k_lds_buf<R> / 1024; q++) {
        const uint32_t off = 1024u * q + 16u * (uint32_t)l;
        lds_load16_nt(rs, buf + 1024 * q, off < span ? base + off : 0x80000000u, 0);
    }
}

// Waits for gemv_q4k_rows_issue's loads and returns the R rows' results in
// lanes 0, 32, 16, 48 (reduce4's order).  Row r's arithmetic starts once its
// copies have landed (loads complete in order; the later rows' copies may
// still be in flight), so only the last row's is left after the last byte.
template <int R>
__device__ __forceinline__ float gemv_q4k_rows_finish(int nblk, int l, const uint8_t* buf, Q4KXRaw& xr) {
    static_assert(R == 1 || R == 2 || R == 4, "one, two or four rows per wave");
    using F = FmtQ4K;
    const F::Lane c = F::lane(l);
    const uint32_t rb = (uint32_t)nblk * Q4_K_BYTES;
    constexpr uint32_t n_all = q4k_lds_buf<R> / 1024;   // copies issued
    const bool act = F::active(0, c, nblk);
    const uint8_t* b = buf + Q4_K_BYTES * c.sbl;
    F::X xs;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    #pragma unroll
    for (int r = 0; r < R; r++) {
        // copies issued after the last one row r needs
        wait_vmcnt_upto8(n_all - (rb * (r + 1) + 1023) / 1024);
        if (r == 0) {
            // the activation loads precede all n_all copies: a constant wait
            // that the runtime one above already implies, and that the
            // build's assembly check can verify on every path
            wait_vmcnt<n_all>();
        }
        asm volatile("" ::: "memory");
        if (r == 0) q4k_x_ready(xr, xs);
        if (act) {
            F::Wt w;
            w.hdr = *reinterpret_cast<const uint4*>(b + r * rb);
            w.q0 = *reinterpret_cast<const uint4*>(b + r * rb + 16 + 32 * c.p);
            w.q1 = *reinterpret_cast<const uint4*>(b + r * rb + 32 + 32 * c.p);
            acc[r] = F::dot(w, xs, c);
        }
    }
    return reduce4(acc[0], acc[1], acc[2], acc[3]);
}

// Two rows (row0's result in lane 0, row0 + 1's in lane 32)
__device__ __forceinline__ float gemv_q4k_pair_lds(const uint8_t* __restrict__ W, uint32_t w_bytes,
                                                   const uint8_t* __restrict__ xq, int row0, int nblk, int l,
                                                   uint8_t* buf) {
    Q4KXRaw xr;
    gemv_q4k_rows_issue<2>(W, w_bytes, xq, row0, nblk, l, buf, xr);
    __builtin_amdgcn_sched_barrier(0);
    return gemv_q4k_rows_finish<2>(nblk, l, buf, xr);
}

__device__ __forceinline__ void gemv_q4k_rows_lds(const uint8_t* __restrict__ W, uint32_t w_bytes,
                                                  const uint8_t* __restrict__ xq, float* __restrict__ y, int row0,
                                                  int n_rows, int nblk, int l, uint8_t* buf) {
    const float v = gemv_q4k_pair_lds(W, w_bytes, xq, row0, nblk, l, buf);
    if ((l & 31) == 0) {
        const int rr = l >> 5;
        if (row0 + rr < n_rows) y[row0 + rr] = v;
    }
}

template <int WAVES, int R>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q4k_lds_kernel(const uint8_t* __restrict__ W, uint32_t w_bytes, const uint8_t* __restrict__ xq,
                         float* __restrict__ y, int n_rows, int nblk) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES][q4k_lds_buf<R>];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (wg_rows_remap<R * WAVES>(blockIdx.x, gridDim.x) * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    Q4KXRaw xr;
    gemv_q4k_rows_issue<R>(W, w_bytes, xq, row0, nblk, l, lds[wave], xr);
    __builtin_amdgcn_sched_barrier(0);
    const float v = gemv_q4k_rows_finish<R>(nblk, l, lds[wave], xr);
    if ((l & 15) == 0) {
        const int rr = l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3;
        if (rr < R && row0 + rr < n_rows) y[row0 + rr] = v;
    }
}

// Q4_K with k <= 4096 for NX = 2-4 activation rows (a small decode batch):
// the LDS-staged rows above, each wave copying its R weight rows once and
// loading its lanes' slice of every activation row by inline asm ahead of the
// copies.  Each (token, row) product is FmtQ4K::dot on the one-token kernel's
// lane slices, reduced by reduce4, so y[j][r] equals the one-token GEMV of
// activation row j bit for bit.
template <int WAVES, int R, int NX>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q4k_lds_multi_kernel(const uint8_t* __restrict__ W, uint32_t w_bytes, const uint8_t* __restrict__ xq,
                               uint32_t x_row_bytes, float* __restrict__ y, int n_rows, int nblk) {
    using F = FmtQ4K;
    constexpr int NA = NX * R;   // token j, row r at j * R + r
    __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES][q4k_lds_buf<R>];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (wg_rows_remap<R * WAVES>(blockIdx.x, gridDim.x) * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    uint8_t* buf = lds[wave];
    Q4KXRaw xr[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) q4k_x_issue(xr[j], xq + (size_t)j * x_row_bytes, min(l >> 2, nblk - 1), l & 3);
    const uint32_t rb = (uint32_t)nblk * Q4_K_BYTES, span = R * rb;
    const i32x4v rs = make_rsrc4(W, w_bytes);
    const uint32_t base = (uint32_t)row0 * rb;
    // every copy instruction is issued (a constant count; lanes past the span
    // read out of range)
    #pragma unroll
    for (int q = 0; q < q4k_lds_buf<R> / 1024; q++) {
        const uint32_t off = 1024u * q + 16u * (uint32_t)l;
        lds_load16_nt(rs, buf + 1024 * q, off < span ? base + off : 0x80000000u, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const F::Lane c = F::lane(l);
    constexpr uint32_t n_all = q4k_lds_buf<R> / 1024;
    const bool act = F::active(0, c, nblk);
    const uint8_t* b = buf + Q4_K_BYTES * c.sbl;
    F::X xs[NX];
    float acc[NA];
    #pragma unroll
    for (int i = 0; i < NA; i++) acc[i] = 0.0f;
    #pragma unroll
    for (int r = 0; r < R; r++) {
        // the activation rows and row r's copies (loads complete in order)
        wait_vmcnt_upto8(n_all - (rb * (r + 1) + 1023) / 1024);
        if (r == 0) wait_vmcnt<n_all>();   // the activation loads precede every copy
        asm volatile("" ::: "memory");
        if (r == 0) {
            #pragma unroll
            for (int j = 0; j < NX; j++) q4k_x_ready(xr[j], xs[j]);
        }
        if (act) {
            F::Wt w;
            w.hdr = *reinterpret_cast<const uint4*>(b + r * rb);
            w.q0 = *reinterpret_cast<const uint4*>(b + r * rb + 16 + 32 * c.p);
            w.q1 = *reinterpret_cast<const uint4*>(b + r * rb + 32 + 32 * c.p);
            #pragma unroll
            for (int j = 0; j < NX; j++) acc[j * R + r] = F::dot(w, xs[j], c);
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

// One row of W by this wave with the single-chunk lane slicing (k <= 4096):
// gemv_q8_rows<F, 1, true>'s arithmetic, the result in lane 0.
template <class F>
__device__ __forceinline__ float gemv_q8_row1(const uint8_t* __restrict__ W, size_t row_bytes,
                                              const uint8_t* __restrict__ xq, int row, int k, int l) {
    const typename F::Lane c = F::lane(l);
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    float acc = 0.0f;
    if (F::active(0, c, nblk)) {
        typename F::X xs;
        F::load_x(xs, xq, 0, c, nblk);
        typename F::Wt w;
        F::load_w(w, W + (size_t)row * row_bytes, 0, c, nblk);
        __builtin_amdgcn_sched_barrier(0);
        acc += F::dot(w, xs, c);
    }
    return reduce4(acc, 0.0f, 0.0f, 0.0f);
}

// The q, k and v projections of one token with RoPE and the cache append in
// their epilogue (self_attention for one token, transformer.rs:212-245):
// workgroups 0 .. wg_q - 1 take q's rows, then k's, then v's.  A wave's two
// Q4_K rows 2i and 2i + 1 of a head are one rotary pair of the interleaved
// layout, so the wave rotates them itself with rope_qkv_kernel's angle and
// products (the same bits) and writes q_out or the cache row; v's rows go to
// the cache as they are.  The pair's angle is computed before the rows'
// loads land.
struct QkvRopeArgs {
    const uint8_t* w[3];
    uint32_t bytes[3];        // matrix bytes (the buffer descriptors' ranges)
    int rows[3];
    int wg_q, wg_k;
    int hd;
    float* q_out;             // [n_head][hd]
    float* k_dst;             // cache row of the new position, kv head 0; head h at + h * head_stride
    float* v_dst;
    size_t head_stride;
    long long start_pos;
    float freq_scale;
    const float* inv_freq;
};

template <bool V6, int WAVES>
__global__ __launch_bounds__(WAVES * 64)
void gemv_qkv_rope_kernel(QkvRopeArgs a, const uint8_t* __restrict__ xq, int k) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES][Q4K_LDS_BUF];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int id = blockIdx.x, mat = 0;
    if (id >= a.wg_q) {
        id -= a.wg_q;
        mat = 1;
        if (id >= a.wg_k) {
            id -= a.wg_k;
            mat = 2;
        }
    }
    if (mat == 2 && V6) {
        const int row = id * WAVES + wave;
        if (row >= a.rows[2]) return;
        const float v = gemv_q8_row1<FmtQ6K>(a.w[2], (size_t)(k / 256) * Q6_K_BYTES, xq, row, k, l);
        if (l == 0) a.v_dst[(size_t)(row / a.hd) * a.head_stride + row % a.hd] = v;
        return;
    }
    const int row0 = (id * WAVES + wave) * 2;
    if (row0 >= a.rows[mat]) return;
    Q4KXRaw xr;
    gemv_q4k_rows_issue<2>(a.w[mat], a.bytes[mat], xq, row0, k / 256, l, lds[wave], xr);
    __builtin_amdgcn_sched_barrier(0);
    float sn = 0.0f, cs = 1.0f;
    if (mat < 2) {
        // (abs_pos as f32 * rope_freq_scale) * rope_inv_freq[i], as rope_qkv_kernel.
        // The frequency is a scalar load (lgkmcnt): a vector load's wait
        // would also wait for the row copies in flight.
        const int i = __builtin_amdgcn_readfirstlane((row0 % a.hd) / 2);
        const float f = *reinterpret_cast<const __attribute__((address_space(4))) float*>(
            reinterpret_cast<uintptr_t>(a.inv_freq + i));
        const float angle = ((float)a.start_pos * a.freq_scale) * f;
        sincosf(angle, &sn, &cs);
    }
    __builtin_amdgcn_sched_barrier(0);
    const float v = gemv_q4k_rows_finish<2>(k / 256, l, lds[wave], xr);
    const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float x1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    if (l == 0) {
        const int h = row0 / a.hd, d0 = row0 % a.hd;
        if (mat == 2) {
            float* dst = a.v_dst + (size_t)h * a.head_stride + d0;
            dst[0] = x0;
            dst[1] = x1;
        } else {
            float* dst = mat == 0 ? a.q_out + (size_t)h * a.hd + d0 : a.k_dst + (size_t)h * a.head_stride + d0;
            dst[0] = x0 * cs - x1 * sn;
            dst[1] = x0 * sn + x1 * cs;
        }
    }
}

// Several projections of one activation row in one launch (the q, k and v
// projections of self_attention, transformer.rs:212-220, all on the same
// normalized x): matrices 0 .. NA-1 are in format FA (RA rows per wave),
// matrix NA (if NB) in format FB (RB rows per wave); the first workgroups
// take FA's rows, the rest FB's.  One launch pays the ramp-up and drain of a
// memory-bound kernel once for all of them (the k and v projections of
// Llama-3-8B are 1024 rows each: alone they leave most CUs idle).
struct GemvGroupArgs {
    const uint8_t* w[4];
    float* y[4];
    int rows[4];
    int n_a;              // matrices in format FA
    int wg_a;             // workgroups of the FA matrices (each matrix's rows padded to whole workgroups)
    size_t rb_a, rb_b;    // row bytes
};

// The FA matrices are Q4_K (two rows per wave, staged through LDS as in
// gemv_q4k_lds_kernel).
template <class FB, int RB, int WAVES>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q8_group_kernel(GemvGroupArgs g, const uint8_t* __restrict__ xq, int k) {
    constexpr int RA = 2;
    __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES][Q4K_LDS_BUF];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int id = blockIdx.x;
    if (id < g.wg_a) {
        int mi = 0;
        #pragma unroll
        for (int i = 0; i < 3; i++) {
            const int wg = (g.rows[mi] + RA * WAVES - 1) / (RA * WAVES);
            if (mi + 1 < g.n_a && id >= wg) {
                id -= wg;
                mi++;
            }
        }
        const int row0 = (id * WAVES + wave) * RA;
        if (row0 < g.rows[mi])
            gemv_q4k_rows_lds(g.w[mi], (uint32_t)g.rows[mi] * (uint32_t)g.rb_a, xq, g.y[mi], row0, g.rows[mi], k / 256,
                              l, lds[wave]);
    } else {
        id -= g.wg_a;
        const int row0 = (id * WAVES + wave) * RB;
        if (row0 < g.rows[g.n_a]) gemv_q8_rows<FB, RB, true>(g.w[g.n_a], g.rb_b, xq, g.y[g.n_a], row0, g.rows[g.n_a], k, l);
    }
}

// The SwiGLU of LlamaTransformer::feed_forward (transformer.rs:394-399):
// (g * (1 / (1 + exp(-g)))) * u, each operation rounded as written.
__device__ __forceinline__ float ffn_swiglu(float g, float u) {
    return (g * (1.0f / (1.0f + expf(-g)))) * u;
}

// Gate and up projections of one activation row in one launch, with the
// SwiGLU applied in the epilogue: h[i] = swiglu(G[i] . x, U[i] . x).  A wave
// owns P consecutive outputs and loads the P gate rows and the P up rows
// (2P rows in flight, as R = 2P rows of gemv_q8_kernel); the partial sums
// fold as (g0, u0, g1, u1) through reduce4, so g_i and u_i meet in one lane
// with one cross-half exchange.  Reading both matrices in one launch pays
// the ramp-up and drain of a memory-bound kernel once for both.
template <class F, int P, int WAVES, bool ONE>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q8_glu_kernel(const uint8_t* __restrict__ G, const uint8_t* __restrict__ U, size_t row_bytes,
                        const uint8_t* __restrict__ xq, float* __restrict__ h, int n_rows, int k) {
    static_assert(P == 1 || P == 2, "one or two outputs per wave");
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (wg_rows_remap<P * WAVES>(blockIdx.x, gridDim.x) * WAVES + wave) * P;
    if (row0 >= n_rows) return;
    const typename F::Lane c = F::lane(l);
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    const int n_it = ONE ? 1 : (k + 4095) / 4096;
    const int last = n_rows - 1 - row0;
    const uint8_t* grow = G + (size_t)row0 * row_bytes;
    const uint8_t* urow = U + (size_t)row0 * row_bytes;

    float acc[2 * P];   // g0, u0, g1, u1
    #pragma unroll
    for (int r = 0; r < 2 * P; r++) acc[r] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        if (F::active(it, c, nblk)) {
            typename F::X xs;
            F::load_x(xs, xq, it, c, nblk);
            typename F::Wt w[2 * P];
            #pragma unroll
            for (int p = 0; p < P; p++) {
                const size_t off = (size_t)min(p, last) * row_bytes;
                F::load_w(w[2 * p], grow + off, it, c, nblk);
                F::load_w(w[2 * p + 1], urow + off, it, c, nblk);
            }
            __builtin_amdgcn_sched_barrier(0);
            #pragma unroll
            for (int r = 0; r < 2 * P; r++) acc[r] += F::dot(w[r], xs, c);
        }
    }

    // lane 0: g0, lane 32: u0, lane 16: g1, lane 48: u1
    const float v = reduce4(acc[0], acc[1], P > 1 ? acc[2] : 0.0f, P > 1 ? acc[3] : 0.0f);
    const float other = upper_half(v);
    if (l == 0) h[row0] = ffn_swiglu(v, other);
    if (P > 1 && l == 16 && last >= 1) h[row0 + 1] = ffn_swiglu(v, other);
}

// The fused gate/up GEMV for k <= 4096 staged through LDS (the Q4_K rows'
// scheme above): a wave copies gate row i and up row i (2304 bytes each at
// k = 4096) into its own 4.5 KB LDS buffer, the up row right after the gate
// row, with whole-line non-temporal buffer->LDS loads, its activation slice
// loaded ahead of the copies by inline asm; the gate row's dot product runs
// once its three copies have landed.  The arithmetic and reduction are
// gemv_q8_glu_kernel<FmtQ4K, 1, ...>'s, so h is bit-identical.
constexpr int GLU_ROW = 2304;                 // a Q4_K row of 4096 elements
constexpr int GLU_LDS_BUF = 2 * GLU_ROW;      // gate row, then up row

//
// NX = 2-4 activation rows (x_row_bytes apart; h is [NX x n_rows]): the wave
// loads its lanes' slice of every row ahead of the copies and computes each
// token's g and u the same way, so h[j] equals the one-token launch's h for
// activation row j bit for bit.
template <int WAVES, int NX = 1>
__global__ __launch_bounds__(WAVES * 64)
void gemv_glu_lds_kernel(const uint8_t* __restrict__ G, const uint8_t* __restrict__ U, uint32_t m_bytes,
                         const uint8_t* __restrict__ xq, float* __restrict__ h, int n_rows, int nblk,
                         uint32_t x_row_bytes) {
    using F = FmtQ4K;
    __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES][GLU_LDS_BUF];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = wg_rows_remap<WAVES>(blockIdx.x, gridDim.x) * WAVES + wave;
    if (row >= n_rows) return;
    uint8_t* buf = lds[wave];
    Q4KXRaw xr[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) q4k_x_issue(xr[j], xq + (size_t)j * x_row_bytes, min(l >> 2, nblk - 1), l & 3);
    const uint32_t rb = (uint32_t)nblk * Q4_K_BYTES, base = (uint32_t)row * rb;
    const i32x4v gs = make_rsrc4(G, m_bytes), us = make_rsrc4(U, m_bytes);
    // per row two 1 KB copies and one 256-byte copy (64 lanes x 4 bytes):
    // the up row right after the gate row, 4.5 KB per wave
    #pragma unroll
    for (int m = 0; m < 2; m++) {
        const i32x4v rs = m ? us : gs;
        uint8_t* dst = buf + m * GLU_ROW;
        #pragma unroll
        for (int q = 0; q < 2; q++) {
            const uint32_t off = 1024u * q + 16u * (uint32_t)l;
            lds_load16_nt(rs, dst + 1024 * q, off < rb ? base + off : 0x80000000u, 0);
        }
        const uint32_t off = 2048u + 4u * (uint32_t)l;
        lds_load4_nt(rs, dst + 2048, off < rb ? base + off : 0x80000000u, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    const F::Lane c = F::lane(l);
    const bool act = F::active(0, c, nblk);
    wait_vmcnt<3>();   // the activation and the gate row's copies
    asm volatile("" ::: "memory");
    F::X xs[NX];
    #pragma unroll
    for (int j = 0; j < NX; j++) q4k_x_ready(xr[j], xs[j]);
    const uint8_t* b = buf + Q4_K_BYTES * c.sbl;
    float acc[2 * NX];   // token j: g at 2 j, u at 2 j + 1
    #pragma unroll
    for (int i = 0; i < 2 * NX; i++) acc[i] = 0.0f;
    if (act) {
        F::Wt w;
        w.hdr = *reinterpret_cast<const uint4*>(b);
        w.q0 = *reinterpret_cast<const uint4*>(b + 16 + 32 * c.p);
        w.q1 = *reinterpret_cast<const uint4*>(b + 32 + 32 * c.p);
        #pragma unroll
        for (int j = 0; j < NX; j++) acc[2 * j] = F::dot(w, xs[j], c);
    }
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    if (act) {
        F::Wt w;
        w.hdr = *reinterpret_cast<const uint4*>(b + GLU_ROW);
        w.q0 = *reinterpret_cast<const uint4*>(b + GLU_ROW + 16 + 32 * c.p);
        w.q1 = *reinterpret_cast<const uint4*>(b + GLU_ROW + 32 + 32 * c.p);
        #pragma unroll
        for (int j = 0; j < NX; j++) acc[2 * j + 1] = F::dot(w, xs[j], c);
    }
    // per group of two tokens: lane 0 g and lane 32 u of the first, lanes 16
    // and 48 those of the second
    #pragma unroll
    for (int t = 0; t < NX; t += 2) {
        const float v = reduce4(acc[2 * t], acc[2 * t + 1], t + 1 < NX ? acc[2 * t + 2] : 0.0f,
                                t + 1 < NX ? acc[2 * t + 3] : 0.0f);
        const float other = upper_half(v);
        if (l == 0) h[(size_t)t * n_rows + row] = ffn_swiglu(v, other);
        if (t + 1 < NX && l == 16) h[(size_t)(t + 1) * n_rows + row] = ffn_swiglu(v, other);
    }
}

// A few activation rows (2-4 tokens of a small decode batch): each wave's
// weight slices are loaded once per chunk and dotted with every row's
// activation slice, so the weights are read once instead of once per token.
// y is [NX x n_rows] (row-major, token-major).
// nvalid <= NX tokens are real: the others re-read token nvalid - 1 and are
// not stored (one instantiation serves every count up to NX).
template <class F, int R, int WAVES, int NX>
__device__ __forceinline__ void gemv_multi_body(const uint8_t* __restrict__ W, size_t row_bytes,
                                                const uint8_t* __restrict__ xq, size_t x_row_bytes,
                                                float* __restrict__ y, int n_rows, int k, int nvalid = NX) {
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (wg_rows_remap<R * WAVES>(blockIdx.x, gridDim.x) * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    const typename F::Lane c = F::lane(l);
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    const int n_it = (k + 4095) / 4096;
    const int last = n_rows - 1 - row0;
    const uint8_t* wrow = W + (size_t)row0 * row_bytes;
    constexpr int NA = NX * R;   // sums per lane: token j, weight row r at j * R + r

    float acc[NA];
    #pragma unroll
    for (int i = 0; i < NA; i++) acc[i] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        if (F::active(it, c, nblk)) {
            typename F::X xs[NX];
            #pragma unroll
            for (int j = 0; j < NX; j++) F::load_x(xs[j], xq + (size_t)min(j, nvalid - 1) * x_row_bytes, it, c, nblk);
            typename F::Wt w[R];
            #pragma unroll
            for (int r = 0; r < R; r++) F::load_w(w[r], wrow + (size_t)min(r, last) * row_bytes, it, c, nblk);
            __builtin_amdgcn_sched_barrier(0);
            #pragma unroll
            for (int j = 0; j < NX; j++)
                #pragma unroll
                for (int r = 0; r < R; r++) acc[j * R + r] += F::dot(w[r], xs[j], c);
        }
    }

    #pragma unroll
    for (int g = 0; g < NA; g += 4) {
        const float v = reduce4(acc[g], g + 1 < NA ? acc[g + 1] : 0.0f, g + 2 < NA ? acc[g + 2] : 0.0f,
                                g + 3 < NA ? acc[g + 3] : 0.0f);
        if ((l & 15) == 0) {
            const int f = g + (l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3);
            const int j = f / R, rr = f - j * R;
            if (f < NA && j < nvalid && rr <= last) y[(size_t)j * n_rows + row0 + rr] = v;
        }
    }
}

template <class F, int R, int WAVES, int NX>
__global__ __launch_bounds__(WAVES * 64)
void gemv_q8_multi_kernel(const uint8_t* __restrict__ W, size_t row_bytes, const uint8_t* __restrict__ xq,
                          size_t x_row_bytes, float* __restrict__ y, int n_rows, int k) {
    gemv_multi_body<F, R, WAVES, NX>(W, row_bytes, xq, x_row_bytes, y, n_rows, k);
}

// Expert-grouped GEMV for decode-size MoE steps.  A step of na assignments
// has rows in at most na experts, so the grid has `slots` = min(na, ne) rows
// of workgroups per weight set: blockIdx.y = mat * slots + slot takes the
// slot-th expert e that has rows (found from the device offsets with one
// ballot: no host synchronisation), i.e. rows [offsets[e], offsets[e + 1])
// of the grouped activation rows X against the weights w[mat * ne + e]
// (n_rows x k) into rows of Y + mat * ymat, NXP tokens per pass (the host
// sets NXP to the step's token count, which bounds an expert's rows unless a
// token repeats an expert; the VGPRs, and so the waves per SIMD, follow NXP).
// Slots past the experts that have rows exit at once.
struct MoeGemvWeights { const uint8_t* w[MOE_GEMV_MAXE]; };

template <class F, int R, int WAVES, int NXP>
__global__ __launch_bounds__(WAVES * 64)
void moe_gemv_kernel(MoeGemvWeights wt, const int32_t* __restrict__ offsets, int ne, int slots,
                     const uint8_t* __restrict__ X, size_t xrb, float* __restrict__ Y, size_t ymat, size_t row_bytes,
                     int n_rows, int k) {
    const int mat = blockIdx.y / slots;
    int slot = blockIdx.y - mat * slots;
    const int lane = threadIdx.x & 63;
    int e = -1;
    for (int e0 = 0; e0 < ne; e0 += 64) {   // wave-uniform
        const int ee = e0 + lane;
        const uint64_t has = __ballot(ee < ne && offsets[ee + 1] > offsets[ee]);
        const int cnt = __popcll(has);
        if (slot < cnt) {
            uint64_t m = has;
            for (int i = 0; i < slot; i++) m &= m - 1;
            e = e0 + __ffsll((unsigned long long)m) - 1;
            break;
        }
        slot -= cnt;
    }
    if (e < 0) return;
    const int r0 = offsets[e], c = offsets[e + 1] - r0;
    const uint8_t* W = wt.w[mat * ne + e];
    for (int j0 = 0; j0 < c; j0 += NXP) {
        const uint8_t* xq = X + (size_t)(r0 + j0) * xrb;
        float* y = Y + (size_t)mat * ymat + (size_t)(r0 + j0) * n_rows;
        gemv_multi_body<F, R, WAVES, NXP>(W, row_bytes, xq, xrb, y, n_rows, k, c - j0 < NXP ? c - j0 : NXP);
    }
}

// Literal path: x (f32) staged in LDS, weights dequantized in registers.
template <class F, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64)
void gemv_f32_kernel(const uint8_t* __restrict__ W, size_t row_bytes, const float* __restrict__ x,
                     float* __restrict__ y, int n_rows, int k) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    {
        const float4* src = reinterpret_cast<const float4*>(x);
        float4* dst = reinterpret_cast<float4*>(xs);
        for (int t = threadIdx.x; t < k / 4; t += blockDim.x) dst[t] = src[t];
    }
    __syncthreads();

    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * R;
    if (row0 >= n_rows) return;
    const typename F::Lane c = F::lane(l);
    const int nblk = k / F::ROW_BLOCK_ELEMS;
    const int n_it = (k + 4095) / 4096;
    const int last = n_rows - 1 - row0;
    const uint8_t* wrow = W + (size_t)row0 * row_bytes;

    float acc[R];
    #pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (int it = 0; it < n_it; it++) {
        if (!F::active(it, c, nblk)) continue;
        typename F::Wt w[R];
        #pragma unroll
        for (int r = 0; r < R; r++) F::load_w(w[r], wrow + (size_t)min(r, last) * row_bytes, it, c, nblk);
        // two-block formats: the second block of the last lane may be absent
        const int kbase = it * 4096;
        #pragma unroll
        for (int g = 0; g < 16; g++) {
            const int off = kbase + F::xoff(l, g);
            if (off >= k) continue;
            const float4 xv = *reinterpret_cast<const float4*>(xs + off);
            #pragma unroll
            for (int r = 0; r < R; r++) {
                float v[4];
                F::deq4(w[r], c, g, v);
                acc[r] = __builtin_fmaf(v[0], xv.x, acc[r]);
                acc[r] = __builtin_fmaf(v[1], xv.y, acc[r]);
                acc[r] = __builtin_fmaf(v[2], xv.z, acc[r]);
                acc[r] = __builtin_fmaf(v[3], xv.w, acc[r]);
            }
        }
    }

    #pragma unroll
    for (int g = 0; g < R; g += 4) {
        const float v = reduce4(acc[g], g + 1 < R ? acc[g + 1] : 0.0f, g + 2 < R ? acc[g + 2] : 0.0f,
                                g + 3 < R ? acc[g + 3] : 0.0f);
        if ((l & 15) == 0) {
            const int rr = g + (l == 0 ? 0 : l == 32 ? 1 : l == 16 ? 2 : 3);
            if (rr < R && rr <= last) y[row0 + rr] = v;
        }
    }
}

// ---- launch configuration ---------------------------------------------------
// (rows per wave, waves per workgroup) for the integer path.  The default for
// each format was chosen by sweeping on MI355X.
struct GemvCfg { int r, waves; };

// BARQ_GEMV_CFG="R,W" overrides the launch shape (used for tuning sweeps).
static GemvCfg env_cfg() {
    return GemvCfg{tuning_env(TUNE_GEMV_CFG_R), tuning_env(TUNE_GEMV_CFG_W)};
}


template <class F, int R, int WAVES>
static hipError_t launch_q8(const uint8_t* W, size_t row_bytes, const uint8_t* xq, float* y,
                            int n_rows, int k, hipStream_t s) {
    const int rows_per_block = R * WAVES;
    const unsigned grid = (unsigned)((n_rows + rows_per_block - 1) / rows_per_block);
    if (k <= 4096)
        hipLaunchKernelGGL((gemv_q8_kernel<F, R, WAVES, true>), dim3(grid), dim3(WAVES * 64), 0, s,
                           W, row_bytes, xq, y, n_rows, k);
    else
        hipLaunchKernelGGL((gemv_q8_kernel<F, R, WAVES, false>), dim3(grid), dim3(WAVES * 64), 0, s,
                           W, row_bytes, xq, y, n_rows, k);
    return hipGetLastError();
}

template <class F>
static hipError_t dispatch_q8(const uint8_t* W, size_t row_bytes, const uint8_t* xq, float* y,
                              int n_rows, int k, hipStream_t s, GemvCfg def) {
    const GemvCfg e = env_cfg();
    const GemvCfg c = e.r ? e : def;
#define BARQ_GEMV_CASE(RR, WW) \
    if (c.r == RR && c.waves == WW) return launch_q8<F, RR, WW>(W, row_bytes, xq, y, n_rows, k, s);
    BARQ_GEMV_CASE(1, 4) BARQ_GEMV_CASE(2, 4) BARQ_GEMV_CASE(4, 4) BARQ_GEMV_CASE(8, 4)
    BARQ_GEMV_CASE(1, 8) BARQ_GEMV_CASE(2, 8) BARQ_GEMV_CASE(4, 8)
    BARQ_GEMV_CASE(2, 2) BARQ_GEMV_CASE(4, 2) BARQ_GEMV_CASE(8, 2) BARQ_GEMV_CASE(4, 1)
#undef BARQ_GEMV_CASE
    return launch_q8<F, 2, 4>(W, row_bytes, xq, y, n_rows, k, s);
}

template <class F, int R, int WAVES>
static hipError_t launch_f32(const uint8_t* W, size_t row_bytes, const float* x, float* y,
                             int n_rows, int k, hipStream_t s) {
    const int rows_per_block = R * WAVES;
    const unsigned grid = (unsigned)((n_rows + rows_per_block - 1) / rows_per_block);
    const size_t lds = (size_t)k * 4;
    hipLaunchKernelGGL((gemv_f32_kernel<F, R, WAVES>), dim3(grid), dim3(WAVES * 64), lds, s,
                       W, row_bytes, x, y, n_rows, k);
    return hipGetLastError();
}

template <class F, int R, int WAVES, int NX>
static hipError_t launch_q8_multi(const uint8_t* W, size_t row_bytes, const uint8_t* xq, size_t x_row_bytes,
                                  float* y, int n_rows, int k, hipStream_t s) {
    const int rows_per_block = R * WAVES;
    const unsigned grid = (unsigned)((n_rows + rows_per_block - 1) / rows_per_block);
    hipLaunchKernelGGL((gemv_q8_multi_kernel<F, R, WAVES, NX>), dim3(grid), dim3(WAVES * 64), 0, s,
                       W, row_bytes, xq, x_row_bytes, y, n_rows, k);
    return hipGetLastError();
}

static int dma_bit(int w_type);

// A matmul of 2-4 tokens as one GEMV over all of them: the register GEMV for
// Q4_K, the LDS-streamed one for the formats that take it at batch 1 (its
// layout conditions, and the tokens' staged rows within LDS).
// BARQ_GEMV_MULTI_MAX caps the tokens (0 turns it off).
static bool multi_dma(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m) {
    return (tuning_env(TUNE_GEMV_DMA_TYPES, 2 | 4 | 8 | 16) & dma_bit(w_type)) &&
           gemv_dma_supported(w_type, W, n_rows, k, xq) && gemv_dma_multi_fits(w_type, k, m);
}

bool gemv_multi_supported(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m) {
    const int mx = tuning_env(TUNE_GEMV_MULTI_MAX, 4);
    if (m < 2 || (int)m > (mx < 4 ? mx : 4) || n_rows > (size_t)INT32_MAX) return false;
    if (multi_dma(w_type, W, n_rows, k, xq, m)) return true;
    return w_type == TYPE_Q4_K && k % 256 == 0;
}

hipError_t gemv_q8_multi_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m,
                                float* y, hipStream_t s) {
    if (!gemv_multi_supported(w_type, W, n_rows, k, xq, m)) return hipErrorInvalidValue;
    if (multi_dma(w_type, W, n_rows, k, xq, m)) return gemv_dma_launch(w_type, W, n_rows, k, xq, y, s, m);
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const size_t rb = k / 256 * 144, xrb = k / 256 * 292;
    const int n = (int)n_rows, kk = (int)k;
    // measured at 14336 x 4096 (two paired runs on one box, us per call for
    // 2 / 3 / 4 tokens): four rows per wave 8.40 / 10.05 / 11.58, two rows
    // (BARQ_GEMV_LDS=2) 8.54 / 10.39 / 12.11, the register GEMV
    // (BARQ_GEMV_LDS=0) 9.35 / 12.30 / 13.17
    const int lds_mode = tuning_env(TUNE_GEMV_LDS, 1);
    if (k <= 4096 && n_rows * rb < 0x80000000ull && lds_mode != 0) {
        constexpr int WAVES = 4;
        const int R = lds_mode == 2 ? 2 : 4;
        const unsigned grid = (unsigned)((n_rows + (size_t)R * WAVES - 1) / ((size_t)R * WAVES));
#define BARQ_LDS_MULTI(RR, NN)                                                                                    \
    hipLaunchKernelGGL((gemv_q4k_lds_multi_kernel<WAVES, RR, NN>), dim3(grid), dim3(WAVES * 64), 0, s, w,          \
                       (uint32_t)(n_rows * rb), x, (uint32_t)xrb, y, n, kk / 256);                                \
    return hipGetLastError();
        if (R == 2) {
            if (m == 2) { BARQ_LDS_MULTI(2, 2) }
            if (m == 3) { BARQ_LDS_MULTI(2, 3) }
            BARQ_LDS_MULTI(2, 4)
        } else {
            if (m == 2) { BARQ_LDS_MULTI(4, 2) }
            if (m == 3) { BARQ_LDS_MULTI(4, 3) }
            BARQ_LDS_MULTI(4, 4)
        }
#undef BARQ_LDS_MULTI
    }
    switch (m) {
    case 2: return launch_q8_multi<FmtQ4K, 2, 4, 2>(w, rb, x, xrb, y, n, kk, s);
    case 3: return launch_q8_multi<FmtQ4K, 2, 4, 3>(w, rb, x, xrb, y, n, kk, s);
    default: return launch_q8_multi<FmtQ4K, 2, 4, 4>(w, rb, x, xrb, y, n, kk, s);
    }
}

template <class F, int R, int WAVES, int NXP>
static hipError_t launch_moe_gemv_t(const MoeGemvWeights& wt, const int32_t* offsets, int ne, int nm, int slots,
                                    const uint8_t* x, size_t xrb, float* y, size_t ymat, size_t rb, int n, int k,
                                    hipStream_t s) {
    const unsigned gx = (unsigned)((n + R * WAVES - 1) / (R * WAVES));
    hipLaunchKernelGGL((moe_gemv_kernel<F, R, WAVES, NXP>), dim3(gx, (unsigned)(slots * nm)), dim3(WAVES * 64), 0, s,
                       wt, offsets, ne, slots, x, xrb, y, ymat, rb, n, k);
    return hipGetLastError();
}

template <class F, int R, int WAVES>
static hipError_t launch_moe_gemv(const MoeGemvWeights& wt, const int32_t* offsets, int ne, int nm, int slots, int nxp,
                                  const uint8_t* x, size_t xrb, float* y, size_t ymat, size_t rb, int n, int k,
                                  hipStream_t s) {
    switch (nxp) {
    case 1: return launch_moe_gemv_t<F, R, WAVES, 1>(wt, offsets, ne, nm, slots, x, xrb, y, ymat, rb, n, k, s);
    case 2: return launch_moe_gemv_t<F, R, WAVES, 2>(wt, offsets, ne, nm, slots, x, xrb, y, ymat, rb, n, k, s);
    case 3: return launch_moe_gemv_t<F, R, WAVES, 3>(wt, offsets, ne, nm, slots, x, xrb, y, ymat, rb, n, k, s);
    default: return launch_moe_gemv_t<F, R, WAVES, 4>(wt, offsets, ne, nm, slots, x, xrb, y, ymat, rb, n, k, s);
    }
}

// BARQ_MOE_GEMV: 1 (default) single-token MoE steps take the grouped GEMVs,
// 2 any step of at most 4 assignments, 0 none
int moe_gemv_enabled() { return tuning_env(TUNE_MOE_GEMV, 1); }

bool moe_gemv_supported(int w_type, size_t n_experts, size_t n_mats, size_t n_rows, size_t k) {
    return (w_type == TYPE_Q4_K || w_type == TYPE_Q6_K) && k % 256 == 0 && k > 0 && n_experts > 0 && n_mats > 0 &&
           n_experts * n_mats <= (size_t)MOE_GEMV_MAXE && n_rows > 0 && n_rows <= (size_t)INT32_MAX &&
           k <= (size_t)INT32_MAX;
}

hipError_t moe_gemv_launch(int w_type, const void* const* W, size_t n_experts, size_t n_mats, const int32_t* offsets,
                           size_t n_assign, size_t tokens, const void* xq, size_t n_rows, size_t k, float* y,
                           size_t y_mat_stride, hipStream_t s) {
    if (!moe_gemv_supported(w_type, n_experts, n_mats, n_rows, k) || n_assign == 0 || tokens == 0)
        return hipErrorInvalidValue;
    const int slots = (int)(n_assign < n_experts ? n_assign : n_experts);
    const int nxp = (int)(tokens < 4 ? tokens : 4);
    MoeGemvWeights wt = {};
    for (size_t i = 0; i < n_experts * n_mats; i++) wt.w[i] = static_cast<const uint8_t*>(W[i]);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const size_t xrb = k / 256 * 292;
    const int ne = (int)n_experts, nm = (int)n_mats, n = (int)n_rows, kk = (int)k;
    if (w_type == TYPE_Q4_K)
        return launch_moe_gemv<FmtQ4K, 2, 4>(wt, offsets, ne, nm, slots, nxp, x, xrb, y, y_mat_stride, k / 256 * 144, n,
                                             kk, s);
    return launch_moe_gemv<FmtQ6K, 1, 8>(wt, offsets, ne, nm, slots, nxp, x, xrb, y, y_mat_stride, k / 256 * 210, n,
                                         kk, s);
}

// Formats that take the LDS-streaming GEMV (gemv_dma.hip) when its layout
// conditions hold; BARQ_GEMV_DMA_TYPES (bit per format, tuning) overrides.
// The LDS-staged Q4_K GEMV: one 4096-element chunk per row, 16-byte aligned
// blocks, and the matrix within the buffer descriptor's 31-bit range.
static bool q4k_lds_supported(const void* W, size_t n_rows, size_t k) {
    return k > 0 && k <= 4096 && k % 256 == 0 && n_rows > 0 && (reinterpret_cast<uintptr_t>(W) & 15) == 0 &&
           n_rows * (k / 256 * Q4_K_BYTES) < 0x80000000ull;
}

static int dma_bit(int w_type) {
    switch (w_type) {
    case TYPE_Q4_K: return 1;
    case TYPE_Q6_K: return 2;
    case TYPE_Q4_0: return 4;
    case TYPE_Q8_0: return 8;
    case TYPE_Q4_0_BARQ: return 16;
    default: return 0;
    }
}

hipError_t gemv_q8_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq,
                          float* y, hipStream_t s) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const int n = (int)n_rows, kk = (int)k;
    if (tuning_env(TUNE_GEMV_DMA_TYPES, 2 | 4 | 8 | 16) & dma_bit(w_type) &&
        gemv_dma_supported(w_type, W, n_rows, k, xq))
        return gemv_dma_launch(w_type, W, n_rows, k, xq, y, s);
    switch (w_type) {
    case TYPE_Q4_K:
        if (q4k_lds_supported(W, n_rows, k) && tuning_env(TUNE_GEMV_LDS, 1) && !env_cfg().r) {
            constexpr int WAVES = 4;
            const uint32_t bytes = (uint32_t)(n_rows * (k / 256 * Q4_K_BYTES));
            // rows per wave: one up to 4096 rows, two above (measured in one
            // process, us per call, one row against two, k = 4096: 1024 rows
            // 2.50-2.52 / 2.95-2.99, 4096 rows 3.77-3.79 / 3.90, 6144 rows
            // 4.59 / 4.55, 14336 rows 7.95 / 7.19; outputs bit-identical).
            // BARQ_GEMV_LDS = 2 / 3 / 4 force two / one / four.
            const int mode = tuning_env(TUNE_GEMV_LDS, 1);
            if (mode == 4) {
                const unsigned grid = (unsigned)((n_rows + 4 * WAVES - 1) / (4 * WAVES));
                hipLaunchKernelGGL((gemv_q4k_lds_kernel<WAVES, 4>), dim3(grid), dim3(WAVES * 64), 0, s, w, bytes, x,
                                   y, n, (int)(k / 256));
            } else if (mode == 3 || (mode == 1 && n_rows <= 4096)) {
                const unsigned grid = (unsigned)((n_rows + WAVES - 1) / WAVES);
                hipLaunchKernelGGL((gemv_q4k_lds_kernel<WAVES, 1>), dim3(grid), dim3(WAVES * 64), 0, s, w, bytes, x,
                                   y, n, (int)(k / 256));
            } else {
                const unsigned grid = (unsigned)((n_rows + 2 * WAVES - 1) / (2 * WAVES));
                hipLaunchKernelGGL((gemv_q4k_lds_kernel<WAVES, 2>), dim3(grid), dim3(WAVES * 64), 0, s, w, bytes, x,
                                   y, n, (int)(k / 256));
            }
            return hipGetLastError();
        }
        return dispatch_q8<FmtQ4K>(w, k / 256 * 144, x, y, n, kk, s, kk <= 4096 ? GemvCfg{2, 4} : GemvCfg{2, 2});
    case TYPE_Q6_K: return dispatch_q8<FmtQ6K>(w, k / 256 * 210, x, y, n, kk, s, {1, 8});
    case TYPE_Q4_0: return dispatch_q8<FmtQ40>(w, k / 32 * 18, x, y, n, kk, s, {1, 4});
    case TYPE_Q8_0: return dispatch_q8<FmtQ80>(w, k / 32 * 34, x, y, n, kk, s, {1, 4});
    case TYPE_Q4_0_BARQ: return dispatch_q8<FmtQ40Barq>(w, k / 32 * 20, x, y, n, kk, s, {1, 4});
    default: return hipErrorInvalidValue;
    }
}


// The grouped launch: up to three Q4_K matrices, optionally followed by one
// Q4_K or Q6_K matrix, k <= 4096 (one chunk), Q8_K activation; four waves
// per workgroup, two rows per wave for Q4_K and one for Q6_K (the register
// GEMV's Q4_K and Q6_K lane slicing).
bool gemv_group_supported(size_t n, const int* types, const void* const* W, const size_t* rows, size_t k) {
    if (n < 2 || n > 4 || k == 0 || k > 4096 || k % 256) return false;
    size_t total = 0;
    for (size_t i = 0; i < n; i++) {
        const bool last = i + 1 == n;
        if (types[i] != TYPE_Q4_K && !(last && types[i] == TYPE_Q6_K)) return false;
        if (rows[i] == 0 || rows[i] > (size_t)INT32_MAX) return false;
        if (types[i] == TYPE_Q4_K && (reinterpret_cast<uintptr_t>(W[i]) & 15)) return false;
        if (types[i] == TYPE_Q4_K && rows[i] * (k / 256 * Q4_K_BYTES) >= 0x80000000ull) return false;
        if (types[i] == TYPE_Q6_K && (reinterpret_cast<uintptr_t>(W[i]) & 1)) return false;
        total += rows[i];
    }
    return total <= (size_t)INT32_MAX;
}

hipError_t gemv_group_launch(size_t n, const int* types, const void* const* W, const size_t* rows, size_t k,
                             const void* xq, float* const* y, hipStream_t s) {
    constexpr int WAVES = 4, RA = 2, RB6 = 1;
    GemvGroupArgs g{};
    const bool b6 = types[n - 1] == TYPE_Q6_K;
    g.n_a = (int)(b6 ? n - 1 : n);
    int wg_a = 0;
    for (size_t i = 0; i < n; i++) {
        g.w[i] = static_cast<const uint8_t*>(W[i]);
        g.y[i] = y[i];
        g.rows[i] = (int)rows[i];
        if ((int)i < g.n_a) wg_a += (int)((rows[i] + RA * WAVES - 1) / (RA * WAVES));
    }
    g.wg_a = wg_a;
    g.rb_a = k / 256 * Q4_K_BYTES;
    g.rb_b = k / 256 * (b6 ? Q6_K_BYTES : Q4_K_BYTES);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    if (b6) {
        const unsigned grid = (unsigned)(wg_a + (rows[n - 1] + RB6 * WAVES - 1) / (RB6 * WAVES));
        hipLaunchKernelGGL((gemv_q8_group_kernel<FmtQ6K, RB6, WAVES>), dim3(grid), dim3(WAVES * 64), 0, s,
                           g, x, (int)k);
    } else {
        // every matrix in the FA part (n_a = n); no FB part
        hipLaunchKernelGGL((gemv_q8_group_kernel<FmtQ4K, RA, WAVES>), dim3((unsigned)wg_a),
                           dim3(WAVES * 64), 0, s, g, x, (int)k);
    }
    return hipGetLastError();
}

// The fused q/k/v + RoPE + append launch: Q4_K q and k (16-byte aligned),
// Q4_K or Q6_K v, k <= 4096, every matrix within the 31-bit buffer range,
// head_dim even (rows of a head pair up).
bool qkv_rope_supported(const int* types, const void* const* W, size_t n_q_rows, size_t n_kv_rows, size_t k,
                        size_t hd) {
    if (k == 0 || k > 4096 || k % 256 || hd == 0 || hd % 2 || n_q_rows == 0 || n_kv_rows == 0) return false;
    const size_t rows[3] = {n_q_rows, n_kv_rows, n_kv_rows};
    for (int i = 0; i < 3; i++) {
        const bool v6 = i == 2 && types[i] == TYPE_Q6_K;
        if (types[i] != TYPE_Q4_K && !v6) return false;
        const size_t bytes = rows[i] * (k / 256) * (v6 ? Q6_K_BYTES : Q4_K_BYTES);
        if (bytes >= 0x80000000ull) return false;
        if ((reinterpret_cast<uintptr_t>(W[i]) & (v6 ? 1 : 15)) != 0) return false;
    }
    return true;
}

hipError_t qkv_rope_launch(const int* types, const void* const* W, size_t n_q_rows, size_t n_kv_rows, size_t k,
                           const void* xq, size_t hd, float* q_out, float* k_dst, float* v_dst, size_t head_stride,
                           size_t start_pos, float freq_scale, const float* inv_freq, hipStream_t s) {
    constexpr int WAVES = 4;
    QkvRopeArgs a{};
    const size_t rows[3] = {n_q_rows, n_kv_rows, n_kv_rows};
    const bool v6 = types[2] == TYPE_Q6_K;
    for (int i = 0; i < 3; i++) {
        a.w[i] = static_cast<const uint8_t*>(W[i]);
        a.rows[i] = (int)rows[i];
        a.bytes[i] = (uint32_t)(rows[i] * (k / 256) * (i == 2 && v6 ? Q6_K_BYTES : Q4_K_BYTES));
    }
    a.wg_q = (int)((n_q_rows + 2 * WAVES - 1) / (2 * WAVES));
    a.wg_k = (int)((n_kv_rows + 2 * WAVES - 1) / (2 * WAVES));
    const int wg_v = (int)(v6 ? (n_kv_rows + WAVES - 1) / WAVES : (n_kv_rows + 2 * WAVES - 1) / (2 * WAVES));
    a.hd = (int)hd;
    a.q_out = q_out;
    a.k_dst = k_dst;
    a.v_dst = v_dst;
    a.head_stride = head_stride;
    a.start_pos = (long long)start_pos;
    a.freq_scale = freq_scale;
    a.inv_freq = inv_freq;
    const dim3 grid((unsigned)(a.wg_q + a.wg_k + wg_v));
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    if (v6)
        hipLaunchKernelGGL((gemv_qkv_rope_kernel<true, WAVES>), grid, dim3(WAVES * 64), 0, s, a, x, (int)k);
    else
        hipLaunchKernelGGL((gemv_qkv_rope_kernel<false, WAVES>), grid, dim3(WAVES * 64), 0, s, a, x, (int)k);
    return hipGetLastError();
}

bool gemv_glu_supported(int w_type, const void* G, const void* U, size_t n_rows, size_t k) {
    return w_type == TYPE_Q4_K && k % 256 == 0 && k > 0 && n_rows > 0 && n_rows <= (size_t)INT32_MAX &&
           (reinterpret_cast<uintptr_t>(G) & 15) == 0 && (reinterpret_cast<uintptr_t>(U) & 15) == 0;
}

template <int P, int WAVES>
static hipError_t launch_glu(const uint8_t* G, const uint8_t* U, size_t rb, const uint8_t* x, float* h, int n, int k,
                             hipStream_t s) {
    const unsigned grid = (unsigned)((n + P * WAVES - 1) / (P * WAVES));
    if (k <= 4096)
        hipLaunchKernelGGL((gemv_q8_glu_kernel<FmtQ4K, P, WAVES, true>), dim3(grid), dim3(WAVES * 64), 0, s, G, U, rb,
                           x, h, n, k);
    else
        hipLaunchKernelGGL((gemv_q8_glu_kernel<FmtQ4K, P, WAVES, false>), dim3(grid), dim3(WAVES * 64), 0, s, G, U, rb,
                           x, h, n, k);
    return hipGetLastError();
}

bool gemv_glu_multi_supported(int w_type, const void* G, const void* U, size_t n_rows, size_t k, size_t m) {
    return m >= 2 && m <= 4 && gemv_glu_supported(w_type, G, U, n_rows, k) && k <= 4096 &&
           n_rows * (k / 256 * 144) < 0x80000000ull && tuning_env(TUNE_GEMV_LDS, 1) != 0;
}

hipError_t gemv_glu_launch(int w_type, const void* G, const void* U, size_t n_rows, size_t k, const void* xq, float* h,
                           hipStream_t s, size_t m) {
    if (m > 1) {
        if (!gemv_glu_multi_supported(w_type, G, U, n_rows, k, m)) return hipErrorInvalidValue;
        constexpr int WAVES = 4;
        const dim3 grid((unsigned)((n_rows + WAVES - 1) / WAVES)), block(WAVES * 64);
        const uint8_t* g = static_cast<const uint8_t*>(G);
        const uint8_t* u = static_cast<const uint8_t*>(U);
        const uint8_t* x = static_cast<const uint8_t*>(xq);
        const uint32_t mb = (uint32_t)(n_rows * (k / 256 * 144)), xrb = (uint32_t)(k / 256 * Q8_K_BYTES);
        const int n = (int)n_rows, nb = (int)(k / 256);
        switch (m) {
        case 2: hipLaunchKernelGGL((gemv_glu_lds_kernel<WAVES, 2>), grid, block, 0, s, g, u, mb, x, h, n, nb, xrb); break;
        case 3: hipLaunchKernelGGL((gemv_glu_lds_kernel<WAVES, 3>), grid, block, 0, s, g, u, mb, x, h, n, nb, xrb); break;
        default: hipLaunchKernelGGL((gemv_glu_lds_kernel<WAVES, 4>), grid, block, 0, s, g, u, mb, x, h, n, nb, xrb); break;
        }
        return hipGetLastError();
    }
    if (!gemv_glu_supported(w_type, G, U, n_rows, k)) return hipErrorInvalidValue;
    const uint8_t* g = static_cast<const uint8_t*>(G);
    const uint8_t* u = static_cast<const uint8_t*>(U);
    const uint8_t* x = static_cast<const uint8_t*>(xq);
    const size_t rb = k / 256 * 144;
    const int n = (int)n_rows, kk = (int)k;
    // measured at the Llama-3-8B FFN (14336 x 4096, three paired runs on one
    // box): the whole FFN 23.98-24.03 against 25.09-25.12 us
    if (k <= 4096 && n_rows * rb < 0x80000000ull && tuning_env(TUNE_GEMV_LDS, 1) != 0) {
        constexpr int WAVES = 4;
        hipLaunchKernelGGL((gemv_glu_lds_kernel<WAVES, 1>), dim3((unsigned)((n + WAVES - 1) / WAVES)), dim3(WAVES * 64),
                           0, s, g, u, (uint32_t)(n_rows * rb), x, h, n, kk / 256, 0u);
        return hipGetLastError();
    }
    // BARQ_GEMV_GLU = 10 * P + W: P outputs per wave (1 or 2), W waves (2, 4, 8)
    const int t = tuning_env(TUNE_GEMV_GLU, 14);
    const int p = t / 10 == 2 ? 2 : 1;
    const int w = t % 10 == 2 || t % 10 == 8 ? t % 10 : 4;
    if (p == 2) return w == 2 ? launch_glu<2, 2>(g, u, rb, x, h, n, kk, s) : w == 8 ? launch_glu<2, 8>(g, u, rb, x, h, n, kk, s)
                                                                                   : launch_glu<2, 4>(g, u, rb, x, h, n, kk, s);
    return w == 2 ? launch_glu<1, 2>(g, u, rb, x, h, n, kk, s) : w == 8 ? launch_glu<1, 8>(g, u, rb, x, h, n, kk, s)
                                                                       : launch_glu<1, 4>(g, u, rb, x, h, n, kk, s);
}

hipError_t gemv_f32_launch(int w_type, const void* W, size_t n_rows, size_t k, const float* x,
                           float* y, hipStream_t s) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    const int n = (int)n_rows, kk = (int)k;
    switch (w_type) {
    case TYPE_Q4_K: return launch_f32<FmtQ4K, 2, 4>(w, k / 256 * 144, x, y, n, kk, s);
    case TYPE_Q6_K: return launch_f32<FmtQ6K, 2, 4>(w, k / 256 * 210, x, y, n, kk, s);
    case TYPE_Q4_0: return launch_f32<FmtQ40, 2, 4>(w, k / 32 * 18, x, y, n, kk, s);
    case TYPE_Q8_0: return launch_f32<FmtQ80, 2, 4>(w, k / 32 * 34, x, y, n, kk, s);
    case TYPE_Q4_0_BARQ: return launch_f32<FmtQ40Barq, 2, 4>(w, k / 32 * 20, x, y, n, kk, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace barq
