// Batched K-quant x Q8_K GEMM: tile and launch-shape choice and the entry
// points (the kernels are in gemm_kq.hpp).
#include "gemm_kq.hpp"

namespace barq {

// Overrides: BARQ_GEMM_BM (16, 32, 64, or 65 = 64 rows with eight waves of
// 32 x 32 per K-group),
// BARQ_GEMM_NS (stages), BARQ_GEMM_KG (K-groups, ungrouped), BARQ_GEMM_KS
// (K slices: the MoE down projection, and ungrouped launches).

// rows: M (ungrouped) or the expected rows per expert (grouped).  Stage
// counts are the most that fit the 160 KiB of LDS (deeper pipelines keep
// more HBM requests in flight per CU).
// Q6_K prompts: 64-row tiles of four waves (each weight slice decoded once for
// two MFMA row tiles) where the tiles fill the CUs without K slices or K is
// long; measured on MI355X, M = 128 / 256 / 512, us per call (default against
// these tiles): 4096 x 14336 44.9 / 78.9 / 155.4 against 38.7 / 67.3 / 119.8;
// 4096 x 4096 19.3 / 25.9 / 49.5 against 19.5 / 27.9 / 38.3; M = 64: 27.7 and
// 14.5 against 37.1 and 16.4.
static bool kq6_wide_tiles(size_t m, size_t n_rows, size_t nsb) {
    const size_t tiles = (m + 63) / 64 * ((n_rows + KQ_BN - 1) / KQ_BN);
    return tiles >= 256 || (m >= 128 && nsb >= 32);
}

// Q6_K prompts of 256+ rows against long K or many weight rows: 128 x 128
// tiles (kq6_tall_launch; K slices fill the CUs).  Measured on MI355X, us per
// call against the 64-row tiles (paired runs, one box): 4096 x 14336 (the down
// projection) M = 512 / 256: 110.0-110.5 / 64.2-64.5 against 129.1-129.5 /
// 73.1-74.7; 14336 x 4096 M = 512 / 256: 121.5 / 64.0-64.8 against 155.3-155.4
// / 79.6; 4096 x 4096 M = 512: 43.6-44.0 against 43.9-44.4 and M = 256:
// 30.3-30.6 against 28.5-28.7, 1024 x 4096 M = 512: 22.3 against 19.0-19.1
// (so those keep the 64-row tiles).  BARQ_GEMM_BM=67 forces them.
static bool kq6_tall_tiles(size_t m, size_t n_rows, size_t nsb) {
    const int bm_env = tuning_env(TUNE_GEMM_BM);
    if (bm_env) return bm_env == 67;
    return m >= 256 && (nsb >= 32 || n_rows >= 8192);
}

template <class F, bool GROUPED>
static hipError_t kq_dispatch(const KQArgs& a, size_t rows, hipStream_t s) {
    // measured on MI355X: 64x128 tiles above 32 rows, 32-row tiles with four
    // waves for small expert groups.  With two K-groups, each wave of a 64-row
    // tile covers both 32-row halves of its 32 columns (bm 64: the weight
    // fragment is decoded once for two MFMA row tiles; 26.5-27.1 against
    // 27.6-29.0 us at C4 for eight waves of 32 x 32, bm 65)
    const int g_kq_ns = tuning_env(TUNE_GEMM_NS), g_kq_bm = tuning_env(TUNE_GEMM_BM);
    const int bm = g_kq_bm ? g_kq_bm
                 : (!GROUPED && F::TYPE == TYPE_Q6_K && kq6_wide_tiles(rows, (size_t)a.N, (size_t)a.nsb)) ? 66
                 : (rows > 32 ? 64 : 32);
    if (bm == 16) {
        if (g_kq_ns == 2) return kq_launch_t<F, 16, 2, 4, GROUPED>(a, s);
        if (g_kq_ns == 4) return kq_launch_t<F, 16, 4, 4, GROUPED>(a, s);
        return kq_launch_t<F, 16, 3, 4, GROUPED>(a, s);
    }
    // 32-row tiles: two stages per workgroup and two workgroups per CU for
    // expert groups (measured best for C5), the deepest pipeline otherwise
    const int ns = g_kq_ns ? g_kq_ns : (GROUPED ? 2 : 0);
    if constexpr (!GROUPED && F::TYPE == TYPE_Q6_K) {
        if (kq6_tall_tiles(rows, (size_t)a.N, (size_t)a.nsb)) return kq6_tall_launch(a, s);
        // 64 x 128 tiles with four waves of 64 x 32 (each weight slice decoded
        // once for two MFMA row tiles), one K-group, three stages
        if (bm == 66) return kq_launch_t<F, 64, 3, 4, GROUPED>(a, s);
    }
    if constexpr (!GROUPED) {
        // two K-groups of waves share a tile's pipeline (twice the waves per
        // SIMD for the same LDS) when the super-block count is even
        const int kg = tuning_env(TUNE_GEMM_KG, 2);
        if (kg == 2 && (a.nsb / a.ks) % 2 == 0) {
            if constexpr (F::TYPE == TYPE_Q4_K) {
                if (bm == 65) return kq_launch_t<F, 64, 2, 8, GROUPED, 2>(a, s);
                if (bm == 64) {
                    // BARQ_GEMM_DEFER: bit 0 defers group 1's epilogue, bit 1 loads weight
                    // pairs; measured at C4 on MI355X (alternating runs, one process):
                    // 24.7-24.8 us with neither, 23.7-24.3 / 24.3-24.4 with one, 23.6-23.9 with both
                    const int mode = tuning_env(TUNE_GEMM_DEFER, 3);
                    if (mode == 3) return kq_launch_t<F, 64, 2, 4, GROUPED, 2, true, true>(a, s);
                    if (mode == 2) return kq_launch_t<F, 64, 2, 4, GROUPED, 2, false, true>(a, s);
                    if (mode == 1) return kq_launch_t<F, 64, 2, 4, GROUPED, 2, true>(a, s);
                    return kq_launch_t<F, 64, 2, 4, GROUPED, 2>(a, s);
                }
                return kq_launch_t<F, 32, 2, 4, GROUPED, 2>(a, s);
            } else {
                return kq_launch_t<F, 32, 2, 4, GROUPED, 2>(a, s);
            }
        }
    }
    if constexpr (F::TYPE == TYPE_Q4_K) {
        if (bm >= 64) return kq_launch_t<F, 64, 4, 8, GROUPED>(a, s);
        if (ns == 2) return kq_launch_t<F, 32, 2, 4, GROUPED>(a, s);
        if (ns == 3) return kq_launch_t<F, 32, 3, 4, GROUPED>(a, s);
        if (ns == 4) return kq_launch_t<F, 32, 4, 4, GROUPED>(a, s);
        return kq_launch_t<F, 32, 5, 4, GROUPED>(a, s);
    } else {
        if (bm >= 64) return kq_launch_t<F, 64, 3, 8, GROUPED>(a, s);
        if (ns == 2) return kq_launch_t<F, 32, 2, 4, GROUPED>(a, s);
        if (ns == 3) return kq_launch_t<F, 32, 3, 4, GROUPED>(a, s);
        return kq_launch_t<F, 32, 4, 4, GROUPED>(a, s);
    }
}

// Raw buffer loads use 32-bit offsets: each weight matrix and the activation
// rows must stay below 2 GiB.  Q6_K needs row bytes that are a multiple of 4
// (an even number of super-blocks).
int kq_k_slices_override() { return tuning_env(TUNE_GEMM_KS); }

// Activation rows from which matmul runs the MFMA GEMMs instead of one GEMV
// per row (BARQ_GEMM_MIN_M overrides; at least 2).  Measured on MI355X at
// 4096 x 4096, 14336 x 4096 and 4096 x 14336 (K slices spread the few tiles):
// the K-quant and Q8_0 GEMMs beat three GEMVs, and the Q4_0 GEMM four (Q4_K
// 4096 x 4096: 9.5 us against 9.3 / 12.1 us for three / four GEMVs; Q4_0
// 12.8 against 10.2 / 13.4).
int gemm_min_rows(int w_type) {
    const int def = w_type == TYPE_Q4_0 || w_type == TYPE_Q4_0_BARQ ? 4 : 3;
    const int v = tuning_env(TUNE_GEMM_MIN_M, def);
    return v < 2 ? 2 : v;
}

bool kq_supported(int w_type, size_t n_rows, size_t k, size_t m) {
    if ((w_type != TYPE_Q4_K && w_type != TYPE_Q6_K) || k % 256 != 0 || k == 0 || n_rows == 0) return false;
    const size_t nsb = k / 256;
    if (w_type == TYPE_Q6_K && (nsb & 1)) return false;
    const size_t wbytes = n_rows * nsb * (w_type == TYPE_Q4_K ? Q4_K_BYTES : Q6_K_BYTES);
    const size_t xbytes = m * nsb * Q8_K_BYTES;
    return wbytes < (1ull << 31) && xbytes < (1ull << 31) && n_rows <= (size_t)INT32_MAX;
}

static KQArgs kq_args(int w_type, size_t n_rows, size_t k, const void* xq, float* y) {
    KQArgs a = {};
    a.nsb = (int)(k / 256);
    a.wrb = (uint32_t)(a.nsb * (w_type == TYPE_Q4_K ? Q4_K_BYTES : Q6_K_BYTES));
    a.xrb = (uint32_t)(a.nsb * Q8_K_BYTES);
    a.X = static_cast<const uint8_t*>(xq);
    a.Y = y;
    a.N = (int)n_rows;
    a.ne = a.nmat = a.ks = 1;
    return a;
}

// K slices of an ungrouped launch when the tiles alone would leave most CUs
// idle: doubled while the grid stays within 256 workgroups and every slice
// keeps an even number of super-blocks (two K-groups; Q6_K windows keep
// their parity).  BARQ_GEMM_KS overrides (a power of two up to 16).
// The tile height kq_dispatch picks (for an even super-block count per slice).
static size_t kq_tile_rows(int w_type, size_t m, size_t n_rows, size_t nsb) {
    const int bm_env = tuning_env(TUNE_GEMM_BM);
    const int bm = bm_env ? bm_env : (w_type == TYPE_Q6_K && kq6_wide_tiles(m, n_rows, nsb)) ? 66 : (m > 32 ? 64 : 32);
    if (w_type == TYPE_Q6_K && kq6_tall_tiles(m, n_rows, nsb)) return 128;
    if (bm == 16) return 16;
    if (bm == 66 && w_type == TYPE_Q6_K) return 64;
    if (tuning_env(TUNE_GEMM_KG, 2) == 2) return w_type == TYPE_Q4_K && (bm == 64 || bm == 65) ? 64 : 32;
    return bm >= 64 ? 64 : 32;
}

int kq_k_slices(int w_type, size_t m, size_t n_rows, size_t k) {
    const size_t bm = kq_tile_rows(w_type, m, n_rows, k / 256);
    const size_t tiles = (m + bm - 1) / bm * ((n_rows + KQ_BN - 1) / KQ_BN), nsb = k / 256;
    int ks = 1;
    while (ks < 16 && tiles * ks * 2 <= 256 && nsb % (size_t)(ks * 4) == 0) ks *= 2;
    const int ovr = tuning_env(TUNE_GEMM_KS);
    if (ovr > 0 && (ovr & (ovr - 1)) == 0 && ovr <= 16 && nsb % (size_t)(2 * ovr) == 0) ks = ovr;
    return ks;
}

size_t kq_workspace(int w_type, size_t m, size_t n_rows, size_t k) {
    const int ks = kq_k_slices(w_type, m, n_rows, k);
    return ks > 1 ? (size_t)ks * m * n_rows * 4 : 0;
}

hipError_t kq_gemm_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m, void* ws,
                          float* y, hipStream_t s) {
    if (m == 0 || n_rows == 0) return hipSuccess;
    if (!kq_supported(w_type, n_rows, k, m)) return hipErrorInvalidValue;
    const int ks = ws ? kq_k_slices(w_type, m, n_rows, k) : 1;   // no workspace: one slice
    float* parts = ks > 1 ? static_cast<float*>(ws) : y;
    KQArgs a = kq_args(w_type, n_rows, k, xq, parts);
    a.wt.w[0] = static_cast<const uint8_t*>(W);
    a.M = (int)m;
    a.ks = ks;
    hipError_t e = w_type == TYPE_Q4_K ? kq_dispatch<KQ4, false>(a, m, s) : kq_dispatch<KQ6, false>(a, m, s);
    if (e != hipSuccess || ks == 1) return e;
    return slice_sum_launch(parts, ks, m * n_rows, y, s);
}

hipError_t kq_grouped_launch(int w_type, const void* const* W, size_t n_experts, size_t n_mats, const int32_t* offsets,
                             size_t total_rows, size_t n_rows, size_t k, const void* xq, float* y, size_t y_mat_stride,
                             size_t k_slices, size_t y_k_stride, hipStream_t s) {
    if (n_experts == 0 || n_mats == 0 || total_rows == 0 || n_rows == 0) return hipSuccess;
    if (n_experts * n_mats > (size_t)KQ_MAXE || n_experts > 64 || !kq_supported(w_type, n_rows, k, total_rows) ||
        total_rows > (size_t)INT32_MAX || k_slices == 0 || (k_slices > 1 && (k / 256) % (2 * k_slices) != 0))
        return hipErrorInvalidValue;
    KQArgs a = kq_args(w_type, n_rows, k, xq, y);
    for (size_t i = 0; i < n_experts * n_mats; i++) a.wt.w[i] = static_cast<const uint8_t*>(W[i]);
    a.offsets = offsets;
    a.ne = (int)n_experts;
    a.nmat = (int)n_mats;
    a.total_rows = total_rows;
    a.ymat = y_mat_stride;
    a.ks = (int)k_slices;
    a.ykstride = y_k_stride;
    const size_t per_expert = (total_rows + n_experts - 1) / n_experts;
    return w_type == TYPE_Q4_K ? kq_dispatch<KQ4, true>(a, per_expert, s) : kq_dispatch<KQ6, true>(a, per_expert, s);
}

}  // namespace barq
