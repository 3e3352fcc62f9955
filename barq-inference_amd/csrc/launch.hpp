// Host-side launchers of the gfx950 kernels (internal to libbarq_rocm).
// Every launcher enqueues on `s` and returns hipGetLastError().
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace barq {

// dequant.hip
hipError_t dequant_launch(int type, const void* blocks, size_t n_elems, float* out, hipStream_t s);
// get_embeddings: rows tokens[t] of a table of n_rows rows (k elements,
// row_bytes each) decoded to f32 rows of out; out-of-range ids give zeros
hipError_t get_rows_launch(int type, const void* table, size_t row_bytes, size_t n_rows, size_t k,
                           const int32_t* tokens, size_t n_tokens, float* out, hipStream_t s);
hipError_t dequant_split_launch(int kind_q8_0, const uint8_t* quants, size_t n_quants,
                                const float* scales, size_t n_scales, size_t block_size,
                                float* out, size_t n_out, hipStream_t s);

// quantize.hip
hipError_t quantize_q8_0_launch(const float* x, size_t n_rows, size_t k, void* out, hipStream_t s);
hipError_t quantize_q8_k_launch(const float* x, size_t n_rows, size_t k, void* out, hipStream_t s);
hipError_t quantize_q4_0_barq_launch(const float* x, size_t n, uint8_t* out, hipStream_t s);
// quant::Q4_K::quantize (quant/src/q4_k.rs:23-73): 136-byte blocks, a shorter last one
hipError_t quantize_q4_k_barq_launch(const float* x, size_t n, uint8_t* out, hipStream_t s);
// Q8_K rows of x[rows_idx[i] * k ..] for i < n_rows (gather fused in)
hipError_t quantize_q8_k_gather_launch(const float* x, const int32_t* rows_idx, size_t n_rows, size_t k, void* out,
                                       hipStream_t s);
// Q8_K rows of silu(g) * u with ops::Silu's rounding (the MoE expert FFN;
// k-element rows; the product is not stored)
hipError_t swiglu_q8_k_launch(const float* g, const float* u, size_t n_rows, size_t k, void* out, hipStream_t s);
// The dense FFN's SwiGLU (transformer.rs:394-399) of n_rows rows of n:
// out_type TYPE_F32 writes f32 h, TYPE_Q8_K / TYPE_Q8_0 its blocks
hipError_t ffn_swiglu_launch(int out_type, const float* g, const float* u, size_t n_rows, size_t n, void* out,
                             hipStream_t s);

// norm.hip: RMSNorm rows (transformer.rs:148-172), alone or fused with the
// Q8_K / Q8_0 quantizer (n % 256 == 0 for the fused form)
bool rms_norm_supported(size_t n);
hipError_t rms_norm_launch(const float* x, const float* w, size_t rows, size_t n, float eps, float* y,
                           hipStream_t s);
hipError_t rms_norm_quantize_launch(int act_type, const float* x, const float* w, size_t rows, size_t n, float eps,
                                    void* out, hipStream_t s);
// RMSNorm of x + d (d may be null), the sum stored to `sum` when non-null;
// out_type TYPE_F32 (f32 rows), TYPE_Q8_K or TYPE_Q8_0 (n % 256 == 0)
hipError_t add_rms_norm_launch(int out_type, const float* x, const float* d, const float* w, size_t rows, size_t n,
                               float eps, float* sum, void* out, hipStream_t s);
// y[r, j] += bias[j] (rows x dim, in place)
hipError_t add_bias_launch(float* y, const float* bias, size_t rows, size_t dim, hipStream_t s);

// gemv.hip
hipError_t gemv_q8_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq,
                          float* y, hipStream_t s);
hipError_t gemv_f32_launch(int w_type, const void* W, size_t n_rows, size_t k, const float* x,
                           float* y, hipStream_t s);
// Expert-grouped GEMV for decode-size MoE steps (Q4_K or Q6_K weights
// W[mat * n_experts + e], grouped Q8_K rows, row ranges from the device
// offsets; y rows of y + mat * y_mat_stride in grouped order)
constexpr int MOE_GEMV_MAXE = 64;
bool moe_gemv_supported(int w_type, size_t n_experts, size_t n_mats, size_t n_rows, size_t k);
int moe_gemv_enabled();   // BARQ_MOE_GEMV (0: off, 1: one-token steps, 2: up to 4 assignments)
hipError_t moe_gemv_launch(int w_type, const void* const* W, size_t n_experts, size_t n_mats, const int32_t* offsets,
                           size_t n_assign, size_t tokens, const void* xq, size_t n_rows, size_t k, float* y,
                           size_t y_mat_stride, hipStream_t s);
// Gate and up of one Q8_K row in one launch with the dense SwiGLU in the
// epilogue: h[n_rows] (Q4_K weights, 16-byte aligned)
bool gemv_glu_supported(int w_type, const void* G, const void* U, size_t n_rows, size_t k);
// m = 2-4 activation rows (x_row_bytes apart, h [m x n_rows]): the
// LDS-staged launch only (gemv_glu_multi_supported)
hipError_t gemv_glu_launch(int w_type, const void* G, const void* U, size_t n_rows, size_t k, const void* xq, float* h,
                           hipStream_t s, size_t m = 1);
bool gemv_glu_multi_supported(int w_type, const void* G, const void* U, size_t n_rows, size_t k, size_t m);
// 2-4 Q8 activation rows at once (y[m x n_rows]): the weights read once
bool gemv_multi_supported(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m);
hipError_t gemv_q8_multi_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m,
                                float* y, hipStream_t s);

// gemv_dma.hip: the same GEMV streaming row slices through LDS
bool gemv_dma_supported(int w_type, const void* W, size_t n_rows, size_t k, const void* xq);
hipError_t gemv_dma_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, float* y,
                           hipStream_t s, size_t m = 1);
bool gemv_dma_multi_fits(int w_type, size_t k, size_t m);

// gemm_mfma.hip: Y[m x n] = X W^T with int8 MFMA (X as Q8_K rows); ws holds
// gemm_mfma_workspace(...) bytes (K slices' partial products, often none)
hipError_t gemm_q8k_mfma_launch(int w_type, const void* W, size_t n_rows, size_t k,
                                const void* xq, size_t m, void* ws, float* y, hipStream_t s);
bool gemm_mfma_supported(int w_type, size_t n_rows, size_t k, size_t m);
size_t gemm_mfma_workspace(int w_type, size_t n_rows, size_t k, size_t m);

// gemm_b32.hip: Y[m x n] = X W^T for Q4_0, Q8_0 and Q4_0_BARQ weights against
// Q8_0 rows xq (k % 256 == 0); ws holds b32_workspace(m, n_rows, k) bytes
// (the activation repacked into int8 rows, an f32 scale table and, when few
// tiles split K across workgroups, the slices' partial products)
bool b32_supported(int w_type, size_t n_rows, size_t k, size_t m);
size_t b32_workspace(size_t m, size_t n_rows, size_t k);
// y[i] = sum over ks slices of parts[slice * n + i], in slice order
hipError_t slice_sum_launch(const float* parts, int ks, size_t n, float* y, hipStream_t s);
hipError_t b32_gemm_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m, void* ws,
                           float* y, hipStream_t s);

// gemm_kq.hip: the same product with 32x32x32 int8 MFMA tiles fed by
// buffer->LDS loads; Q4_K any k % 256 == 0, Q6_K an even number of super-blocks.
bool kq_supported(int w_type, size_t n_rows, size_t k, size_t m);
// ws holds kq_workspace(w_type, m, n_rows, k) bytes: with few tiles K is split across
// workgroups, whose partial products slice_sum_launch adds (ws null: one slice)
hipError_t kq_gemm_launch(int w_type, const void* W, size_t n_rows, size_t k, const void* xq, size_t m, void* ws,
                          float* y, hipStream_t s);
int kq_k_slices(int w_type, size_t m, size_t n_rows, size_t k);
size_t kq_workspace(int w_type, size_t m, size_t n_rows, size_t k);
// Expert-grouped form: rows [offsets[e], offsets[e+1]) of xq, and of
// y + mat * y_mat_stride, use weights W[mat * n_experts + e] (offsets on the
// device; n_experts * n_mats <= 64).  total_rows bounds offsets[n_experts].
// With k_slices > 1 slice i covers super-blocks [i, i + 1) * nsb / k_slices
// and writes its partial product to y + i * y_k_stride (nsb / k_slices even).
hipError_t kq_grouped_launch(int w_type, const void* const* W, size_t n_experts, size_t n_mats, const int32_t* offsets,
                             size_t total_rows, size_t n_rows, size_t k, const void* xq, float* y, size_t y_mat_stride,
                             size_t k_slices, size_t y_k_stride, hipStream_t s);
int kq_k_slices_override();
// rows from which matmul takes the MFMA GEMMs (BARQ_GEMM_MIN_M overrides)
int gemm_min_rows(int w_type);

// f32blas.hip
hipError_t gemm_f32_launch(const float* a, const float* b, size_t m, size_t k, size_t n, float* c,
                           hipStream_t s);
hipError_t gemv_f32_plain_launch(const float* a, const float* x, size_t m, size_t n, float* y,
                                 hipStream_t s);
// C[m x n] = A[m x k] B^T with B stored [n x k] (dequantized GGUF rows)
hipError_t gemm_f32_nt_launch(const float* a, const float* b_nk, size_t m, size_t k, size_t n, float* c,
                              hipStream_t s);

// moe.hip
// top-k routing; max_active > 0 adds reduce_expert_assignments (dropped
// slots: id -1, weight 0)
hipError_t moe_route_launch(const float* logits, size_t rows, size_t n_experts, size_t top_k,
                            int32_t* ids, float* weights, hipStream_t s, size_t max_active = 0,
                            float min_weight = 0.0f);
// reduce_expert_assignments on rows x k slots (out may alias in)
hipError_t moe_reduce_launch(const int32_t* ids, const float* weights, size_t rows, size_t k, size_t max_active,
                             float min_weight, int32_t* out_ids, float* out_weights, hipStream_t s);
// CSR grouping of routing assignments (batch_by_expert): offsets[n_experts+1],
// tokens/wts[rows*top_k] in expert-major, ascending-token order.
hipError_t moe_group_launch(const int32_t* ids, const float* weights, size_t rows, size_t top_k,
                            size_t n_experts, int32_t* offsets, int32_t* tokens, float* wts,
                            int32_t* rowpos, hipStream_t s);
// moe_group_launch followed by quantize_q8_k_gather_launch(x, tokens) in one
// launch (rows * top_k <= 2048, hidden % 256 == 0); the second reports the
// BARQ_MOE_FUSED_GROUP tuning switch (0: two launches)
int moe_fused_group_enabled();
hipError_t moe_group_gather_q8k_launch(const int32_t* ids, const float* weights, size_t rows, size_t top_k,
                                       size_t n_experts, const float* x, size_t hidden, void* out, int32_t* offsets,
                                       int32_t* tokens, float* wts, int32_t* rowpos, hipStream_t s);
// xg[i] = x[tokens[i]] for i < n_assign
hipError_t moe_gather_launch(const float* x, const int32_t* tokens, size_t n_assign, size_t hidden,
                             float* xg, hipStream_t s);
// h = silu(g) * u elementwise (ops.rs:191-211 and moe_fused.rs:61-66)
hipError_t swiglu_launch(const float* g, const float* u, size_t n, float* h, hipStream_t s);
// out[t] = sum over t's assignments in ascending expert id of w * yg[row]
// rowpos[t*top_k+i] is the grouped row of assignment (t, i) or -1
// yg holds `parts` partial results yg + i * part_stride that are summed first
hipError_t moe_scatter_launch(const float* yg, const int32_t* ids, const float* weights,
                              const int32_t* rowpos, size_t rows, size_t top_k, size_t hidden,
                              float* out, hipStream_t s, int parts = 1, size_t part_stride = 0);

// ---- attention (attention.hip) ----
constexpr int ROPE_INTERLEAVED = 0, ROPE_SPLIT_HALF = 1;
// apply_rope: x [seq, heads * hd] -> out[h * out_head_stride + p * hd + d]
hipError_t rope_launch(int layout, const float* x, float* out, size_t seq, size_t heads, size_t hd, size_t start_pos,
                       float freq_scale, const float* inv_freq, size_t out_head_stride, hipStream_t s);
// transpose_heads: x [seq, heads * hd] -> out[h * out_head_stride + p * hd + d]
hipError_t transpose_heads_launch(const float* x, float* out, size_t seq, size_t heads, size_t hd,
                                  size_t out_head_stride, hipStream_t s);
struct AttnArgs {
    const float* q;           // [n_head, q_len, head_dim]
    const float* k;           // cache base: [layer][kv head][position][head_dim]
    const float* v;
    size_t layer_off;         // floats from the base to the layer
    size_t head_stride;       // floats between kv heads (max_size * head_dim)
    size_t n_head, n_head_kv, head_dim, q_len, kv_len, start_pos;
    float* part;              // split partials (attention_workspace bytes)
    float* out;               // [q_len, n_head, head_dim]
    uint8_t* out_q8;          // optional: the output rows as Q8_K blocks (see attention_q8_direct)
};
bool attention_q8_direct(const AttnArgs& a);
bool gemv_group_supported(size_t n, const int* types, const void* const* W, const size_t* rows, size_t k);
bool qkv_rope_supported(const int* types, const void* const* W, size_t n_q_rows, size_t n_kv_rows, size_t k,
                        size_t hd);
hipError_t qkv_rope_launch(const int* types, const void* const* W, size_t n_q_rows, size_t n_kv_rows, size_t k,
                           const void* xq, size_t hd, float* q_out, float* k_dst, float* v_dst, size_t head_stride,
                           size_t start_pos, float freq_scale, const float* inv_freq, hipStream_t s);
hipError_t gemv_group_launch(size_t n, const int* types, const void* const* W, const size_t* rows, size_t k,
                             const void* xq, float* const* y, hipStream_t s);
hipError_t rope_qkv_launch(int layout, const float* qx, const float* kx, const float* vx, float* q_out, float* k_out,
                           float* v_out, size_t seq, size_t n_q, size_t n_kv, size_t hd, size_t start_pos,
                           float freq_scale, const float* inv_freq, size_t cache_head_stride, hipStream_t s);
bool attention_supported(size_t head_dim);
// probe.hip: read `bytes` (rounded down to 16) once with non-temporal loads
hipError_t stream_read_launch(const void* p, size_t bytes, uint32_t* sink, hipStream_t s);

void attention_plan(size_t n_head, size_t n_head_kv, size_t q_len, size_t kv_len, int* n_split, int* chunk);
size_t attention_workspace(size_t n_head, size_t head_dim, size_t q_len, size_t kv_len, size_t n_head_kv);
hipError_t attention_launch(const AttnArgs& a, hipStream_t s);

}  // namespace barq
