/*
 * barq_oracle.h — CPU restatement of barq-inference's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X kernels in libbarq_rocm.so.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it, and only as the checker
 * or the timed CPU baseline — never as a product code path.
 *
 * Every function restates a piece of the reference (Rust, read as text at
 * /root/reference) and cites the file:line it follows.  The reference could
 * not be compiled here (no Rust toolchain), so this restatement is pinned by
 * known-answer tests, closed forms and brute force (tests/test_oracle_*.py).
 *
 * Build: gcc -O2 -ffp-contract=off (Rust never contracts a*b-c into an FMA;
 * the decoders must round every product and difference separately).
 */
#ifndef BARQ_ORACLE_H
#define BARQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids: barq_core/src/gguf.rs:117-137 */
enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_Q4_0 = 2,  /* GGUF/llama.cpp block_q4_0: f16 d + 16 B, 18 B / 32 */
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
    ORC_Q6_K = 14,
    ORC_Q8_K = 15,
    /* The reference's own Q4_0 layout (gguf.rs:521-578, quant/src/q4_0.rs):
       f32 scale + 16 B, interleaved sign-extended nibbles, 20 B / 32. */
    ORC_Q4_0_BARQ = 0x10002,
};

/* Block geometry: elements per block and bytes per block (0 for unknown). */
size_t orc_block_elems(int type);
size_t orc_block_bytes(int type);

/* IEEE binary16 <-> binary32.  to_f32 restates half 2.7.1 f16::to_f32
   (exact widening, used at gguf.rs:661,763,768,869).  from_f32 is
   round-to-nearest-even (half::f16::from_f32; GGML_FP32_TO_FP16). */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- block decoders (dequantize to f32) -------------------------------- */
/* Each returns the number of elements written (the reference truncates to
   total_elements, gguf.rs:576,679,821,912). */
size_t orc_dequant_q4_0_barq(const uint8_t* data, size_t total_elements, float* out); /* gguf.rs:521-578 */
size_t orc_dequant_q8_0(const uint8_t* data, size_t total_elements, float* out);      /* gguf.rs:634-681 */
size_t orc_dequant_q4_k(const uint8_t* data, size_t total_elements, float* out);      /* gguf.rs:730-823 */
size_t orc_dequant_q6_k(const uint8_t* data, size_t total_elements, float* out);      /* gguf.rs:839-914 */
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);          /* gguf.rs:825-837 */
/* GGUF Q4_0 (18 B) decoded through the byte adapter onto the reference's
   20-B decoder: the two decode to identical f32. */
void orc_q4_0_gguf_to_barq(const uint8_t* gguf, size_t n_blocks, uint8_t* barq);
size_t orc_dequant_q4_0_gguf(const uint8_t* data, size_t total_elements, float* out);
/* Q8_K activation blocks: y = d * q (llama.cpp dequantize_row_q8_K). */
size_t orc_dequant_q8_k(const uint8_t* data, size_t total_elements, float* out);
/* Dispatch on type id, mirroring GgufReader::load_tensor (gguf.rs:437-514).
   Returns elements written or (size_t)-1 for an unsupported type. */
size_t orc_dequantize(int type, const uint8_t* data, size_t total_elements, float* out);

/* K-quant scale packing encoder (quant/src/q5_k.rs:175-182): 8 six-bit
   scales and 8 six-bit mins -> 12 bytes.  Used to pin the decoder. */
void orc_pack_scale_min_k4(const uint8_t ls[8], const uint8_t lm[8], uint8_t out[12]);

/* ---- activation quantizers (absent from the reference; llama.cpp spec) -- */
/* Q8_0: d = amax/127 (stored f16), q = roundf(x * (1/d)).  34 B / 32. */
void orc_quantize_q8_0(const float* x, size_t k, uint8_t* out);
/* Q8_K: iscale = -127/max (max = signed value of largest |x|, first wins),
   q = min(127, rne(iscale*x)), d = 1/iscale, bsums[16].  292 B / 256. */
void orc_quantize_q8_k(const float* x, size_t k, uint8_t* out);

/* ---- the reference's f32 arithmetic ----------------------------------- */
/* blas::gemv_f32 CPU fallback, barq_core/src/blas.rs:292-303:
   y[i] = sum_j a[i*n+j]*x[j], sequential f32, unfused. */
/* RMSNorm rows (transformer.rs:148-172), sequential sum of squares */
void orc_rms_norm(const float* x, const float* w, size_t rows, size_t n, float eps, float* y);
void orc_gemv_f32(const float* a, const float* x, size_t m, size_t n, float* y);
/* blas::gemm_f32 CPU fallback, blas.rs:193-212: C[m x n] = A[m x k] B[k x n],
   per (i,j) a sequential unfused f32 sum over kk. */
void orc_gemm_f32(const float* a, const float* b, size_t m, size_t k, size_t n, float* c);

/* Quantized matvec / matmul semantics, W is GGUF [n_rows x k] with blocks
   along k.  act_type = ORC_F32: y = gemv_f32(dequant(W), x)  (the literal
   reference path).  act_type = ORC_Q8_0 / ORC_Q8_K: x is already-quantized
   activation blocks; y = gemv_f32(dequant(W), dequant(x)).  Returns 0 on
   success, -1 on a bad type/shape. */
int orc_matvec(int w_type, const uint8_t* w, size_t n_rows, size_t k,
               int act_type, const void* x, float* y);
/* Y[m x n_rows] row-major: row r of X (f32 or Q8 blocks, k per row). */
int orc_matmul(int w_type, const uint8_t* w, size_t n_rows, size_t k,
               int act_type, const void* x, size_t m, float* y);

/* ---- the reference's quant crate and split-scale operator API ---------- */
/* quant::Q4_0::quantize (quant/src/q4_0.rs:23-67): 20-B barq blocks.
   Returns bytes written. */
size_t orc_q4_0_quantize_barq(const float* x, size_t n, uint8_t* out);
/* backend/src/cuda_quant.rs:44-75 dequantize_packed_4bit_host */
void orc_dequantize_packed_4bit_split(const uint8_t* quants, size_t n_quants,
                                      const float* scales, size_t n_scales,
                                      size_t block_size, float* out, size_t n_out);
/* backend/src/cuda_quant.rs:77-102 dequantize_signed_8bit_host */
void orc_dequantize_signed_8bit_split(const uint8_t* quants, size_t n_quants,
                                      const float* scales, size_t n_scales,
                                      size_t block_size, float* out, size_t n_out);
/* backend/src/cuda_quant.rs:104-126 quantized_matmul_host: dequantize B
   [k x n] (split layout, kind 8 = Q8_0 signed bytes, else packed 4-bit),
   then gemm_f32(a, B, m, k, n).  c is m x n. */
void orc_quantized_matmul_split(const float* a, const uint8_t* bq, size_t n_bq,
                                const float* bscales, size_t n_bscales,
                                size_t m, size_t n, size_t k, int quant_is_q8_0,
                                size_t block_size, float* c);

/* ---- fused MoE helpers (models/src/moe_fused.rs) ----------------------- */
/* select_top_k_experts (moe_fused.rs:95-144).  ids/weights are
   rows x k_eff, k_eff = clamp(k, 1, cols) is returned (0 on bad input). */
size_t orc_moe_select_top_k(const float* logits, size_t rows, size_t cols,
                            size_t k, int32_t* ids, float* weights);
/* reduce_expert_assignments (moe_fused.rs:147-194), smart expert reduction:
   per row, keep the assignments with weight >= min_weight (if none, the
   largest, the later slot winning ties), sorted by weight descending
   (stable), at most max(max_active, 1), weights renormalised by their
   sequential sum floored at f32::EPSILON.  ids/weights are rows x k; ids < 0
   are absent slots.  Output rows x k: kept assignments first, then id -1,
   weight 0 (out may alias in). */
void orc_moe_reduce_experts(const int32_t* ids, const float* weights, size_t rows, size_t k,
                            size_t max_active, float min_weight, int32_t* out_ids, float* out_weights);
/* batch_by_expert (moe_fused.rs:196-223): CSR grouping.  offsets has
   n_experts+1 entries; tokens/wts have rows*k entries (ascending token order
   inside an expert).  Empty experts have offsets[e]==offsets[e+1]. */
void orc_moe_batch_by_expert(const int32_t* ids, const float* weights,
                             size_t rows, size_t k, size_t n_experts,
                             int32_t* offsets, int32_t* tokens, float* wts);
/* Expert closure used by dispatch_experts: in [rows x hidden] -> out. */
typedef int (*orc_expert_fn)(int expert, const float* in, size_t rows,
                             size_t hidden, float* out, void* ctx);
/* dispatch_experts (moe_fused.rs:226-308): gather rows per expert, call the
   closure, out[t] += w * expert_row in ascending expert id order. */
int orc_moe_dispatch(const float* input, size_t rows, size_t hidden,
                     size_t n_experts, const int32_t* ids, const float* weights,
                     size_t k, orc_expert_fn fn, void* ctx, float* out);
/* The quantized expert FFN the GPU path computes, in the reference's
   arithmetic (fused_ffn, moe_fused.rs:84-92 with ops::MatMul ops.rs:72-128,
   ops::Silu ops.rs:191-211 and the gate*up product moe_fused.rs:61-66):
   act = ORC_Q8_K quantizes the input rows and the gated hidden rows to Q8_K
   before each contraction (the GPU's integer path); act = ORC_F32 keeps
   everything f32 (the literal reference).  gate/up are [n_ff x hidden],
   down is [hidden x n_ff] GGUF blocks. */
int orc_moe_ffn(int gate_type, const uint8_t* const* gate,
                int up_type, const uint8_t* const* up,
                int down_type, const uint8_t* const* down,
                size_t n_experts, size_t hidden, size_t n_ff,
                const float* x, size_t rows, const int32_t* ids,
                const float* weights, size_t k, int act, float* out);

/* ---- dense FFN (models/src/transformer.rs:378-408) -------------------- */
/* The SwiGLU of feed_forward (:394-399): h = (g * (1 / (1 + expf(-g)))) * u,
   rounded in that order (h may alias g). */
void orc_ffn_swiglu(const float* g, const float* u, size_t n, float* h);
/* feed_forward of m rows: out[m x n_embd] = down(swiglu(gate x, up x)).
   act = ORC_F32: x is f32 and everything stays f32 (the literal reference);
   act = ORC_Q8_K / ORC_Q8_0: x is quantized rows (gate's and up's Q8
   partner) and h is quantized to down's partner before the down product.
   Returns 0, or -1 on a bad type/shape. */
int orc_ffn(int gate_type, const uint8_t* gate, int up_type, const uint8_t* up,
            int down_type, const uint8_t* down, size_t n_embd, size_t n_ff,
            int act, const void* x, size_t m, float* out);

/* ---- the quant crate's own Q4_K (quant/src/q4_k.rs, not GGUF) --------- */
/* Q4_K::quantize (:23-73): blocks of 256, the last may be shorter; per
   block f32 scale_min, f32 scale_max (= max - min), ceil(len/2) nibble
   bytes.  Returns the bytes written. */
size_t orc_q4_k_barq_quantize(const float* x, size_t n, uint8_t* out);
/* Q4_K::dequantize (:75-133): whole 136-byte blocks while the input lasts,
   truncated to output_size.  Returns the number of values written. */
size_t orc_q4_k_barq_dequantize(const uint8_t* in, size_t in_len, size_t output_size, float* out);

/* ---- attention (transformer.rs:176-374, context.rs:245-340) ------------ */
/* apply_rope (models/src/transformer.rs:514-562): x [seq x heads*hd] ->
   out [heads x seq x hd]; layout 0 = Interleaved (pairs 2i, 2i+1), 1 =
   SplitHalf (pairs i, i+hd/2); angle = ((float)(start+p) * freq_scale) *
   inv_freq[i]; sinf / cosf as Rust's f32::sin_cos calls them. */
void orc_rope(const float* x, size_t seq, size_t heads, size_t hd, size_t start_pos,
              float freq_scale, const float* inv_freq, int layout, float* out);
/* transpose_heads (transformer.rs:598-611): [seq x heads*hd] -> [heads x seq x hd] */
void orc_transpose_heads(const float* x, size_t seq, size_t heads, size_t hd, float* out);
/* compute_attention (transformer.rs:301-374): q [n_head x q_len x hd]; kc/vc
   hold kv head hk's positions at kc + hk*head_stride (kv_len rows of hd);
   out [q_len x n_head x hd].  Scores by gemv_f32 (sequential dot), times
   1/sqrt(hd), -inf from start_pos+i+1 on, softmax (max by fold, expf,
   sequential sum, division), then gemm_f32 of the weights with V. */
void orc_attention(const float* q, const float* kc, const float* vc, size_t head_stride,
                   size_t n_head, size_t n_head_kv, size_t hd, size_t q_len, size_t kv_len,
                   size_t start_pos, float* out);

#ifdef __cplusplus
}
#endif
#endif
