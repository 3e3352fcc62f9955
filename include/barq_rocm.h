/*
 * barq_rocm.h — C ABI of the MI355X (gfx950) quantized-linear backend.
 *
 * This is the drop-in boundary for barq-inference's quantized-linear hot
 * path: GGUF block-quant dequantize-and-dot for Q4_0, Q8_0, Q4_K and Q6_K
 * (batch-1 GEMV, batched int8-MFMA GEMM, ragged MoE expert GEMM).  The
 * reference is Rust and has no FFI on this path; every entry point below
 * names the Rust interface it replaces, so a `backend` crate arm (or a
 * `BackendPreference::Rocm` in barq_core/src/blas.rs:20-42) can bind it with
 * an `extern "C"` block and a build.rs that runs hipcc.
 *
 * Conventions
 *  - Every function returns a barq_status; 0 is success.  The message of the
 *    last failure on the calling thread is barq_rocm_last_error().
 *  - Buffers are owned by the caller.  `mem` says where they live:
 *      BARQ_MEM_DEVICE — device pointers; the call is enqueued on the
 *        handle's stream and returns without waiting (stream order).
 *      BARQ_MEM_HOST   — host pointers; the call copies in, computes, copies
 *        out and waits (the reference's QuantizedCudaOps round trip,
 *        backend/src/cuda_quant.rs:311-338, but with the compute on device).
 *  - A handle is used by one thread at a time; distinct handles may be used
 *    concurrently (blas::gemm_f32 is called from rayon workers,
 *    models/src/transformer.rs:315-331).
 *  - Weights are GGUF row-major: n_rows rows of k elements, blocks along k
 *    (gguf.rs:415-519 element order).  y = W x, i.e. y[n] = sum_k W[n,k] x[k],
 *    which is blas::gemv_f32(dequant(W), x) (blas.rs:229-304) and the rows of
 *    blas::gemm_f32(x, W^T) (blas.rs:103-213, W^T built by
 *    models/src/weight_cache.rs:172-210).
 */
#ifndef BARQ_ROCM_H
#define BARQ_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BARQ_ROCM_ABI_VERSION 1

/* Status codes: barq_core::error::Error variants (barq_core/src/error.rs:9-57) */
typedef enum {
    BARQ_OK = 0,
    BARQ_E_BACKEND = 1,      /* Error::Backend (error.rs:48): HIP runtime failure */
    BARQ_E_UNSUPPORTED = 2,  /* Error::Unsupported (error.rs:55): no device, type or shape not supported */
    BARQ_E_DIM = 3,          /* Error::DimensionMismatch (error.rs:27) */
    BARQ_E_QUANT = 4,        /* Error::Quantization (error.rs:44): k not a whole number of blocks */
    BARQ_E_INVALID = 5,      /* Error::Tensor (error.rs:11): null pointer or bad argument */
    BARQ_E_ALLOC = 6,        /* Error::Allocation (error.rs:15) */
    BARQ_E_GGUF = 7,         /* Error::InvalidGguf (error.rs:39-40): malformed GGUF file */
    BARQ_E_IO = 8            /* Error::Io (error.rs:31): file cannot be read, or ends early */
} barq_status;

/* Type ids: the GgufTensorType discriminants (barq_core/src/gguf.rs:117-137),
   plus the reference's own 20-byte Q4_0 layout (gguf.rs:521-578,
   quant/src/q4_0.rs:23-115), which differs from GGUF's 18-byte block_q4_0. */
typedef enum {
    BARQ_TYPE_F32 = 0,
    BARQ_TYPE_F16 = 1,
    BARQ_TYPE_Q4_0 = 2,        /* f16 d + 16 B; elem i<16 low nibble of byte i, else high of byte i-16; (nib-8)*d */
    BARQ_TYPE_Q8_0 = 8,        /* f16 d + 32 x i8 */
    BARQ_TYPE_Q4_K = 12,       /* f16 d, f16 dmin, 12 B 6-bit scales/mins, 128 B nibbles; 256 elems */
    BARQ_TYPE_Q6_K = 14,       /* 128 B ql, 64 B qh, 16 x i8 scales, f16 d; 256 elems */
    BARQ_TYPE_Q8_K = 15,       /* f32 d, 256 x i8, 16 x i16 bsums (activations) */
    BARQ_TYPE_Q4_0_BARQ = 0x10002, /* f32 scale + 16 B; elem i in byte i/2 (low if even), sign-extended */
    BARQ_TYPE_Q4_K_BARQ = 0x1000C  /* the quant crate's own Q4_K (quant/src/q4_k.rs:7-133, not GGUF):
                                      f32 min, f32 range, 128 B nibbles (low first); 136 B per 256 */
} barq_type;

/* Activation mode for matvec/matmul.  BARQ_ACT_F32 keeps x in f32 and
   dequantizes W in registers: the literal reference arithmetic.  Passing
   BARQ_TYPE_Q8_0 / BARQ_TYPE_Q8_K means x is already-quantized blocks (from
   barq_rocm_quantize_act) and the product runs on integer dot/MFMA units.
   BARQ_ACT_F32_Q8 means x is f32 and the library quantizes it to the
   weight type's Q8 partner (Q8_0 for Q4_0/Q8_0/Q4_0_BARQ, Q8_K for
   Q4_K/Q6_K) in its workspace first. */
#define BARQ_ACT_F32 0
#define BARQ_ACT_F32_Q8 0x20000

typedef enum { BARQ_MEM_HOST = 0, BARQ_MEM_DEVICE = 1 } barq_mem;

typedef struct barq_rocm_handle barq_rocm_handle;

/* ---- lifecycle ---------------------------------------------------------
 * Replaces CudaBackend::new(device_id) (backend/src/cuda.rs:60-155) and
 * QuantizedCudaOps::new (backend/src/cuda_quant.rs:217-238).  A missing or
 * unusable device returns BARQ_E_UNSUPPORTED, as cuda.rs:64-77 maps a failed
 * CudaDevice::new to Error::Unsupported, so callers fall back to the CPU
 * chain of blas.rs:134-212.  The handle owns a HIP stream and a workspace. */
int barq_rocm_create(int device, barq_rocm_handle** out);
int barq_rocm_destroy(barq_rocm_handle* h);
/* Message of the last failure on this thread ("" if none). */
const char* barq_rocm_last_error(void);
/* Use an external hipStream_t for subsequent calls (NULL: the handle's own). */
int barq_rocm_set_stream(barq_rocm_handle* h, void* hip_stream);
void* barq_rocm_get_stream(barq_rocm_handle* h);
int barq_rocm_synchronize(barq_rocm_handle* h);
/* ABI version of the loaded library (BARQ_ROCM_ABI_VERSION). */
int barq_rocm_abi_version(void);

/* ---- block geometry ----------------------------------------------------
 * GgufTensorType::block_size (gguf.rs:168-186) and the per-type block byte
 * sizes of gguf.rs:529-530,645,747,854.  0 for an unknown type. */
size_t barq_rocm_block_elems(int type);
size_t barq_rocm_block_bytes(int type);
/* Bytes of one row of k elements (0 if k is not a whole number of blocks). */
size_t barq_rocm_row_bytes(int type, size_t k);

/* ---- dequantize --------------------------------------------------------
 * Replaces the per-type decoders behind GgufReader::load_tensor
 * (gguf.rs:437-519): load_q4_0 :521-578 (BARQ_TYPE_Q4_0_BARQ; GGUF Q4_0 is
 * BARQ_TYPE_Q4_0), load_q8_0 :634-681, load_q4_k :730-837, load_q6_k
 * :839-914, plus F16 :456-469 and the Q8_K activation blocks.  Output is
 * bit-identical to those decoders.  n_elems must be a whole number of blocks. */
int barq_rocm_dequantize(barq_rocm_handle* h, int type, const void* blocks,
                         size_t n_elems, float* out, int mem);

/* get_embeddings (models/src/transformer.rs:96-119): out row t (k f32) is
 * row tokens[t] of the n_rows x k table (any type barq_rocm_dequantize
 * takes, or BARQ_TYPE_F32; token_embd.weight as the weight cache holds it),
 * decoded bit-identically to dequantizing the whole table; an id outside
 * [0, n_rows) gives a zero row (the reference skips it and leaves its
 * zero-initialised row).  k a multiple of 4 and of the block size; device
 * table aligned as the type's weights (F32 16-byte), out 16-byte.  With
 * host buffers only the named rows are copied to the device. */
int barq_rocm_get_rows(barq_rocm_handle* h, int type, const void* table, size_t n_rows, size_t k,
                       const int32_t* tokens, size_t n_tokens, float* out, int mem);

/* ---- activation quantize -----------------------------------------------
 * No reference counterpart: Q8_K is only an id (gguf.rs:132, quant.rs:29).
 * Implements llama.cpp's block_q8_0 (d = amax/127 stored f16,
 * q = roundf(x/d)) and block_q8_K (iscale = -127/max, q = min(127,
 * rint(iscale*x)), d = 1/iscale, bsums of 16) for n_rows rows of k. */
int barq_rocm_quantize_act(barq_rocm_handle* h, int act_type, const float* x,
                           size_t n_rows, size_t k, void* out_blocks, int mem);

/* ---- RMSNorm -------------------------------------------------------------
 * Replaces LlamaTransformer::rms_norm (models/src/transformer.rs:148-172),
 * the step before every projection (:132, :139, :469): per row of n,
 * y = (x * (1 / sqrt(sum(x^2) / n + max(eps, FLT_EPSILON)))) * weight.
 * The sum of squares runs in a fixed tree order (the reference sums
 * sequentially): results agree with the reference to float rounding.
 * n % 4 == 0, n <= 16384; x, weight, y 16-byte aligned on the device. */
int barq_rocm_rms_norm(barq_rocm_handle* h, const float* x, const float* weight,
                       size_t rows, size_t n, float eps, float* y, int mem);

/* RMSNorm fused with the activation quantizer of the next projection:
 * writes act_type (BARQ_TYPE_Q8_K or BARQ_TYPE_Q8_0) blocks of the
 * normalized rows without storing them in f32.  Byte-identical to
 * barq_rocm_quantize_act(act_type, barq_rocm_rms_norm(x)).  The reference
 * has no fused form (its projections take f32, transformer.rs:274).
 * n % 256 == 0, n <= 16384. */
int barq_rocm_rms_norm_quantize(barq_rocm_handle* h, int act_type, const float* x,
                                const float* weight, size_t rows, size_t n, float eps,
                                void* out_blocks, int mem);

/* The residual add of forward_layer (add_vectors, transformer.rs:505-510,
 * at :136 and :143) fused with the RMSNorm of the next sub-layer and its
 * quantizer: per row, s = x + d (d may be NULL: s = x), stored to sum when
 * sum is not NULL (sum needs d), then out = rms_norm(s) as out_type
 * (BARQ_TYPE_F32 rows, or Q8_K / Q8_0 blocks as barq_rocm_rms_norm_quantize
 * writes them).  A decode layer runs it twice: x + attention output with
 * ffn_norm, then (as the next layer's first call) x + FFN output with
 * attn_norm.  n % 4 == 0 (F32) or n % 256 == 0 (Q8), n <= 16384. */
int barq_rocm_add_rms_norm_quantize(barq_rocm_handle* h, int out_type, const float* x,
                                    const float* d, const float* weight, size_t rows, size_t n,
                                    float eps, float* sum, void* out, int mem);

/* LlamaTransformer::add_bias (transformer.rs:444-465; the q/k/v biases at
 * :206-220) and final_output's output.bias (:487-495): y[r, j] += bias[j]
 * for rows x dim, in place, one f32 addition per element (bit-identical).
 * The reference applies a bias only when its length equals dim; the caller
 * makes that check. */
int barq_rocm_add_bias(barq_rocm_handle* h, float* y, const float* bias, size_t rows, size_t dim, int mem);

/* ---- matvec / matmul ---------------------------------------------------
 * Replace blas::gemv_f32 (blas.rs:229-304; the output head,
 * transformer.rs:486) and blas::gemm_f32 (blas.rs:103-213; every
 * projection, transformer.rs:274,423) when the weight is kept packed instead
 * of dequantized at load (gguf.rs:437-475) and transposed
 * (weight_cache.rs:172-210).
 *   matvec: y[n_rows] = W x.
 *   matmul: Y[m x n_rows] (row-major) = X W^T, X is m rows of k (f32 or Q8
 *           blocks per row) — gemm_f32(X, W^T, m, k, n_rows).
 * m = 2..4 runs one GEMV over all rows (weights read once); from m = 5
 * (or where that GEMV's layout conditions fail, from m = 3, or 4 for
 * Q4_0 / Q4_0_BARQ) matmul runs the LDS-staged int8-MFMA kernel instead of
 * one GEMV per row; it may use the
 * handle's workspace (repacked Q8_0 rows, K-slice partial products), which
 * grows on the first call that needs more. */
int barq_rocm_matvec(barq_rocm_handle* h, int w_type, const void* w,
                     size_t n_rows, size_t k, int act_type, const void* x,
                     float* y, int mem);
int barq_rocm_matmul(barq_rocm_handle* h, int w_type, const void* w,
                     size_t n_rows, size_t k, int act_type, const void* x,
                     size_t m, float* y, int mem);

/* matvec_group = n_mats matvecs of one activation row (the q, k and v
 * projections of LlamaTransformer::self_attention, transformer.rs:212-220,
 * all read the same normalized x): y[i] = W[i] . x for i < n_mats, each
 * within barq_rocm_matvec's bar.  On device buffers with a Q8_K row,
 * k <= 4096, Q4_K matrices and optionally a last Q6_K one (2 to 4
 * matrices), all of them run in one launch of the register GEMV (each
 * output bit-identical to that GEMV on its matrix alone; a Q6_K matvec on
 * its own takes the LDS-streamed GEMV, whose summation order differs);
 * any other case runs the matvecs one after another. */
int barq_rocm_matvec_group(barq_rocm_handle* h, size_t n_mats, const int* w_types, const void* const* w,
                           const size_t* n_rows, size_t k, int act_type, const void* x, float* const* y,
                           int mem);

/* ---- dense FFN ------------------------------------------------------------
 * swiglu: the SwiGLU of LlamaTransformer::feed_forward
 *   (models/src/transformer.rs:394-399), h = (g * (1 / (1 + exp(-g)))) * u
 *   with each operation rounded as written (the MoE expert FFN rounds
 *   silu(g) = g / (1 + exp(-g)) instead, ops.rs:191-211), over rows x n of
 *   gate/up f32.  out_type BARQ_TYPE_F32 writes f32 h; BARQ_TYPE_Q8_K /
 *   BARQ_TYPE_Q8_0 write h's activation blocks for the down projection
 *   (byte-identical to barq_rocm_quantize_act of the f32 h) without storing
 *   it.  exp is the device's expf: h agrees with the reference to a few ulp.
 * ffn: feed_forward (transformer.rs:378-408) of m rows of x [m x n_embd]:
 *   out = down(swiglu(gate(x), up(x))); gate/up are [n_ff x n_embd], down
 *   [n_embd x n_ff] GGUF weights (proj_with_in_dim, :411-442).  act:
 *   BARQ_ACT_F32 the literal f32 arithmetic; BARQ_ACT_F32_Q8 x f32,
 *   quantized here to gate's Q8 partner and h to down's; BARQ_TYPE_Q8_K /
 *   BARQ_TYPE_Q8_0 x already quantized (e.g. by barq_rocm_rms_norm_quantize).
 *   One row with Q4_K gate and up runs both projections in one launch with
 *   the SwiGLU in its epilogue.  Uses the handle's workspace. */
int barq_rocm_swiglu(barq_rocm_handle* h, int out_type, const float* gate, const float* up,
                     size_t rows, size_t n, void* out, int mem);
int barq_rocm_ffn(barq_rocm_handle* h, int gate_type, const void* gate, int up_type,
                  const void* up, int down_type, const void* down, size_t n_embd,
                  size_t n_ff, int act, const void* x, size_t m, float* out, int mem);

/* ---- f32 BLAS ----------------------------------------------------------
 * Device arms of blas::gemm_f32 (blas.rs:103-213: C[m x n] = A[m x k]
 * B[k x n], row-major) and blas::gemv_f32 (blas.rs:229-304: y = A[m x n] x),
 * for callers that keep f32 weights. */
int barq_rocm_gemm_f32(barq_rocm_handle* h, const float* a, const float* b,
                       size_t m, size_t k, size_t n, float* c, int mem);
int barq_rocm_gemv_f32(barq_rocm_handle* h, const float* a, const float* x,
                       size_t m, size_t n, float* y, int mem);

/* ---- the reference's split-scale quantized operator API ----------------
 * QuantizedCudaOps (backend/src/cuda_quant.rs:192-338) keeps quants and f32
 * scales in separate buffers.  kind == BARQ_TYPE_Q8_0 decodes signed bytes
 * (dequantize_signed_8bit_host :77-102); any other kind decodes packed
 * sign-extended nibbles (dequantize_packed_4bit_host :44-75), which is what
 * the reference's dequantize_q4k/q5k do.  block_size is elements per scale
 * (the reference passes recommended_block_size(), cuda.rs:228-230, for
 * dequantize_* and QuantizedGemmConfig::block_size, :128-150, for matmul).
 * quantized_matmul: C[m x n] = A[m x k] B, B = [k x n] decoded along its
 * flat row-major index (quantized_matmul_host :104-126). */
int barq_rocm_dequantize_split(barq_rocm_handle* h, int kind,
                               const uint8_t* quants, size_t n_quants,
                               const float* scales, size_t n_scales,
                               size_t block_size, float* out, size_t n_out,
                               int mem);
int barq_rocm_quantized_matmul_split(barq_rocm_handle* h, const float* a,
                                     const uint8_t* b_quantized, size_t n_bq,
                                     const float* b_scales, size_t n_bscales,
                                     float* c, size_t m, size_t n, size_t k,
                                     int kind, size_t block_size, int mem);

/* quant::Q4_0::quantize (quant/src/q4_0.rs:23-67): f32 -> 20-byte
 * BARQ_TYPE_Q4_0_BARQ blocks, bit-identical.  n must be a multiple of 32. */
int barq_rocm_quantize_q4_0_barq(barq_rocm_handle* h, const float* x, size_t n,
                                 uint8_t* out, int mem);

/* quant::Q4_K (quant/src/q4_k.rs:7-133), the quant crate's own 4-bit format
 * (never produced by the GGUF loader): quantize = Q4_K::quantize (:23-73):
 * per block of 256 (the last may be shorter) f32 scale_min = min, f32
 * scale_max = max - min, q = clamp(round((x - min) / scale_max * 15), 0, 15)
 * (7.5 rounded when scale_max is 0), two per byte low nibble first; a block
 * of len elements is 8 + ceil(len/2) bytes (barq_rocm_q4_k_barq_bytes(n)
 * for n elements).  Dequantize with barq_rocm_dequantize(BARQ_TYPE_Q4_K_BARQ)
 * = Q4_K::dequantize (:75-133) on whole 136-byte blocks:
 * y = scale_min + (q / 15) * scale_max. */
size_t barq_rocm_q4_k_barq_bytes(size_t n);
int barq_rocm_quantize_q4_k_barq(barq_rocm_handle* h, const float* x, size_t n, uint8_t* out, int mem);

/* ---- fused MoE ---------------------------------------------------------
 * MoEFusedOps (models/src/moe_fused.rs:41-309).
 * route: select_top_k_experts (:95-144) — per row, the top_k logits
 *   (descending, stable), softmax over the kept k; ids/weights are
 *   rows x top_k.
 * ffn: dispatch_experts (:226-308) with fused_ffn (:84-92) as every expert:
 *   out[t] = sum over t's experts e, ascending e, of
 *   w[t,e] * ( (silu(x_t G_e^T) * (x_t U_e^T)) D_e^T ).
 *   gate/up are [n_ff x hidden], down is [hidden x n_ff] GGUF weights; the
 *   three arrays hold n_experts pointers (host arrays of `mem` pointers).
 *   act = BARQ_ACT_F32_Q8 runs the integer path (rows and the gated hidden
 *   quantized to Q8_K); act = BARQ_ACT_F32 keeps f32 activations. */
int barq_rocm_moe_route(barq_rocm_handle* h, const float* logits, size_t rows,
                        size_t n_experts, size_t top_k, int32_t* ids,
                        float* weights, int mem);
/* reduce: reduce_expert_assignments (moe_fused.rs:147-194), the smart expert
 *   reduction MoEInference::forward_with_routing runs between routing and
 *   dispatch (advanced/src/moe.rs:157-162, ser_threshold 0.05 and
 *   max_active = n_expert_per_token by default, :24-31).  Per row of top_k
 *   slots (id < 0: an absent slot): keep the assignments with weight >=
 *   min_weight (if none, the largest; the later slot wins ties), sort them by
 *   weight descending (stable), keep at most max(max_active, 1), divide by
 *   their sequential f32 sum floored at f32::EPSILON.  Kept assignments come
 *   first; the rest of the row gets id -1 and weight 0, which moe_ffn skips.
 *   out_ids / out_weights may be ids / weights.
 * route_reduce: route then reduce in one launch; ids/weights rows x
 *   clamp(top_k, 1, n_experts). */
int barq_rocm_moe_reduce(barq_rocm_handle* h, const int32_t* ids, const float* weights,
                         size_t rows, size_t top_k, size_t max_active, float min_weight,
                         int32_t* out_ids, float* out_weights, int mem);
int barq_rocm_moe_route_reduce(barq_rocm_handle* h, const float* logits, size_t rows,
                               size_t n_experts, size_t top_k, size_t max_active,
                               float min_weight, int32_t* ids, float* weights, int mem);
int barq_rocm_moe_ffn(barq_rocm_handle* h, size_t n_experts,
                      int gate_type, const void* const* gate,
                      int up_type, const void* const* up,
                      int down_type, const void* const* down,
                      size_t hidden, size_t n_ff, const float* x, size_t rows,
                      const int32_t* ids, const float* weights, size_t top_k,
                      int act, float* out, int mem);

/* ---- GGUF files: packed loader ------------------------------------------
 * Replaces GgufReader::open / tensor_info / get / get_tensor_info
 * (barq_core/src/gguf.rs:250-413).  The file is memory-mapped and read with
 * the reference's rules: magic "GGUF", version <= 3, u64 counts, KV values
 * of the 13 GgufType kinds (arrays nest), general.alignment when it is a
 * u32 (default 32), tensor infos, data section aligned after them.  A
 * tensor is handed out as its packed bytes at data_offset + offset (where
 * load_tensor seeks, gguf.rs:428-431) instead of being dequantized at load
 * (:437-475).  GGUF type 2 is the 18-byte GGUF Q4_0 block (BARQ_TYPE_Q4_0).
 * Errors: BARQ_E_GGUF for malformed content (bad magic, version, value or
 * tensor type, non-UTF-8 string), BARQ_E_IO when the file ends early. */
typedef struct barq_rocm_gguf barq_rocm_gguf;

int barq_rocm_gguf_open(const char* path, barq_rocm_gguf** out);
int barq_rocm_gguf_close(barq_rocm_gguf* g);
int barq_rocm_gguf_info(const barq_rocm_gguf* g, uint32_t* version, uint64_t* n_tensors,
                        uint64_t* n_kv, uint32_t* alignment, uint64_t* data_offset);
/* Tensor `index` in file order: name (owned by g), GGUF type id, dims
 * (dims[0] innermost; up to 4, more fold into dims[3]), offset in the data
 * section, packed size (0 for types whose block layout is not known here,
 * as the reference cannot load them either), and a host pointer to the bytes
 * inside the mapping (BARQ_E_IO if they run past the end of the file). */
int barq_rocm_gguf_tensor(const barq_rocm_gguf* g, uint64_t index, const char** name, int* type,
                          uint32_t* n_dims, uint64_t* dims, uint64_t* offset, uint64_t* nbytes,
                          const void** data);
int barq_rocm_gguf_find_tensor(const barq_rocm_gguf* g, const char* name, uint64_t* index);
/* KV access (GgufReader::get, gguf.rs:390): value type (GgufType id) and,
 * for arrays, element type and length; scalars as int64 or double; strings
 * as a pointer into the mapping and a length (not NUL-terminated). */
int barq_rocm_gguf_kv_type(const barq_rocm_gguf* g, const char* key, int* type, int* array_type,
                           uint64_t* array_len);
int barq_rocm_gguf_kv_int(const barq_rocm_gguf* g, const char* key, int64_t* value);
int barq_rocm_gguf_kv_number(const barq_rocm_gguf* g, const char* key, double* value);
int barq_rocm_gguf_kv_string(const barq_rocm_gguf* g, const char* key, const char** ptr, uint64_t* len);

/* ---- packed weight cache --------------------------------------------------
 * Replaces WeightCache::initialize / build_transposed_entry / get_proj /
 * get_raw (models/src/weight_cache.rs:48-244) without the dequantize and
 * transpose: every sized tensor of the file is copied once, packed, into
 * one device allocation on the handle's device (256-byte aligned each).
 * cache_get returns the device pointer for barq_rocm_matvec / matmul /
 * moe_ffn, with k = dims[0] and n_rows = dims[1] * dims[2] * dims[3].
 * The cache allocates at creation only and frees at destroy. */
typedef struct barq_rocm_cache barq_rocm_cache;

int barq_rocm_cache_create(barq_rocm_handle* h, const barq_rocm_gguf* g, barq_rocm_cache** out);
int barq_rocm_cache_get(const barq_rocm_cache* c, const char* name, int* type, uint64_t* n_rows,
                        uint64_t* k, const void** device_ptr);
uint64_t barq_rocm_cache_bytes(const barq_rocm_cache* c);
int barq_rocm_cache_destroy(barq_rocm_cache* c);

/* ---- attention: RoPE, KV cache, attention ---------------------------------
 * The attention half of LlamaTransformer::self_attention
 * (models/src/transformer.rs:176-265) with f32 tensors, as the reference
 * computes it.  Heads and positions use the reference's layouts:
 *   projections x:  [seq_len, n_heads * head_dim]
 *   RoPE'd q / k, transposed v: [n_heads, seq_len, head_dim]
 *   attention out:  [q_len, n_head, head_dim]
 *
 * barq_rocm_rope = apply_rope (transformer.rs:514-562): pair i of position p
 * of every head is rotated by angle = ((float)(start_pos + p) * freq_scale)
 * * inv_freq[i]; inv_freq has head_dim / 2 entries (the caller's
 * rope_inv_freq, transformer.rs:52-54) and lives where `mem` says.  layout:
 * BARQ_ROPE_INTERLEAVED pairs (2i, 2i+1), BARQ_ROPE_SPLIT_HALF pairs
 * (i, i + head_dim/2) (RopeLayout, :570-595).  sin/cos are the device's
 * sincosf, so results agree with the reference's to a few ulp.
 * barq_rocm_transpose_heads = transpose_heads (:598-611). */
#define BARQ_ROPE_INTERLEAVED 0
#define BARQ_ROPE_SPLIT_HALF 1
int barq_rocm_rope(barq_rocm_handle* h, const float* x, size_t seq_len, size_t n_heads, size_t head_dim,
                   size_t start_pos, float freq_scale, const float* inv_freq, int layout, float* out, int mem);
int barq_rocm_transpose_heads(barq_rocm_handle* h, const float* x, size_t seq_len, size_t n_heads,
                              size_t head_dim, float* out, int mem);

/* KV cache = KVCache (models/src/context.rs:245-340): per layer and kv head,
 * positions x head_dim f32, contiguous per head.  Preallocated in device
 * memory for max_size positions (KVCache::new's max_size, :260).
 * append = KVCache::append (:272-291): k and v are [n_head_kv, n_tokens,
 * head_dim]; they go after the layer's current length; an out-of-range
 * layer is ignored (returns BARQ_OK, as the reference returns silently); a
 * layer 0 append advances size (:287-289).  Unlike the reference's growing
 * vectors, appending past max_size fails with BARQ_E_INVALID.
 * append_rope fuses apply_rope on k and transpose_heads on v into the
 * append: k_proj and v_proj are the projections [n_tokens, n_head_kv *
 * head_dim] (transformer.rs:222-245).
 * head = get_k_head / get_v_head (:316-323): device pointers to the layer's
 * positions of kv head `head` (len(layer) rows of head_dim). */
typedef struct barq_rocm_kv_cache barq_rocm_kv_cache;
int barq_rocm_kv_cache_create(barq_rocm_handle* h, size_t max_size, size_t n_layers, size_t n_head_kv,
                              size_t head_dim, barq_rocm_kv_cache** out);
int barq_rocm_kv_cache_append(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const float* k,
                              const float* v, size_t n_tokens, size_t head_dim, int mem);
int barq_rocm_kv_cache_append_rope(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer,
                                   const float* k_proj, const float* v_proj, size_t n_tokens,
                                   size_t start_pos, float freq_scale, const float* inv_freq, int layout,
                                   int mem);
/* append_rope_q = the three steps of self_attention between the projections
 * and compute_attention (transformer.rs:222-245: apply_rope on q, apply_rope
 * on k and transpose_heads on v, then KVCache::append) in one launch:
 * q_proj [n_tokens, n_head * head_dim] is rotated into q_out [n_head,
 * n_tokens, head_dim]; k_proj and v_proj go into the cache as for
 * append_rope.  The same bits as barq_rocm_rope on q followed by
 * barq_rocm_kv_cache_append_rope.  An out-of-range layer appends nothing and
 * still rotates q. */
int barq_rocm_kv_cache_append_rope_q(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer,
                                     const float* q_proj, size_t n_head, float* q_out, const float* k_proj,
                                     const float* v_proj, size_t n_tokens, size_t start_pos, float freq_scale,
                                     const float* inv_freq, int layout, int mem);
/* qkv_append_rope = self_attention from the normalized row to the cache for
 * ONE token (transformer.rs:212-245): the q, k and v projections of x (one
 * activation row of act_type; w_types[3] / w[3] are W_q [n_head * head_dim
 * rows], W_k and W_v [n_head_kv * head_dim rows], k columns), apply_rope on
 * q into q_out [n_head, 1, head_dim], apply_rope on k and v appended to the
 * cache at layer `layer`.  The same bits as barq_rocm_matvec_group followed
 * by barq_rocm_kv_cache_append_rope_q (n_tokens = 1).  On device buffers
 * with a Q8_K row, Q4_K W_q and W_k, a Q4_K or Q6_K W_v, k <= 4096 and the
 * interleaved layout it is one launch (each wave rotates its own rotary
 * pair and writes the cache); otherwise those two calls run (device buffers
 * then need act_type BARQ_TYPE_Q8_K).  An out-of-range layer appends
 * nothing and still writes q_out. */
int barq_rocm_qkv_append_rope(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const int* w_types,
                              const void* const* w, size_t n_head, size_t k, int act_type, const void* x,
                              float* q_out, size_t start_pos, float freq_scale, const float* inv_freq, int layout,
                              int mem);
size_t barq_rocm_kv_cache_size(const barq_rocm_kv_cache* c);
size_t barq_rocm_kv_cache_layer_len(const barq_rocm_kv_cache* c, size_t layer);
int barq_rocm_kv_cache_head(const barq_rocm_kv_cache* c, size_t layer, size_t head, const float** k,
                            const float** v);
int barq_rocm_kv_cache_clear(barq_rocm_kv_cache* c);
int barq_rocm_kv_cache_destroy(barq_rocm_kv_cache* c);

/* Attention = LlamaTransformer::compute_attention (transformer.rs:301-374):
 * q is [n_head, q_len, head_dim] (mem), K/V are the cache's layer; query
 * head h reads kv head h * n_head_kv / n_head; query i sees positions
 * j < min(kv_len, start_pos + i + 1) with weights softmax((q . K[j]) /
 * sqrt(head_dim)); out[i, h, :] = sum_j p_j V[j, :].  kv_len must be at most
 * the layer's length; head_dim 64, 128 or 256 (else BARQ_E_UNSUPPORTED).
 * n_head_kv and head_dim must be the cache's.  Uses the handle's workspace
 * for the partial results of long sequences. */
int barq_rocm_attention(barq_rocm_handle* h, const float* q, const barq_rocm_kv_cache* c, size_t layer,
                        size_t n_head, size_t n_head_kv, size_t head_dim, size_t q_len, size_t kv_len,
                        size_t start_pos, float* out, int mem);
/* attention_q8k = compute_attention followed by the o projection's activation
 * quantizer (transformer.rs:255-262: the attention rows are the input of
 * proj(wo)): out_q8k receives q_len rows of n_head * head_dim / 256 Q8_K
 * blocks (n_head * head_dim must be a multiple of 256), the bytes
 * barq_rocm_quantize_act(BARQ_Q8_K) writes for barq_rocm_attention's rows.
 * When the positions are split over workgroups the merge kernel writes the
 * blocks itself (one launch fewer). */
int barq_rocm_attention_q8k(barq_rocm_handle* h, const float* q, const barq_rocm_kv_cache* c, size_t layer,
                            size_t n_head, size_t n_head_kv, size_t head_dim, size_t q_len, size_t kv_len,
                            size_t start_pos, void* out_q8k, int mem);

/* ---- measurement ------------------------------------------------------------
 * No counterpart in the reference.  Reads bytes (rounded down to 16) at the
 * device pointer p once, with coalesced non-temporal loads and nothing else:
 * the HBM streaming floor a GEMV over the same bytes is measured against
 * (bench.py times it in the same graph, on the same stream, as the GEMV).
 * sink: a device word written only when the XOR of all the data equals a
 * fixed constant.  p 16-byte aligned. */
int barq_rocm_stream_read(barq_rocm_handle* h, const void* p, size_t bytes, uint32_t* sink);

/* ---- matmul without allocation -------------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc.  Same product, dispatch and results as barq_rocm_matmul with
 * mem = BARQ_MEM_DEVICE (all buffers are device pointers), but its scratch
 * (activation rows quantized in the call for BARQ_ACT_F32_Q8, the
 * 32-element-block GEMM's repacked rows, K-slice partial products, the
 * literal f32 path's dequantized weights) is a fixed array of
 * BARQ_NOALLOC_SCRATCH_BYTES per GPU, set up by barq_rocm_create, instead of
 * the handle's growable workspace.  A call that needs more scratch fails
 * with BARQ_E_UNSUPPORTED before anything is enqueued.  Calls allocate
 * nothing.  Every no-allocation call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (other streams, other handles, other
 * threads) race on it and must be ordered by the caller. */
#define BARQ_NOALLOC_SCRATCH_BYTES (32u << 20)
int barq_rocm_matmul_noalloc(barq_rocm_handle* h, int w_type, const void* w,
                             size_t n_rows, size_t k, int act_type, const void* x,
                             size_t m, float* y);

#ifdef __cplusplus
}
#endif
#endif /* BARQ_ROCM_H */
