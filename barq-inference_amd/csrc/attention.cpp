// C ABI for the attention half of a transformer layer (include/barq_rocm.h):
// RoPE, head transpose, the device KV cache and attention.
//
//   apply_rope / transpose_heads   models/src/transformer.rs:514-562, 598-611
//   KVCache                        models/src/context.rs:245-340
//   compute_attention              models/src/transformer.rs:301-374
#include "../../include/barq_rocm.h"

#include <hip/hip_runtime.h>

#include <vector>

#include "api_internal.hpp"
#include "launch.hpp"

using namespace barq_api;

// Device KV cache: K and V each [n_layers][n_head_kv][max_size][head_dim] f32
// in one allocation; per-layer lengths on the host (the reference's per-layer
// vectors grow independently; size() follows layer 0).
struct barq_rocm_kv_cache {
    int device = 0;
    size_t max_size = 0, n_layers = 0, n_head_kv = 0, head_dim = 0;
    float* k = nullptr;
    float* v = nullptr;
    std::vector<size_t> len;
    size_t size = 0;

    size_t head_stride() const { return max_size * head_dim; }
    size_t layer_stride() const { return n_head_kv * head_stride(); }
};

namespace {

int check_rope_args(size_t head_dim, int layout) {
    if (head_dim == 0 || head_dim % 2 != 0) return fail(BARQ_E_DIM, "rope: head_dim=%zu must be even", head_dim);
    if (layout != BARQ_ROPE_INTERLEAVED && layout != BARQ_ROPE_SPLIT_HALF)
        return fail(BARQ_E_INVALID, "rope: layout must be BARQ_ROPE_INTERLEAVED or BARQ_ROPE_SPLIT_HALF");
    return ok();
}

int check_int_range(size_t v, const char* what) {
    if (v > (size_t)0x7fffffff) return fail(BARQ_E_DIM, "%s=%zu exceeds 2^31-1", what, v);
    return ok();
}

}  // namespace

extern "C" {

int barq_rocm_rope(barq_rocm_handle* h, const float* x, size_t seq_len, size_t n_heads, size_t head_dim,
                   size_t start_pos, float freq_scale, const float* inv_freq, int layout, float* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    BARQ_CHECK(check_rope_args(head_dim, layout));
    if (seq_len == 0 || n_heads == 0) return ok();
    if (!x || !inv_freq || !out) return fail(BARQ_E_INVALID, "rope: null buffer");
    BARQ_CHECK(check_int_range(seq_len * n_heads * head_dim, "rope: seq_len*n_heads*head_dim"));
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t n = seq_len * n_heads * head_dim;
    if (mem == BARQ_MEM_DEVICE)
        return launched(barq::rope_launch(layout, x, out, seq_len, n_heads, head_dim, start_pos, freq_scale, inv_freq,
                                          seq_len * head_dim, h->stream), "rope");
    Arena a;
    const size_t ox = a.add(n * 4), of = a.add(head_dim / 2 * 4), oo = a.add(n * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, of), inv_freq, head_dim / 2 * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::rope_launch(layout, at<float>(h, ox), at<float>(h, oo), seq_len, n_heads, head_dim,
                                          start_pos, freq_scale, at<float>(h, of), seq_len * head_dim, h->stream),
                        "rope"));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), n * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_transpose_heads(barq_rocm_handle* h, const float* x, size_t seq_len, size_t n_heads, size_t head_dim,
                              float* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (seq_len == 0 || n_heads == 0 || head_dim == 0) return ok();
    if (!x || !out) return fail(BARQ_E_INVALID, "transpose_heads: null buffer");
    BARQ_CHECK(check_int_range(seq_len * n_heads * head_dim, "transpose_heads: seq_len*n_heads*head_dim"));
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t n = seq_len * n_heads * head_dim;
    if (mem == BARQ_MEM_DEVICE)
        return launched(barq::transpose_heads_launch(x, out, seq_len, n_heads, head_dim, seq_len * head_dim, h->stream),
                        "transpose_heads");
    Arena a;
    const size_t ox = a.add(n * 4), oo = a.add(n * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::transpose_heads_launch(at<float>(h, ox), at<float>(h, oo), seq_len, n_heads, head_dim,
                                                     seq_len * head_dim, h->stream), "transpose_heads"));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), n * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

// ---------------------------------------------------------------------------
// KV cache

int barq_rocm_kv_cache_create(barq_rocm_handle* h, size_t max_size, size_t n_layers, size_t n_head_kv,
                              size_t head_dim, barq_rocm_kv_cache** out) {
    if (!out) return fail(BARQ_E_INVALID, "kv_cache_create: null output pointer");
    *out = nullptr;
    BARQ_CHECK(check_handle(h));
    if (max_size == 0 || n_layers == 0 || n_head_kv == 0 || head_dim == 0)
        return fail(BARQ_E_DIM, "kv_cache_create: max_size, n_layers, n_head_kv and head_dim must be positive");
    BARQ_CHECK(check_int_range(max_size, "kv_cache_create: max_size"));
    const size_t elems = n_layers * n_head_kv * max_size * head_dim;
    if (elems / n_layers / n_head_kv / max_size != head_dim) return fail(BARQ_E_DIM, "kv_cache_create: size overflow");
    DeviceGuard g(h);
    auto* c = new barq_rocm_kv_cache();
    c->device = h->device;
    c->max_size = max_size;
    c->n_layers = n_layers;
    c->n_head_kv = n_head_kv;
    c->head_dim = head_dim;
    c->len.assign(n_layers, 0);
    hipError_t e = hipMalloc(&c->k, elems * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&c->v, elems * sizeof(float));
    if (e != hipSuccess) {
        if (c->k) (void)hipFree(c->k);
        delete c;
        return fail(BARQ_E_ALLOC, "kv_cache_create: 2 x %zu bytes: %s", elems * sizeof(float), hipGetErrorString(e));
    }
    *out = c;
    return ok();
}

int barq_rocm_kv_cache_destroy(barq_rocm_kv_cache* c) {
    if (!c) return ok();
    DeviceGuard g(c->device);
    (void)hipDeviceSynchronize();
    if (c->k) (void)hipFree(c->k);
    if (c->v) (void)hipFree(c->v);
    delete c;
    return ok();
}

size_t barq_rocm_kv_cache_size(const barq_rocm_kv_cache* c) { return c ? c->size : 0; }

size_t barq_rocm_kv_cache_layer_len(const barq_rocm_kv_cache* c, size_t layer) {
    return (c && layer < c->n_layers) ? c->len[layer] : 0;
}

int barq_rocm_kv_cache_head(const barq_rocm_kv_cache* c, size_t layer, size_t head, const float** k, const float** v) {
    if (!c) return fail(BARQ_E_INVALID, "kv_cache_head: null cache");
    if (layer >= c->n_layers || head >= c->n_head_kv)
        return fail(BARQ_E_INVALID, "kv_cache_head: layer %zu / head %zu out of range (%zu layers, %zu heads)", layer,
                    head, c->n_layers, c->n_head_kv);
    const size_t off = layer * c->layer_stride() + head * c->head_stride();
    if (k) *k = c->k + off;
    if (v) *v = c->v + off;
    return ok();
}

int barq_rocm_kv_cache_clear(barq_rocm_kv_cache* c) {
    if (!c) return fail(BARQ_E_INVALID, "kv_cache_clear: null cache");
    for (auto& n : c->len) n = 0;
    c->size = 0;
    return ok();
}

int barq_rocm_kv_cache_append(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const float* k, const float* v,
                              size_t n_tokens, size_t head_dim, int mem) {
    BARQ_CHECK(check_mem(mem));
    BARQ_CHECK(check_handle(h));
    if (!c) return fail(BARQ_E_INVALID, "kv_cache_append: null cache");
    if (layer >= c->n_layers) return ok();   // the reference ignores such layers (context.rs:273-275)
    if (head_dim != c->head_dim)
        return fail(BARQ_E_DIM, "kv_cache_append: head_dim %zu, cache has %zu", head_dim, c->head_dim);
    if (n_tokens == 0) return ok();
    if (!k || !v) return fail(BARQ_E_INVALID, "kv_cache_append: null buffer");
    if (c->len[layer] + n_tokens > c->max_size)
        return fail(BARQ_E_INVALID, "kv_cache_append: layer %zu holds %zu of %zu positions, %zu more do not fit", layer,
                    c->len[layer], c->max_size, n_tokens);
    if (h->device != c->device) return fail(BARQ_E_INVALID, "kv_cache_append: cache is on another device");
    DeviceGuard g(h);
    const size_t row = n_tokens * head_dim * sizeof(float);
    const size_t dst_off = layer * c->layer_stride() + c->len[layer] * head_dim;
    const hipMemcpyKind kind = mem == BARQ_MEM_DEVICE ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    // head by head (context.rs:278-284): one 2-D copy of n_head_kv rows
    BARQ_HIP(hipMemcpy2DAsync(c->k + dst_off, c->head_stride() * sizeof(float), k, row, row, c->n_head_kv, kind,
                              h->stream));
    BARQ_HIP(hipMemcpy2DAsync(c->v + dst_off, c->head_stride() * sizeof(float), v, row, row, c->n_head_kv, kind,
                              h->stream));
    if (mem == BARQ_MEM_HOST) BARQ_HIP(hipStreamSynchronize(h->stream));
    c->len[layer] += n_tokens;
    if (layer == 0) c->size += n_tokens;
    return ok();
}

}  // extern "C"

namespace {

// append_rope, and with q_proj the RoPE of q into q_out ([n_head, n_tokens,
// head_dim]) in the same launch
int append_rope_any(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const float* q_proj, size_t n_head,
                    float* q_out, const float* k_proj, const float* v_proj, size_t n_tokens, size_t start_pos,
                    float freq_scale, const float* inv_freq, int layout, int mem, const char* who) {
    BARQ_CHECK(check_mem(mem));
    BARQ_CHECK(check_handle(h));
    if (!c) return fail(BARQ_E_INVALID, "%s: null cache", who);
    BARQ_CHECK(check_rope_args(c->head_dim, layout));
    if (q_proj && (!q_out || n_head == 0)) return fail(BARQ_E_INVALID, "%s: null q output or no query heads", who);
    if (n_tokens == 0) return ok();
    if (!k_proj || !v_proj || !inv_freq) return fail(BARQ_E_INVALID, "%s: null buffer", who);
    // an out-of-range layer appends nothing (the reference returns silently); q is still rotated
    const bool append = layer < c->n_layers;
    if (append && c->len[layer] + n_tokens > c->max_size)
        return fail(BARQ_E_INVALID, "%s: layer %zu holds %zu of %zu positions, %zu more do not fit", who, layer,
                    c->len[layer], c->max_size, n_tokens);
    if (!append && !q_proj) return ok();
    if (h->device != c->device) return fail(BARQ_E_INVALID, "%s: cache is on another device", who);
    const size_t hd = c->head_dim, n = n_tokens * c->n_head_kv * hd, nq = q_proj ? n_tokens * n_head * hd : 0;
    BARQ_CHECK(check_int_range(n, "kv_cache_append_rope: elements"));
    BARQ_CHECK(check_int_range(n_tokens * (n_head + 2 * c->n_head_kv) * hd, "kv_cache_append_rope: elements"));
    DeviceGuard g(h);
    const size_t dst_off = append ? layer * c->layer_stride() + c->len[layer] * hd : 0;
    const float *qp = q_proj, *kp = k_proj, *vp = v_proj, *fp = inv_freq;
    float* qo = q_out;
    if (mem == BARQ_MEM_HOST) {
        Arena a;
        const size_t ok_ = a.add(n * 4), ov = a.add(n * 4), of = a.add(hd / 2 * 4);
        const size_t oq = nq ? a.add(nq * 4) : 0, oqo = nq ? a.add(nq * 4) : 0;
        BARQ_CHECK(ensure_ws(h, a.used));
        BARQ_HIP(hipMemcpyAsync(at<float>(h, ok_), k_proj, n * 4, hipMemcpyHostToDevice, h->stream));
        BARQ_HIP(hipMemcpyAsync(at<float>(h, ov), v_proj, n * 4, hipMemcpyHostToDevice, h->stream));
        BARQ_HIP(hipMemcpyAsync(at<float>(h, of), inv_freq, hd / 2 * 4, hipMemcpyHostToDevice, h->stream));
        kp = at<float>(h, ok_);
        vp = at<float>(h, ov);
        fp = at<float>(h, of);
        if (nq) {
            BARQ_HIP(hipMemcpyAsync(at<float>(h, oq), q_proj, nq * 4, hipMemcpyHostToDevice, h->stream));
            qp = at<float>(h, oq);
            qo = at<float>(h, oqo);
        }
    }
    if (!q_proj) {
        BARQ_CHECK(launched(barq::rope_launch(layout, kp, c->k + dst_off, n_tokens, c->n_head_kv, hd, start_pos,
                                              freq_scale, fp, c->head_stride(), h->stream), "kv_cache_append_rope (k)"));
        BARQ_CHECK(launched(barq::transpose_heads_launch(vp, c->v + dst_off, n_tokens, c->n_head_kv, hd,
                                                         c->head_stride(), h->stream), "kv_cache_append_rope (v)"));
    } else if (append) {
        BARQ_CHECK(launched(barq::rope_qkv_launch(layout, qp, kp, vp, qo, c->k + dst_off, c->v + dst_off, n_tokens,
                                                  n_head, c->n_head_kv, hd, start_pos, freq_scale, fp, c->head_stride(),
                                                  h->stream), who));
    } else {
        BARQ_CHECK(launched(barq::rope_launch(layout, qp, qo, n_tokens, n_head, hd, start_pos, freq_scale, fp,
                                              n_tokens * hd, h->stream), who));
    }
    if (mem == BARQ_MEM_HOST) {
        if (nq) BARQ_HIP(hipMemcpyAsync(q_out, qo, nq * 4, hipMemcpyDeviceToHost, h->stream));
        BARQ_HIP(hipStreamSynchronize(h->stream));
    }
    if (append) {
        c->len[layer] += n_tokens;
        if (layer == 0) c->size += n_tokens;
    }
    return ok();
}

}  // namespace

extern "C" {

int barq_rocm_kv_cache_append_rope(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const float* k_proj,
                                   const float* v_proj, size_t n_tokens, size_t start_pos, float freq_scale,
                                   const float* inv_freq, int layout, int mem) {
    return append_rope_any(h, c, layer, nullptr, 0, nullptr, k_proj, v_proj, n_tokens, start_pos, freq_scale,
                           inv_freq, layout, mem, "kv_cache_append_rope");
}

int barq_rocm_kv_cache_append_rope_q(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const float* q_proj,
                                     size_t n_head, float* q_out, const float* k_proj, const float* v_proj,
                                     size_t n_tokens, size_t start_pos, float freq_scale, const float* inv_freq,
                                     int layout, int mem) {
    if (!q_proj) return fail(BARQ_E_INVALID, "kv_cache_append_rope_q: null q");
    return append_rope_any(h, c, layer, q_proj, n_head, q_out, k_proj, v_proj, n_tokens, start_pos, freq_scale,
                           inv_freq, layout, mem, "kv_cache_append_rope_q");
}

int barq_rocm_qkv_append_rope(barq_rocm_handle* h, barq_rocm_kv_cache* c, size_t layer, const int* w_types,
                              const void* const* w, size_t n_head, size_t k, int act_type, const void* x,
                              float* q_out, size_t start_pos, float freq_scale, const float* inv_freq, int layout,
                              int mem) {
    const char* who = "qkv_append_rope";
    BARQ_CHECK(check_mem(mem));
    BARQ_CHECK(check_handle(h));
    if (!c) return fail(BARQ_E_INVALID, "%s: null cache", who);
    if (!w_types || !w || !x || !q_out || !inv_freq) return fail(BARQ_E_INVALID, "%s: null buffer", who);
    for (int i = 0; i < 3; i++)
        if (!w[i]) return fail(BARQ_E_INVALID, "%s: null weight %d", who, i);
    if (n_head == 0) return fail(BARQ_E_INVALID, "%s: no query heads", who);
    BARQ_CHECK(check_rope_args(c->head_dim, layout));
    if (h->device != c->device) return fail(BARQ_E_INVALID, "%s: cache is on another device", who);
    const size_t hd = c->head_dim, nq = n_head * hd, nkv = c->n_head_kv * hd;
    BARQ_CHECK(check_int_range(nq + 2 * nkv, "qkv_append_rope: rows"));
    const bool append = layer < c->n_layers;
    if (append && c->len[layer] + 1 > c->max_size)
        return fail(BARQ_E_INVALID, "%s: layer %zu holds %zu of %zu positions, one more does not fit", who, layer,
                    c->len[layer], c->max_size);
    const size_t rows[3] = {nq, nkv, nkv};
    if (mem == BARQ_MEM_DEVICE && act_type == BARQ_TYPE_Q8_K && layout == BARQ_ROPE_INTERLEAVED && append &&
        aligned(x, 4) && aligned(q_out, 4) && barq::qkv_rope_supported(w_types, w, nq, nkv, k, hd)) {
        DeviceGuard g(h);
        const size_t dst_off = layer * c->layer_stride() + c->len[layer] * hd;
        BARQ_CHECK(launched(barq::qkv_rope_launch(w_types, w, nq, nkv, k, x, hd, q_out, c->k + dst_off, c->v + dst_off,
                                                  c->head_stride(), start_pos, freq_scale, inv_freq, h->stream),
                            who));
        c->len[layer] += 1;
        if (layer == 0) c->size += 1;
        return ok();
    }
    // the two calls the launch above fuses
    if (mem == BARQ_MEM_HOST) {
        std::vector<float> q(nq), kk(nkv), vv(nkv);
        float* ys[3] = {q.data(), kk.data(), vv.data()};
        BARQ_CHECK(barq_rocm_matvec_group(h, 3, w_types, w, rows, k, act_type, x, ys, mem));
        return append_rope_any(h, c, layer, q.data(), n_head, q_out, kk.data(), vv.data(), 1, start_pos, freq_scale,
                               inv_freq, layout, mem, who);
    }
    // device buffers: the projections go to the workspace, which the Q8_K
    // matvecs and the device append do not use themselves
    if (act_type != BARQ_TYPE_Q8_K)
        return fail(BARQ_E_UNSUPPORTED, "%s: device buffers take a Q8_K activation row (act_type %d)", who, act_type);
    Arena a;
    const size_t oq = a.add(nq * 4), ok_ = a.add(nkv * 4), ov = a.add(nkv * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    float* ys[3] = {at<float>(h, oq), at<float>(h, ok_), at<float>(h, ov)};
    BARQ_CHECK(barq_rocm_matvec_group(h, 3, w_types, w, rows, k, act_type, x, ys, mem));
    return append_rope_any(h, c, layer, ys[0], n_head, q_out, ys[1], ys[2], 1, start_pos, freq_scale, inv_freq,
                           layout, mem, who);
}

// ---------------------------------------------------------------------------
// attention

}  // extern "C"

namespace {

// attention into f32 rows (out) or Q8_K rows (out_q8)
int attention_any(barq_rocm_handle* h, const float* q, const barq_rocm_kv_cache* c, size_t layer, size_t n_head,
                  size_t n_head_kv, size_t head_dim, size_t q_len, size_t kv_len, size_t start_pos, float* out,
                  void* out_q8, int mem) {
    BARQ_CHECK(check_mem(mem));
    BARQ_CHECK(check_handle(h));
    if (!c) return fail(BARQ_E_INVALID, "attention: null cache");
    if (q_len == 0 || n_head == 0) return ok();
    if (!q || (!out && !out_q8)) return fail(BARQ_E_INVALID, "attention: null buffer");
    if (out_q8 && (n_head * head_dim) % 256 != 0)
        return fail(BARQ_E_DIM, "attention_q8k: n_head * head_dim = %zu is not a multiple of 256", n_head * head_dim);
    if (layer >= c->n_layers) return fail(BARQ_E_INVALID, "attention: layer %zu of %zu", layer, c->n_layers);
    if (n_head_kv != c->n_head_kv || head_dim != c->head_dim)
        return fail(BARQ_E_DIM, "attention: n_head_kv %zu / head_dim %zu, cache has %zu / %zu", n_head_kv, head_dim,
                    c->n_head_kv, c->head_dim);
    if (!barq::attention_supported(head_dim))
        return fail(BARQ_E_UNSUPPORTED, "attention: head_dim %zu (64, 128 or 256 supported)", head_dim);
    if (kv_len == 0 || kv_len > c->len[layer])
        return fail(BARQ_E_DIM, "attention: kv_len %zu, layer %zu holds %zu positions", kv_len, layer, c->len[layer]);
    if (h->device != c->device) return fail(BARQ_E_INVALID, "attention: cache is on another device");
    BARQ_CHECK(check_int_range(q_len, "attention: q_len"));
    BARQ_CHECK(check_int_range(start_pos + q_len, "attention: start_pos + q_len"));
    if (q_len > 65535) return fail(BARQ_E_DIM, "attention: q_len %zu above 65535", q_len);
    DeviceGuard g(h);
    const size_t nq = n_head * q_len * head_dim;
    const size_t wsp = barq::attention_workspace(n_head, head_dim, q_len, kv_len, n_head_kv);
    Arena a;
    const size_t nq8 = out_q8 ? q_len * (n_head * head_dim / 256) * 292 : 0;
    const size_t op = a.add(wsp ? wsp : 4);
    const size_t oq = mem == BARQ_MEM_HOST ? a.add(nq * 4) : 0;
    // f32 rows: the caller's, or the workspace's when they are quantized afterwards
    const size_t oo = (mem == BARQ_MEM_HOST || out_q8) ? a.add(nq * 4) : 0;
    const size_t oq8 = (mem == BARQ_MEM_HOST && out_q8) ? a.add(nq8) : 0;
    BARQ_CHECK(ensure_ws(h, a.used));
    barq::AttnArgs args{};
    args.q = q;
    args.out = out_q8 ? at<float>(h, oo) : out;
    args.out_q8 = static_cast<uint8_t*>(out_q8);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(q, 16) || (out && !aligned(out, 4)) || (out_q8 && !aligned(out_q8, 4)))
            return fail(BARQ_E_INVALID, "attention: q must be 16-byte aligned, the output 4-byte aligned");
    } else {
        BARQ_HIP(hipMemcpyAsync(at<float>(h, oq), q, nq * 4, hipMemcpyHostToDevice, h->stream));
        args.q = at<float>(h, oq);
        args.out = at<float>(h, oo);
        if (out_q8) args.out_q8 = at<uint8_t>(h, oq8);
    }
    args.k = c->k;
    args.v = c->v;
    args.layer_off = layer * c->layer_stride();
    args.head_stride = c->head_stride();
    args.n_head = n_head;
    args.n_head_kv = n_head_kv;
    args.head_dim = head_dim;
    args.q_len = q_len;
    args.kv_len = kv_len;
    args.start_pos = start_pos;
    args.part = at<float>(h, op);
    BARQ_CHECK(launched(barq::attention_launch(args, h->stream), "attention"));
    if (out_q8 && !barq::attention_q8_direct(args))
        BARQ_CHECK(launched(barq::quantize_q8_k_launch(args.out, q_len, n_head * head_dim, args.out_q8, h->stream),
                            "attention_q8k (quantize)"));
    if (mem == BARQ_MEM_HOST) {
        if (out_q8) BARQ_HIP(hipMemcpyAsync(out_q8, args.out_q8, nq8, hipMemcpyDeviceToHost, h->stream));
        else BARQ_HIP(hipMemcpyAsync(out, args.out, nq * 4, hipMemcpyDeviceToHost, h->stream));
        BARQ_HIP(hipStreamSynchronize(h->stream));
    }
    return ok();
}

}  // namespace

extern "C" {

int barq_rocm_attention(barq_rocm_handle* h, const float* q, const barq_rocm_kv_cache* c, size_t layer, size_t n_head,
                        size_t n_head_kv, size_t head_dim, size_t q_len, size_t kv_len, size_t start_pos, float* out,
                        int mem) {
    if (!out && q_len && n_head) return fail(BARQ_E_INVALID, "attention: null buffer");
    return attention_any(h, q, c, layer, n_head, n_head_kv, head_dim, q_len, kv_len, start_pos, out, nullptr, mem);
}

int barq_rocm_attention_q8k(barq_rocm_handle* h, const float* q, const barq_rocm_kv_cache* c, size_t layer,
                            size_t n_head, size_t n_head_kv, size_t head_dim, size_t q_len, size_t kv_len,
                            size_t start_pos, void* out_q8k, int mem) {
    if (!out_q8k && q_len && n_head) return fail(BARQ_E_INVALID, "attention_q8k: null buffer");
    return attention_any(h, q, c, layer, n_head, n_head_kv, head_dim, q_len, kv_len, start_pos, nullptr, out_q8k,
                         mem);
}


}  // extern "C"
