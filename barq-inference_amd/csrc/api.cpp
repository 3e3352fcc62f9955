// C ABI of libbarq_rocm (include/barq_rocm.h): argument checking, memory
// staging for host buffers, workspace management and kernel dispatch.
#include "../../include/barq_rocm.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "api_internal.hpp"
#include "launch.hpp"

namespace {
thread_local std::string g_last_error;
}

int barq_api::fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

namespace {

using barq_api::DeviceGuard;
using barq_api::fail;
using barq_api::ok;

bool is_weight_type(int t) {
    return t == BARQ_TYPE_Q4_0 || t == BARQ_TYPE_Q8_0 || t == BARQ_TYPE_Q4_K || t == BARQ_TYPE_Q6_K ||
           t == BARQ_TYPE_Q4_0_BARQ;
}

int q8_partner(int w_type) {
    return (w_type == BARQ_TYPE_Q4_K || w_type == BARQ_TYPE_Q6_K) ? BARQ_TYPE_Q8_K : BARQ_TYPE_Q8_0;
}

size_t blk_elems(int t) {
    switch (t) {
    case BARQ_TYPE_F32: case BARQ_TYPE_F16: return 1;
    case BARQ_TYPE_Q4_0: case BARQ_TYPE_Q8_0: case BARQ_TYPE_Q4_0_BARQ: return 32;
    case BARQ_TYPE_Q4_K: case BARQ_TYPE_Q6_K: case BARQ_TYPE_Q8_K: case BARQ_TYPE_Q4_K_BARQ: return 256;
    default: return 0;
    }
}

size_t blk_bytes(int t) {
    switch (t) {
    case BARQ_TYPE_F32: return 4;
    case BARQ_TYPE_F16: return 2;
    case BARQ_TYPE_Q4_0: return 18;
    case BARQ_TYPE_Q4_0_BARQ: return 20;
    case BARQ_TYPE_Q4_K_BARQ: return 136;
    case BARQ_TYPE_Q8_0: return 34;
    case BARQ_TYPE_Q4_K: return 144;
    case BARQ_TYPE_Q6_K: return 210;
    case BARQ_TYPE_Q8_K: return 292;
    default: return 0;
    }
}

size_t row_bytes_of(int t, size_t k) {
    const size_t be = blk_elems(t);
    if (!be || k % be) return 0;
    return k / be * blk_bytes(t);
}

// alignment the kernels need for a packed weight / activation buffer
size_t weight_align(int t) {
    switch (t) {
    case BARQ_TYPE_Q4_K: return 16;
    case BARQ_TYPE_Q4_0_BARQ: case BARQ_TYPE_Q4_K_BARQ: case BARQ_TYPE_Q8_K: case BARQ_TYPE_F32: return 4;
    default: return 2;
    }
}

}  // namespace

int barq_api::ensure_ws(barq_rocm_handle* h, size_t bytes) {
    if (bytes <= h->ws_size) return ok();
    // At least double, so the retired buffers together stay smaller than the
    // live one.  The old buffer is not freed here: kernels still running on
    // any stream, and HIP graphs captured earlier, may reference it.
    size_t want = bytes < 16 * 1024 * 1024 ? 16 * 1024 * 1024 : bytes;
    if (want < 2 * h->ws_size) want = 2 * h->ws_size;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess && want > bytes) {
        (void)hipGetLastError();
        want = bytes;
        e = hipMalloc(&p, want);
    }
    if (e != hipSuccess) return fail(BARQ_E_ALLOC, "workspace of %zu bytes: %s", want, hipGetErrorString(e));
    if (h->ws) h->retired.push_back(h->ws);
    h->ws = p;
    h->ws_size = want;
    return ok();
}

namespace {

using namespace barq_api;

constexpr size_t LDS_LIMIT = 64 * 1024;

}  // namespace

extern "C" {

int barq_rocm_abi_version(void) { return BARQ_ROCM_ABI_VERSION; }

const char* barq_rocm_last_error(void) { return g_last_error.c_str(); }

size_t barq_rocm_block_elems(int type) { return blk_elems(type); }
size_t barq_rocm_block_bytes(int type) { return blk_bytes(type); }
size_t barq_rocm_row_bytes(int type, size_t k) { return row_bytes_of(type, k); }

int barq_rocm_create(int device, barq_rocm_handle** out) {
    if (!out) return fail(BARQ_E_INVALID, "null output pointer");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return fail(BARQ_E_UNSUPPORTED, "ROCm runtime not available: no HIP device");
    if (device < 0 || device >= n) return fail(BARQ_E_UNSUPPORTED, "device %d out of range (%d devices)", device, n);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(BARQ_E_BACKEND, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(BARQ_E_UNSUPPORTED, "device %d is %s; libbarq_rocm is built for gfx950 only", device, prop.gcnArchName);
    DeviceGuard g(device);
    if (hipSetDevice(device) != hipSuccess) return fail(BARQ_E_BACKEND, "hipSetDevice(%d) failed", device);
    if (const int rc = barq::noalloc_init(device)) return rc;
    auto* h = new barq_rocm_handle();
    h->device = device;
    h->tuning = barq::Tuning::from_env();
    e = hipStreamCreateWithFlags(&h->own, hipStreamNonBlocking);
    if (e == hipSuccess) {
        e = hipEventCreateWithFlags(&h->switch_ev, hipEventDisableTiming);
        if (e != hipSuccess) (void)hipStreamDestroy(h->own);
    }
    if (e != hipSuccess) {
        delete h;
        return fail(BARQ_E_BACKEND, "stream/event creation: %s", hipGetErrorString(e));
    }
    h->stream = h->own;
    *out = h;
    return ok();
}

int barq_rocm_destroy(barq_rocm_handle* h) {
    if (!h) return ok();
    DeviceGuard g(h);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->own && h->own != h->stream) (void)hipStreamSynchronize(h->own);
    if (h->ws) (void)hipFree(h->ws);
    for (void* p : h->retired) (void)hipFree(p);
    if (h->switch_ev) (void)hipEventDestroy(h->switch_ev);
    if (h->own) (void)hipStreamDestroy(h->own);
    delete h;
    return ok();
}

int barq_rocm_set_stream(barq_rocm_handle* h, void* stream) {
    BARQ_CHECK(check_handle(h));
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : h->own;
    if (next == h->stream) return ok();
    // Work already enqueued on the old stream (which may still use the
    // workspace) completes before anything enqueued on the new one starts.
    DeviceGuard g(h);
    BARQ_HIP(hipEventRecord(h->switch_ev, h->stream));
    BARQ_HIP(hipStreamWaitEvent(next, h->switch_ev, 0));
    h->stream = next;
    return ok();
}

void* barq_rocm_get_stream(barq_rocm_handle* h) { return h ? static_cast<void*>(h->stream) : nullptr; }

int barq_rocm_synchronize(barq_rocm_handle* h) {
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

// ---------------------------------------------------------------------------
int barq_rocm_dequantize(barq_rocm_handle* h, int type, const void* blocks, size_t n_elems, float* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    const size_t be = blk_elems(type);
    if (!be || type == BARQ_TYPE_F32) return fail(BARQ_E_UNSUPPORTED, "dequantize: unsupported type %d", type);
    if (n_elems % be || n_elems % 4) return fail(BARQ_E_QUANT, "dequantize: %zu elements is not a whole number of %zu-element blocks", n_elems, be);
    if (n_elems == 0) return ok();
    if (!blocks || !out) return fail(BARQ_E_INVALID, "dequantize: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t in_bytes = n_elems / be * blk_bytes(type);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(blocks, type == BARQ_TYPE_F16 ? 8 : weight_align(type)) || !aligned(out, 16))
            return fail(BARQ_E_INVALID, "dequantize: misaligned buffer (blocks %zu-byte, out 16-byte)", weight_align(type));
        return launched(barq::dequant_launch(type, blocks, n_elems, out, h->stream), "dequantize");
    }
    Arena a;
    size_t oi = a.add(in_bytes), oo = a.add(n_elems * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, oi), blocks, in_bytes, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::dequant_launch(type, at<uint8_t>(h, oi), n_elems, at<float>(h, oo), h->stream), "dequantize"));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), n_elems * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_get_rows(barq_rocm_handle* h, int type, const void* table, size_t n_rows, size_t k,
                       const int32_t* tokens, size_t n_tokens, float* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (type == BARQ_TYPE_Q4_K_BARQ || (type != BARQ_TYPE_F32 && !blk_elems(type)))
        return fail(BARQ_E_UNSUPPORTED, "get_rows: unsupported type %d", type);
    const size_t rb = type == BARQ_TYPE_F32 ? k * 4 : row_bytes_of(type, k);
    if (k % 4 || (k && !rb))
        return fail(BARQ_E_QUANT, "get_rows: k=%zu is not a whole number of blocks (and of 4 elements)", k);
    if (n_tokens == 0 || k == 0) return ok();
    if (!table || !tokens || !out) return fail(BARQ_E_INVALID, "get_rows: null buffer");
    if (n_rows > UINT32_MAX || k / 4 > UINT32_MAX) return fail(BARQ_E_DIM, "get_rows: table of %zu x %zu is too large", n_rows, k);
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) {
        const size_t ta = type == BARQ_TYPE_F32 ? 16 : type == BARQ_TYPE_F16 ? 8 : weight_align(type);
        if (!aligned(table, ta) || !aligned(tokens, 4) || !aligned(out, 16))
            return fail(BARQ_E_INVALID, "get_rows: misaligned buffer (table %zu-byte, tokens 4-byte, out 16-byte)", ta);
        return launched(barq::get_rows_launch(type, table, rb, n_rows, k, tokens, n_tokens, out, h->stream), "get_rows");
    }
    // host buffers: only the rows the tokens name travel (slot j holds the
    // j-th in-range token's row; the others map to -1 and stay zero)
    std::vector<int32_t> ids(n_tokens);
    size_t used = 0;
    for (size_t t = 0; t < n_tokens; t++)
        ids[t] = tokens[t] >= 0 && (size_t)tokens[t] < n_rows ? (int32_t)used++ : -1;
    Arena a;
    const size_t orows = a.add(used * rb), oid = a.add(n_tokens * 4), oo = a.add(n_tokens * k * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    const uint8_t* tb = static_cast<const uint8_t*>(table);
    for (size_t t = 0; t < n_tokens; t++)
        if (ids[t] >= 0)
            BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, orows) + (size_t)ids[t] * rb, tb + (size_t)tokens[t] * rb, rb,
                                    hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<int32_t>(h, oid), ids.data(), n_tokens * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::get_rows_launch(type, at<uint8_t>(h, orows), rb, used, k, at<int32_t>(h, oid), n_tokens,
                                              at<float>(h, oo), h->stream), "get_rows"));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), n_tokens * k * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_stream_read(barq_rocm_handle* h, const void* p, size_t bytes, uint32_t* sink) {
    if (bytes < 16) return ok();
    if (!p || !sink) return fail(BARQ_E_INVALID, "stream_read: null buffer");
    if (!aligned(p, 16) || !aligned(sink, 4)) return fail(BARQ_E_INVALID, "stream_read: p must be 16-byte aligned");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    return launched(barq::stream_read_launch(p, bytes, sink, h->stream), "stream_read");
}

int barq_rocm_add_bias(barq_rocm_handle* h, float* y, const float* bias, size_t rows, size_t dim, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (rows == 0 || dim == 0) return ok();
    if (!y || !bias) return fail(BARQ_E_INVALID, "add_bias: null buffer");
    if (dim > UINT32_MAX) return fail(BARQ_E_DIM, "add_bias: dim %zu exceeds 2^32", dim);
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(y, 4) || !aligned(bias, 4)) return fail(BARQ_E_INVALID, "add_bias: misaligned buffer");
        return launched(barq::add_bias_launch(y, bias, rows, dim, h->stream), "add_bias");
    }
    Arena a;
    const size_t oy = a.add(rows * dim * 4), ob = a.add(dim * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, oy), y, rows * dim * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ob), bias, dim * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::add_bias_launch(at<float>(h, oy), at<float>(h, ob), rows, dim, h->stream), "add_bias"));
    BARQ_HIP(hipMemcpyAsync(y, at<float>(h, oy), rows * dim * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

static hipError_t quantize_act_dev(int act_type, const float* x, size_t n_rows, size_t k, void* out, hipStream_t s) {
    return act_type == BARQ_TYPE_Q8_0 ? barq::quantize_q8_0_launch(x, n_rows, k, out, s)
                                      : barq::quantize_q8_k_launch(x, n_rows, k, out, s);
}

int barq_rocm_quantize_act(barq_rocm_handle* h, int act_type, const float* x, size_t n_rows, size_t k, void* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (act_type != BARQ_TYPE_Q8_0 && act_type != BARQ_TYPE_Q8_K)
        return fail(BARQ_E_UNSUPPORTED, "quantize_act: act_type must be Q8_0 or Q8_K, got %d", act_type);
    const size_t be = blk_elems(act_type);
    if (k % be) return fail(BARQ_E_QUANT, "quantize_act: k=%zu is not a multiple of %zu", k, be);
    if (n_rows == 0 || k == 0) return ok();
    if (!x || !out) return fail(BARQ_E_INVALID, "quantize_act: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t out_bytes = n_rows * row_bytes_of(act_type, k);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(x, 16) || !aligned(out, act_type == BARQ_TYPE_Q8_K ? 4 : 2))
            return fail(BARQ_E_INVALID, "quantize_act: misaligned buffer (x 16-byte, out %d-byte)", act_type == BARQ_TYPE_Q8_K ? 4 : 2);
        return launched(quantize_act_dev(act_type, x, n_rows, k, out, h->stream), "quantize_act");
    }
    Arena a;
    size_t ox = a.add(n_rows * k * 4), oo = a.add(out_bytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, n_rows * k * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(quantize_act_dev(act_type, at<float>(h, ox), n_rows, k, at<uint8_t>(h, oo), h->stream), "quantize_act"));
    BARQ_HIP(hipMemcpyAsync(out, at<uint8_t>(h, oo), out_bytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

// ---------------------------------------------------------------------------
// RMSNorm (transformer.rs:148-172), alone and fused with the quantizer

int barq_rocm_rms_norm(barq_rocm_handle* h, const float* x, const float* weight, size_t rows, size_t n, float eps,
                       float* y, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (rows == 0 || n == 0) return ok();
    if (!barq::rms_norm_supported(n)) return fail(BARQ_E_DIM, "rms_norm: n=%zu must be a multiple of 4 and at most 16384", n);
    if (!x || !weight || !y) return fail(BARQ_E_INVALID, "rms_norm: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(y, 16))
            return fail(BARQ_E_INVALID, "rms_norm: buffers must be 16-byte aligned");
        return launched(barq::rms_norm_launch(x, weight, rows, n, eps, y, h->stream), "rms_norm");
    }
    Arena a;
    const size_t ox = a.add(rows * n * 4), ow = a.add(n * 4), oy = a.add(rows * n * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, rows * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ow), weight, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::rms_norm_launch(at<float>(h, ox), at<float>(h, ow), rows, n, eps, at<float>(h, oy), h->stream),
                        "rms_norm"));
    BARQ_HIP(hipMemcpyAsync(y, at<float>(h, oy), rows * n * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_rms_norm_quantize(barq_rocm_handle* h, int act_type, const float* x, const float* weight, size_t rows,
                                size_t n, float eps, void* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (act_type != BARQ_TYPE_Q8_0 && act_type != BARQ_TYPE_Q8_K)
        return fail(BARQ_E_UNSUPPORTED, "rms_norm_quantize: act_type must be Q8_0 or Q8_K, got %d", act_type);
    if (rows == 0 || n == 0) return ok();
    if (n % 256 != 0 || !barq::rms_norm_supported(n))
        return fail(BARQ_E_DIM, "rms_norm_quantize: n=%zu must be a multiple of 256 and at most 16384", n);
    if (!x || !weight || !out) return fail(BARQ_E_INVALID, "rms_norm_quantize: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t out_bytes = rows * row_bytes_of(act_type, n);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, act_type == BARQ_TYPE_Q8_K ? 4 : 2))
            return fail(BARQ_E_INVALID, "rms_norm_quantize: misaligned buffer (x, weight 16-byte; out %d-byte)",
                        act_type == BARQ_TYPE_Q8_K ? 4 : 2);
        return launched(barq::rms_norm_quantize_launch(act_type, x, weight, rows, n, eps, out, h->stream), "rms_norm_quantize");
    }
    Arena a;
    const size_t ox = a.add(rows * n * 4), ow = a.add(n * 4), oo = a.add(out_bytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, rows * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ow), weight, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::rms_norm_quantize_launch(act_type, at<float>(h, ox), at<float>(h, ow), rows, n, eps,
                                                       at<uint8_t>(h, oo), h->stream), "rms_norm_quantize"));
    BARQ_HIP(hipMemcpyAsync(out, at<uint8_t>(h, oo), out_bytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_add_rms_norm_quantize(barq_rocm_handle* h, int out_type, const float* x, const float* d,
                                    const float* weight, size_t rows, size_t n, float eps, float* sum, void* out,
                                    int mem) {
    BARQ_CHECK(check_mem(mem));
    if (out_type != BARQ_TYPE_F32 && out_type != BARQ_TYPE_Q8_0 && out_type != BARQ_TYPE_Q8_K)
        return fail(BARQ_E_UNSUPPORTED, "add_rms_norm_quantize: out_type must be F32, Q8_0 or Q8_K, got %d", out_type);
    if (rows == 0 || n == 0) return ok();
    if (!barq::rms_norm_supported(n) || (out_type != BARQ_TYPE_F32 && n % 256 != 0))
        return fail(BARQ_E_DIM, "add_rms_norm_quantize: n=%zu must be a multiple of %d and at most 16384", n,
                    out_type == BARQ_TYPE_F32 ? 4 : 256);
    if (!x || !weight || !out) return fail(BARQ_E_INVALID, "add_rms_norm_quantize: null buffer");
    if (sum && !d) return fail(BARQ_E_INVALID, "add_rms_norm_quantize: sum needs d (it receives x + d)");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t out_bytes = rows * (out_type == BARQ_TYPE_F32 ? n * 4 : row_bytes_of(out_type, n));
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(x, 16) || !aligned(weight, 16) || (d && !aligned(d, 16)) || (sum && !aligned(sum, 16)) ||
            !aligned(out, out_type == BARQ_TYPE_F32 ? 16 : out_type == BARQ_TYPE_Q8_K ? 4 : 2))
            return fail(BARQ_E_INVALID, "add_rms_norm_quantize: x, d, weight, sum 16-byte aligned; out %d-byte",
                        out_type == BARQ_TYPE_F32 ? 16 : out_type == BARQ_TYPE_Q8_K ? 4 : 2);
        return launched(barq::add_rms_norm_launch(out_type, x, d, weight, rows, n, eps, sum, out, h->stream),
                        "add_rms_norm_quantize");
    }
    Arena a;
    const size_t ox = a.add(rows * n * 4), od = a.add(d ? rows * n * 4 : 0), ow = a.add(n * 4),
                 os = a.add(sum ? rows * n * 4 : 0), oo = a.add(out_bytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, rows * n * 4, hipMemcpyHostToDevice, h->stream));
    if (d) BARQ_HIP(hipMemcpyAsync(at<float>(h, od), d, rows * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ow), weight, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::add_rms_norm_launch(out_type, at<float>(h, ox), d ? at<float>(h, od) : nullptr,
                                                  at<float>(h, ow), rows, n, eps, sum ? at<float>(h, os) : nullptr,
                                                  at<uint8_t>(h, oo), h->stream), "add_rms_norm_quantize"));
    if (sum) BARQ_HIP(hipMemcpyAsync(sum, at<float>(h, os), rows * n * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipMemcpyAsync(out, at<uint8_t>(h, oo), out_bytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

// ---------------------------------------------------------------------------
// matvec / matmul

namespace {

int check_linear(int w_type, size_t k, int act_type, const char* what) {
    if (!is_weight_type(w_type)) return fail(BARQ_E_UNSUPPORTED, "%s: unsupported weight type %d", what, w_type);
    if (row_bytes_of(w_type, k) == 0) return fail(BARQ_E_QUANT, "%s: k=%zu is not a multiple of the %zu-element block", what, k, blk_elems(w_type));
    if (act_type == BARQ_ACT_F32 || act_type == BARQ_ACT_F32_Q8) return ok();
    if (act_type != BARQ_TYPE_Q8_0 && act_type != BARQ_TYPE_Q8_K)
        return fail(BARQ_E_UNSUPPORTED, "%s: unsupported activation type %d", what, act_type);
    if (act_type != q8_partner(w_type))
        return fail(BARQ_E_UNSUPPORTED, "%s: weight type %d pairs with activation type %d, got %d", what, w_type, q8_partner(w_type), act_type);
    return ok();
}

size_t act_row_bytes(int act_type, int w_type, size_t k) {
    if (act_type == BARQ_ACT_F32 || act_type == BARQ_ACT_F32_Q8) return k * 4;
    return row_bytes_of(act_type, k);
}

// Workspace bytes matmul_dev uses from offset 0: the dequantized weights of
// the literal f32 matmul, or the rows quantized here followed by the
// repacked rows of the 32-element-block GEMM or the K slices' partial
// products of either MFMA GEMM.
size_t matmul_scratch(int w_type, size_t n_rows, size_t k, int act_type, size_t m) {
    if (act_type == BARQ_ACT_F32) return m > 1 ? n_rows * k * 4 : 0;
    const size_t q = act_type == BARQ_ACT_F32_Q8 ? round_up(m * row_bytes_of(q8_partner(w_type), k), 256) : 0;
    if (m < (size_t)barq::gemm_min_rows(w_type)) return q;
    if (barq::b32_supported(w_type, n_rows, k, m)) return q + barq::b32_workspace(m, n_rows, k);
    if (barq::gemm_mfma_supported(w_type, n_rows, k, m)) return q + barq::gemm_mfma_workspace(w_type, n_rows, k, m);
    return q;
}

// Device-pointer matmul core.  x holds m rows (f32 or Q8 blocks).  ws is
// scratch of at least matmul_scratch(...) bytes, or null: then the call
// takes quantized activations only and uses no scratch (no
// 32-element-block GEMM, no K slices; the MoE path keeps its data in the
// workspace meanwhile).
int matmul_dev(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k, int act_type,
               const void* x, size_t m, float* y, uint8_t* ws) {
    hipStream_t s = h->stream;
    const bool use_ws = ws != nullptr;
    if (!use_ws && (act_type == BARQ_ACT_F32_Q8 || (act_type == BARQ_ACT_F32 && m > 1)))
        return fail(BARQ_E_INVALID, "matmul without workspace takes quantized activations (or one f32 row)");
    if (!aligned(w, weight_align(w_type))) return fail(BARQ_E_INVALID, "weights must be %zu-byte aligned", weight_align(w_type));
    if (!aligned(y, 4)) return fail(BARQ_E_INVALID, "output must be 4-byte aligned");
    if (act_type == BARQ_ACT_F32) {
        if (!aligned(x, 16)) return fail(BARQ_E_INVALID, "f32 activations must be 16-byte aligned");
        if (m == 1) {
            if (k * 4 > LDS_LIMIT) return fail(BARQ_E_UNSUPPORTED, "f32-activation matvec supports k <= %zu", LDS_LIMIT / 4);
            return launched(barq::gemv_f32_launch(w_type, w, n_rows, k, static_cast<const float*>(x), y, s), "gemv_f32");
        }
        // literal matmul: dequantize W (bit-exact) then the sequential f32 GEMM
        float* wf = reinterpret_cast<float*>(ws);
        BARQ_CHECK(launched(barq::dequant_launch(w_type, w, n_rows * k, wf, s), "dequantize"));
        return launched(barq::gemm_f32_nt_launch(static_cast<const float*>(x), wf, m, k, n_rows, y, s), "gemm_f32_nt");
    }
    const int aq = q8_partner(w_type);
    const uint8_t* xq = static_cast<const uint8_t*>(x);
    // scratch: the quantized rows (when quantized here), then the repacked
    // rows of the 32-element-block GEMM or the K slices' partial products
    // the MFMA GEMMs copy weight rows with 4-byte buffer->LDS loads
    const bool w4 = aligned(w, 4);
    const bool gemm = m >= (size_t)barq::gemm_min_rows(w_type);
    const bool b32 = use_ws && gemm && w4 && barq::b32_supported(w_type, n_rows, k, m);
    const size_t qbytes = act_type == BARQ_ACT_F32_Q8 ? round_up(m * row_bytes_of(aq, k), 256) : 0;
    if (act_type == BARQ_ACT_F32_Q8) {
        if (!aligned(x, 16)) return fail(BARQ_E_INVALID, "f32 activations must be 16-byte aligned");
        BARQ_CHECK(launched(quantize_act_dev(aq, static_cast<const float*>(x), m, k, ws, s), "quantize_act"));
        xq = ws;
    } else if (!aligned(x, aq == BARQ_TYPE_Q8_K ? 4 : 2)) {
        return fail(BARQ_E_INVALID, "activation blocks misaligned");
    }
    if (barq::gemv_multi_supported(w_type, w, n_rows, k, xq, m))
        return launched(barq::gemv_q8_multi_launch(w_type, w, n_rows, k, xq, m, y, s), "gemv_q8_multi");
    if (b32) return launched(barq::b32_gemm_launch(w_type, w, n_rows, k, xq, m, ws + qbytes, y, s), "gemm_b32");
    if (gemm && w4 && barq::gemm_mfma_supported(w_type, n_rows, k, m))
        return launched(barq::gemm_q8k_mfma_launch(w_type, w, n_rows, k, xq, m, use_ws ? ws + qbytes : nullptr, y, s),
                        "gemm_mfma");
    const size_t xrb = row_bytes_of(aq, k);
    for (size_t r = 0; r < m; r++)
        BARQ_CHECK(launched(barq::gemv_q8_launch(w_type, w, n_rows, k, xq + r * xrb, y + r * n_rows, s), "gemv_q8"));
    return ok();
}

int check_matmul_args(int w_type, size_t n_rows, size_t k, int act_type, const void* w, const void* x, size_t m,
                      const float* y, const char* what) {
    BARQ_CHECK(check_linear(w_type, k, act_type, what));
    if (n_rows == 0 || m == 0) return ok();
    if (!w || !x || !y) return fail(BARQ_E_INVALID, "%s: null buffer", what);
    if (n_rows > (size_t)INT32_MAX || k > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "%s: dimensions exceed 2^31", what);
    return ok();
}

}  // namespace
}  // extern "C"

int barq_api::matmul_fixed_scratch(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k,
                                   int act_type, const void* x, size_t m, float* y, void* ws, size_t ws_bytes,
                                   const char* what) {
    BARQ_CHECK(check_matmul_args(w_type, n_rows, k, act_type, w, x, m, y, what));
    if (n_rows == 0 || m == 0) return ok();
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t need = matmul_scratch(w_type, n_rows, k, act_type, m);
    if (need > ws_bytes)
        return fail(BARQ_E_UNSUPPORTED, "%s: this call needs %zu bytes of scratch, more than the %zu available", what,
                    need, ws_bytes);
    return matmul_dev(h, w_type, w, n_rows, k, act_type, x, m, y, need ? static_cast<uint8_t*>(ws) : nullptr);
}

extern "C" {
namespace {

int matmul_any(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k, int act_type,
               const void* x, size_t m, float* y, int mem, const char* what) {
    BARQ_CHECK(check_mem(mem));
    BARQ_CHECK(check_matmul_args(w_type, n_rows, k, act_type, w, x, m, y, what));
    if (n_rows == 0 || m == 0) return ok();
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t need = matmul_scratch(w_type, n_rows, k, act_type, m);
    if (mem == BARQ_MEM_DEVICE) {
        if (need) BARQ_CHECK(ensure_ws(h, need));
        return matmul_dev(h, w_type, w, n_rows, k, act_type, x, m, y, need ? at<uint8_t>(h, 0) : nullptr);
    }
    // host buffers: stage W, x, y after the region matmul_dev itself may use
    const size_t wbytes = n_rows * row_bytes_of(w_type, k);
    const size_t xbytes = m * act_row_bytes(act_type, w_type, k);
    const size_t ybytes = m * n_rows * 4;
    Arena a;
    a.add(need);
    size_t ow = a.add(wbytes), ox = a.add(xbytes), oy = a.add(ybytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, ow), w, wbytes, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, ox), x, xbytes, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(matmul_dev(h, w_type, at<uint8_t>(h, ow), n_rows, k, act_type, at<uint8_t>(h, ox), m, at<float>(h, oy),
                          need ? at<uint8_t>(h, 0) : nullptr));
    BARQ_HIP(hipMemcpyAsync(y, at<float>(h, oy), ybytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

}  // namespace

int barq_rocm_matvec(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k, int act_type,
                     const void* x, float* y, int mem) {
    return matmul_any(h, w_type, w, n_rows, k, act_type, x, 1, y, mem, "matvec");
}

int barq_rocm_matmul(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k, int act_type,
                     const void* x, size_t m, float* y, int mem) {
    return matmul_any(h, w_type, w, n_rows, k, act_type, x, m, y, mem, "matmul");
}

int barq_rocm_matvec_group(barq_rocm_handle* h, size_t n_mats, const int* w_types, const void* const* w,
                           const size_t* n_rows, size_t k, int act_type, const void* x, float* const* y, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (n_mats == 0) return ok();
    if (!w_types || !w || !n_rows || !y) return fail(BARQ_E_INVALID, "matvec_group: null array");
    for (size_t i = 0; i < n_mats; i++)
        BARQ_CHECK(check_matmul_args(w_types[i], n_rows[i], k, act_type, w[i], x, 1, y[i], "matvec_group"));
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    // one launch for Q4_K matrices (and a last Q6_K one) on device Q8_K rows
    if (mem == BARQ_MEM_DEVICE && act_type == BARQ_TYPE_Q8_K && aligned(x, 4) &&
        barq::gemv_group_supported(n_mats, w_types, w, n_rows, k)) {
        for (size_t i = 0; i < n_mats; i++)
            if (!aligned(y[i], 4)) return fail(BARQ_E_INVALID, "matvec_group: y must be 4-byte aligned");
        return launched(barq::gemv_group_launch(n_mats, w_types, w, n_rows, k, x, y, h->stream), "matvec_group");
    }
    for (size_t i = 0; i < n_mats; i++)
        BARQ_CHECK(matmul_any(h, w_types[i], w[i], n_rows[i], k, act_type, x, 1, y[i], mem, "matvec_group"));
    return ok();
}

// ---------------------------------------------------------------------------
// dense FFN (LlamaTransformer::feed_forward, transformer.rs:378-408)

int barq_rocm_swiglu(barq_rocm_handle* h, int out_type, const float* gate, const float* up, size_t rows, size_t n,
                     void* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (out_type != BARQ_TYPE_F32 && out_type != BARQ_TYPE_Q8_K && out_type != BARQ_TYPE_Q8_0)
        return fail(BARQ_E_UNSUPPORTED, "swiglu: out_type must be F32, Q8_K or Q8_0, got %d", out_type);
    if (rows == 0 || n == 0) return ok();
    if (out_type != BARQ_TYPE_F32 && n % blk_elems(out_type))
        return fail(BARQ_E_QUANT, "swiglu: n=%zu is not a multiple of %zu", n, blk_elems(out_type));
    if (!gate || !up || !out) return fail(BARQ_E_INVALID, "swiglu: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t out_bytes = rows * (out_type == BARQ_TYPE_F32 ? n * 4 : row_bytes_of(out_type, n));
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(out, out_type == BARQ_TYPE_Q8_0 ? 2 : 4))
            return fail(BARQ_E_INVALID, "swiglu: gate/up must be 16-byte aligned, out %d-byte",
                        out_type == BARQ_TYPE_Q8_0 ? 2 : 4);
        return launched(barq::ffn_swiglu_launch(out_type, gate, up, rows, n, out, h->stream), "swiglu");
    }
    Arena a;
    const size_t og = a.add(rows * n * 4), ou = a.add(rows * n * 4), oo = a.add(out_bytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, og), gate, rows * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ou), up, rows * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::ffn_swiglu_launch(out_type, at<float>(h, og), at<float>(h, ou), rows, n, at<uint8_t>(h, oo),
                                                h->stream), "swiglu"));
    BARQ_HIP(hipMemcpyAsync(out, at<uint8_t>(h, oo), out_bytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

namespace {

// Workspace of a device FFN call, from offset `base`: the input rows
// quantized here, g and u (m x n_ff f32 each; h in f32 reuses g), h's
// quantized rows, then scratch for the three projections.
struct FfnArena {
    size_t xq, g, u, hq, mm, end;
};

FfnArena ffn_arena(size_t base, int gt, int ut, int dt, size_t n_embd, size_t n_ff, int act, size_t m) {
    Arena a;
    a.used = base;
    FfnArena L;
    const bool lit = act == BARQ_ACT_F32;
    L.xq = a.add(act == BARQ_ACT_F32_Q8 ? m * row_bytes_of(q8_partner(gt), n_embd) : 0);
    L.g = a.add(m * n_ff * 4);
    L.u = a.add(m * n_ff * 4);
    L.hq = a.add(lit ? 0 : m * row_bytes_of(q8_partner(dt), n_ff));
    const int pa = lit ? BARQ_ACT_F32 : q8_partner(gt), pd = lit ? BARQ_ACT_F32 : q8_partner(dt);
    size_t mm = matmul_scratch(gt, n_ff, n_embd, pa, m);
    mm = std::max(mm, matmul_scratch(ut, n_ff, n_embd, pa, m));
    mm = std::max(mm, matmul_scratch(dt, n_embd, n_ff, pd, m));
    L.mm = a.add(mm);
    L.end = a.used;
    return L;
}

int ffn_dev(barq_rocm_handle* h, int gt, const void* gate, int ut, const void* up, int dt, const void* down,
            size_t n_embd, size_t n_ff, int act, const void* x, size_t m, float* out, size_t base) {
    hipStream_t s = h->stream;
    const FfnArena L = ffn_arena(base, gt, ut, dt, n_embd, n_ff, act, m);
    BARQ_CHECK(ensure_ws(h, L.end));
    float* g = at<float>(h, L.g);
    float* u = at<float>(h, L.u);
    uint8_t* mm = at<uint8_t>(h, L.mm);
    if (act == BARQ_ACT_F32) {
        // the literal f32 arithmetic: f32 projections, f32 SwiGLU, f32 down
        BARQ_CHECK(matmul_dev(h, gt, gate, n_ff, n_embd, BARQ_ACT_F32, x, m, g, mm));
        BARQ_CHECK(matmul_dev(h, ut, up, n_ff, n_embd, BARQ_ACT_F32, x, m, u, mm));
        BARQ_CHECK(launched(barq::ffn_swiglu_launch(BARQ_TYPE_F32, g, u, m, n_ff, g, s), "swiglu"));
        return matmul_dev(h, dt, down, n_embd, n_ff, BARQ_ACT_F32, g, m, out, mm);
    }
    const int pa = q8_partner(gt), pd = q8_partner(dt);
    const void* xq = x;
    if (act == BARQ_ACT_F32_Q8) {
        if (!aligned(x, 16)) return fail(BARQ_E_INVALID, "ffn: f32 activations must be 16-byte aligned");
        BARQ_CHECK(launched(quantize_act_dev(pa, static_cast<const float*>(x), m, n_embd, at<uint8_t>(h, L.xq), s),
                            "quantize_act"));
        xq = at<uint8_t>(h, L.xq);
    }
    uint8_t* hq = at<uint8_t>(h, L.hq);
    if (m == 1 && gt == ut && barq::gemv_glu_supported(gt, gate, up, n_ff, n_embd)) {
        // gate and up in one launch, SwiGLU in its epilogue
        BARQ_CHECK(launched(barq::gemv_glu_launch(gt, gate, up, n_ff, n_embd, xq, g, s), "gemv_glu"));
        BARQ_CHECK(launched(quantize_act_dev(pd, g, 1, n_ff, hq, s), "quantize_act"));
    } else if (gt == ut && barq::gemv_glu_multi_supported(gt, gate, up, n_ff, n_embd, m)) {
        // 2-4 tokens: the same launch over every row (weights read once)
        BARQ_CHECK(launched(barq::gemv_glu_launch(gt, gate, up, n_ff, n_embd, xq, g, s, m), "gemv_glu"));
        BARQ_CHECK(launched(quantize_act_dev(pd, g, m, n_ff, hq, s), "quantize_act"));
    } else {
        BARQ_CHECK(matmul_dev(h, gt, gate, n_ff, n_embd, pa, xq, m, g, mm));
        BARQ_CHECK(matmul_dev(h, ut, up, n_ff, n_embd, pa, xq, m, u, mm));
        BARQ_CHECK(launched(barq::ffn_swiglu_launch(pd, g, u, m, n_ff, hq, s), "swiglu"));
    }
    return matmul_dev(h, dt, down, n_embd, n_ff, pd, hq, m, out, mm);
}

}  // namespace

int barq_rocm_ffn(barq_rocm_handle* h, int gate_type, const void* gate, int up_type, const void* up, int down_type,
                  const void* down, size_t n_embd, size_t n_ff, int act, const void* x, size_t m, float* out,
                  int mem) {
    BARQ_CHECK(check_mem(mem));
    const bool quantized_in = act == BARQ_TYPE_Q8_0 || act == BARQ_TYPE_Q8_K;
    if (act != BARQ_ACT_F32 && act != BARQ_ACT_F32_Q8 && !quantized_in)
        return fail(BARQ_E_UNSUPPORTED, "ffn: act must be BARQ_ACT_F32, BARQ_ACT_F32_Q8, Q8_0 or Q8_K, got %d", act);
    BARQ_CHECK(check_linear(gate_type, n_embd, quantized_in ? act : BARQ_ACT_F32, "ffn gate"));
    BARQ_CHECK(check_linear(up_type, n_embd, quantized_in ? act : BARQ_ACT_F32, "ffn up"));
    BARQ_CHECK(check_linear(down_type, n_ff, BARQ_ACT_F32, "ffn down"));
    if (act != BARQ_ACT_F32 && q8_partner(gate_type) != q8_partner(up_type))
        return fail(BARQ_E_UNSUPPORTED, "ffn: gate and up weights must share an activation type");
    if (act != BARQ_ACT_F32 && row_bytes_of(q8_partner(down_type), n_ff) == 0)
        return fail(BARQ_E_QUANT, "ffn: n_ff=%zu is not a multiple of the down input's block", n_ff);
    if (m == 0 || n_embd == 0 || n_ff == 0) return ok();
    if (!gate || !up || !down || !x || !out) return fail(BARQ_E_INVALID, "ffn: null buffer");
    if (n_embd > (size_t)INT32_MAX || n_ff > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "ffn: dimensions exceed 2^31");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(out, 4)) return fail(BARQ_E_INVALID, "ffn: output must be 4-byte aligned");
        return ffn_dev(h, gate_type, gate, up_type, up, down_type, down, n_embd, n_ff, act, x, m, out, 0);
    }
    const size_t gb = n_ff * row_bytes_of(gate_type, n_embd), ub = n_ff * row_bytes_of(up_type, n_embd),
                 db = n_embd * row_bytes_of(down_type, n_ff);
    const size_t xb = m * (quantized_in ? row_bytes_of(act, n_embd) : n_embd * 4), ob = m * n_embd * 4;
    Arena a;
    const size_t og = a.add(gb), ou = a.add(ub), od = a.add(db), ox = a.add(xb), oo = a.add(ob);
    const FfnArena L = ffn_arena(a.used, gate_type, up_type, down_type, n_embd, n_ff, act, m);
    BARQ_CHECK(ensure_ws(h, L.end));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, og), gate, gb, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, ou), up, ub, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, od), down, db, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, ox), x, xb, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(ffn_dev(h, gate_type, at<uint8_t>(h, og), up_type, at<uint8_t>(h, ou), down_type, at<uint8_t>(h, od),
                       n_embd, n_ff, act, at<uint8_t>(h, ox), m, at<float>(h, oo), a.used));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), ob, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

// ---------------------------------------------------------------------------
// f32 BLAS

int barq_rocm_gemm_f32(barq_rocm_handle* h, const float* a, const float* b, size_t m, size_t k, size_t n, float* c, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (m == 0 || n == 0) return ok();
    if (!a || !b || !c) return fail(BARQ_E_INVALID, "gemm_f32: null buffer");
    if (m > (size_t)INT32_MAX || n > (size_t)INT32_MAX || k > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "gemm_f32: dimensions exceed 2^31");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) return launched(barq::gemm_f32_launch(a, b, m, k, n, c, h->stream), "gemm_f32");
    Arena ar;
    size_t oa = ar.add(m * k * 4), ob = ar.add(k * n * 4), oc = ar.add(m * n * 4);
    BARQ_CHECK(ensure_ws(h, ar.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, oa), a, m * k * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ob), b, k * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::gemm_f32_launch(at<float>(h, oa), at<float>(h, ob), m, k, n, at<float>(h, oc), h->stream), "gemm_f32"));
    BARQ_HIP(hipMemcpyAsync(c, at<float>(h, oc), m * n * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_gemv_f32(barq_rocm_handle* h, const float* a, const float* x, size_t m, size_t n, float* y, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (m == 0) return ok();
    if (!a || !x || !y) return fail(BARQ_E_INVALID, "gemv_f32: null buffer");
    if (m > (size_t)INT32_MAX || n > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "gemv_f32: dimensions exceed 2^31");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) return launched(barq::gemv_f32_plain_launch(a, x, m, n, y, h->stream), "gemv_f32");
    Arena ar;
    size_t oa = ar.add(m * n * 4), ox = ar.add(n * 4), oy = ar.add(m * 4);
    BARQ_CHECK(ensure_ws(h, ar.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, oa), a, m * n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::gemv_f32_plain_launch(at<float>(h, oa), at<float>(h, ox), m, n, at<float>(h, oy), h->stream), "gemv_f32"));
    BARQ_HIP(hipMemcpyAsync(y, at<float>(h, oy), m * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

// ---------------------------------------------------------------------------
// split-scale operator API (QuantizedCudaOps)

int barq_rocm_dequantize_split(barq_rocm_handle* h, int kind, const uint8_t* quants, size_t n_quants,
                               const float* scales, size_t n_scales, size_t block_size, float* out,
                               size_t n_out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (block_size == 0) return fail(BARQ_E_INVALID, "dequantize_split: block_size must be > 0");
    if (n_out == 0) return ok();
    if (!out || (n_quants && !quants) || (n_scales && !scales)) return fail(BARQ_E_INVALID, "dequantize_split: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const int q8 = kind == BARQ_TYPE_Q8_0;
    if (mem == BARQ_MEM_DEVICE)
        return launched(barq::dequant_split_launch(q8, quants, n_quants, scales, n_scales, block_size, out, n_out, h->stream), "dequantize_split");
    Arena a;
    size_t oq = a.add(n_quants), os = a.add(n_scales * 4), oo = a.add(n_out * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    if (n_quants) BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, oq), quants, n_quants, hipMemcpyHostToDevice, h->stream));
    if (n_scales) BARQ_HIP(hipMemcpyAsync(at<float>(h, os), scales, n_scales * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::dequant_split_launch(q8, at<uint8_t>(h, oq), n_quants, at<float>(h, os), n_scales, block_size,
                                                   at<float>(h, oo), n_out, h->stream), "dequantize_split"));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), n_out * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_quantized_matmul_split(barq_rocm_handle* h, const float* a, const uint8_t* bq, size_t n_bq,
                                     const float* bs, size_t n_bs, float* c, size_t m, size_t n, size_t k,
                                     int kind, size_t block_size, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (block_size == 0) return fail(BARQ_E_INVALID, "quantized_matmul: block_size must be > 0");
    if (m == 0 || n == 0) return ok();
    if (!a || !c || (n_bq && !bq) || (n_bs && !bs)) return fail(BARQ_E_INVALID, "quantized_matmul: null buffer");
    if (m > (size_t)INT32_MAX || n > (size_t)INT32_MAX || k > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "quantized_matmul: dimensions exceed 2^31");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const int q8 = kind == BARQ_TYPE_Q8_0;
    Arena ar;
    size_t ob = ar.add(k * n * 4);
    size_t oa = 0, oq = 0, os = 0, oc = 0;
    if (mem == BARQ_MEM_HOST) {
        oa = ar.add(m * k * 4); oq = ar.add(n_bq); os = ar.add(n_bs * 4); oc = ar.add(m * n * 4);
    }
    BARQ_CHECK(ensure_ws(h, ar.used));
    const float* da = a;
    const uint8_t* dq = bq;
    const float* ds = bs;
    float* dc = c;
    if (mem == BARQ_MEM_HOST) {
        BARQ_HIP(hipMemcpyAsync(at<float>(h, oa), a, m * k * 4, hipMemcpyHostToDevice, h->stream));
        if (n_bq) BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, oq), bq, n_bq, hipMemcpyHostToDevice, h->stream));
        if (n_bs) BARQ_HIP(hipMemcpyAsync(at<float>(h, os), bs, n_bs * 4, hipMemcpyHostToDevice, h->stream));
        da = at<float>(h, oa); dq = at<uint8_t>(h, oq); ds = at<float>(h, os); dc = at<float>(h, oc);
    }
    float* b = at<float>(h, ob);
    BARQ_CHECK(launched(barq::dequant_split_launch(q8, dq, n_bq, ds, n_bs, block_size, b, k * n, h->stream), "dequantize_split"));
    BARQ_CHECK(launched(barq::gemm_f32_launch(da, b, m, k, n, dc, h->stream), "gemm_f32"));
    if (mem == BARQ_MEM_HOST) {
        BARQ_HIP(hipMemcpyAsync(c, dc, m * n * 4, hipMemcpyDeviceToHost, h->stream));
        BARQ_HIP(hipStreamSynchronize(h->stream));
    }
    return ok();
}

int barq_rocm_quantize_q4_0_barq(barq_rocm_handle* h, const float* x, size_t n, uint8_t* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (n % 32) return fail(BARQ_E_QUANT, "quantize_q4_0_barq: n=%zu is not a multiple of 32", n);
    if (n == 0) return ok();
    if (!x || !out) return fail(BARQ_E_INVALID, "quantize_q4_0_barq: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t ob_bytes = n / 32 * 20;
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(out, 4)) return fail(BARQ_E_INVALID, "quantize_q4_0_barq: out must be 4-byte aligned");
        return launched(barq::quantize_q4_0_barq_launch(x, n, out, h->stream), "quantize_q4_0_barq");
    }
    Arena a;
    size_t ox = a.add(n * 4), oo = a.add(ob_bytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::quantize_q4_0_barq_launch(at<float>(h, ox), n, at<uint8_t>(h, oo), h->stream), "quantize_q4_0_barq"));
    BARQ_HIP(hipMemcpyAsync(out, at<uint8_t>(h, oo), ob_bytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

int barq_rocm_quantize_q4_k_barq(barq_rocm_handle* h, const float* x, size_t n, uint8_t* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (n == 0) return ok();
    if (!x || !out) return fail(BARQ_E_INVALID, "quantize_q4_k_barq: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    const size_t ob_bytes = barq_rocm_q4_k_barq_bytes(n);
    if (mem == BARQ_MEM_DEVICE) {
        if (!aligned(out, 4)) return fail(BARQ_E_INVALID, "quantize_q4_k_barq: out must be 4-byte aligned");
        return launched(barq::quantize_q4_k_barq_launch(x, n, out, h->stream), "quantize_q4_k_barq");
    }
    Arena a;
    size_t ox = a.add(n * 4), oo = a.add(ob_bytes);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, n * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::quantize_q4_k_barq_launch(at<float>(h, ox), n, at<uint8_t>(h, oo), h->stream),
                        "quantize_q4_k_barq"));
    BARQ_HIP(hipMemcpyAsync(out, at<uint8_t>(h, oo), ob_bytes, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

size_t barq_rocm_q4_k_barq_bytes(size_t n) { return n / 256 * 136 + (n % 256 ? 8 + (n % 256 + 1) / 2 : 0); }

// ---------------------------------------------------------------------------
// MoE

namespace {

int moe_route_any(barq_rocm_handle* h, const float* logits, size_t rows, size_t n_experts, size_t top_k,
                  size_t max_active, float min_weight, int32_t* ids, float* weights, int mem, const char* what) {
    BARQ_CHECK(check_mem(mem));
    if (n_experts == 0) return fail(BARQ_E_INVALID, "Routing logits must contain at least one expert");
    if (n_experts > 256) return fail(BARQ_E_UNSUPPORTED, "%s: at most 256 experts", what);
    size_t k = top_k < 1 ? 1 : (top_k > n_experts ? n_experts : top_k);
    if (k > 64) return fail(BARQ_E_UNSUPPORTED, "%s: top_k at most 64", what);
    if (rows == 0) return ok();
    if (rows > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "%s: rows exceed 2^31", what);
    if (!logits || !ids || !weights) return fail(BARQ_E_INVALID, "%s: null buffer", what);
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE)
        return launched(barq::moe_route_launch(logits, rows, n_experts, k, ids, weights, h->stream, max_active,
                                               min_weight), what);
    Arena a;
    size_t ol = a.add(rows * n_experts * 4), oi = a.add(rows * k * 4), ow = a.add(rows * k * 4);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ol), logits, rows * n_experts * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::moe_route_launch(at<float>(h, ol), rows, n_experts, k, at<int32_t>(h, oi),
                                               at<float>(h, ow), h->stream, max_active, min_weight), what));
    BARQ_HIP(hipMemcpyAsync(ids, at<int32_t>(h, oi), rows * k * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipMemcpyAsync(weights, at<float>(h, ow), rows * k * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

}  // namespace

int barq_rocm_moe_route(barq_rocm_handle* h, const float* logits, size_t rows, size_t n_experts, size_t top_k,
                        int32_t* ids, float* weights, int mem) {
    return moe_route_any(h, logits, rows, n_experts, top_k, 0, 0.0f, ids, weights, mem, "moe_route");
}

int barq_rocm_moe_route_reduce(barq_rocm_handle* h, const float* logits, size_t rows, size_t n_experts,
                               size_t top_k, size_t max_active, float min_weight, int32_t* ids, float* weights,
                               int mem) {
    return moe_route_any(h, logits, rows, n_experts, top_k, max_active > 0 ? max_active : 1, min_weight, ids, weights,
                         mem, "moe_route_reduce");
}

int barq_rocm_moe_reduce(barq_rocm_handle* h, const int32_t* ids, const float* weights, size_t rows, size_t top_k,
                         size_t max_active, float min_weight, int32_t* out_ids, float* out_weights, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (top_k == 0) return fail(BARQ_E_INVALID, "moe_reduce: top_k must be > 0");
    if (top_k > 64) return fail(BARQ_E_UNSUPPORTED, "moe_reduce: top_k at most 64");
    if (rows == 0) return ok();
    if (rows > (size_t)INT32_MAX) return fail(BARQ_E_DIM, "moe_reduce: rows exceed 2^31");
    if (!ids || !weights || !out_ids || !out_weights) return fail(BARQ_E_INVALID, "moe_reduce: null buffer");
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE)
        return launched(barq::moe_reduce_launch(ids, weights, rows, top_k, max_active, min_weight, out_ids, out_weights,
                                                h->stream), "moe_reduce");
    const size_t nb = rows * top_k * 4;
    Arena a;
    size_t oi = a.add(nb), ow = a.add(nb);
    BARQ_CHECK(ensure_ws(h, a.used));
    BARQ_HIP(hipMemcpyAsync(at<int32_t>(h, oi), ids, nb, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ow), weights, nb, hipMemcpyHostToDevice, h->stream));
    BARQ_CHECK(launched(barq::moe_reduce_launch(at<int32_t>(h, oi), at<float>(h, ow), rows, top_k, max_active,
                                                min_weight, at<int32_t>(h, oi), at<float>(h, ow), h->stream),
                        "moe_reduce"));
    BARQ_HIP(hipMemcpyAsync(out_ids, at<int32_t>(h, oi), nb, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipMemcpyAsync(out_weights, at<float>(h, ow), nb, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

namespace {

// Device-pointer MoE FFN.  Work buffers come from one workspace arena that
// is sized up front (ensure_ws may reallocate and so runs before any use).
struct MoeArena {
    size_t off, tok, wts, pos, xg, g, u, yg, q, wf, end;
};

// K slices of the grouped down projection (each writes a partial product)
constexpr size_t MOE_DOWN_KS = 2;
// assignments (rows * k) up to which grouping and gather-quantize share a launch
constexpr size_t MOE_FUSED_GROUP_MAX = 2048;
// assignments up to which the expert projections run as grouped GEMVs
constexpr size_t MOE_GEMV_MAX_ASSIGN = 4;

MoeArena moe_arena(size_t base, size_t ne, size_t hidden, size_t n_ff, size_t na, bool q8) {
    Arena a;
    a.used = base;
    MoeArena m;
    m.off = a.add((ne + 1) * 4);
    m.tok = a.add(na * 4);
    m.wts = a.add(na * 4);
    m.pos = a.add(na * 4);
    m.xg = a.add(na * hidden * 4);
    // gate and up results are adjacent (one grouped launch writes both)
    m.g = a.add(2 * na * n_ff * 4);
    m.u = m.g + na * n_ff * 4;
    m.yg = a.add(MOE_DOWN_KS * na * hidden * 4);   // room for the K-slice partials of the down projection
    const size_t qrow = (hidden > n_ff ? hidden : n_ff) / 256 * 292;
    m.q = a.add(q8 ? na * qrow : 0);
    // the literal path dequantizes one expert matrix at a time
    m.wf = a.add(q8 ? 0 : n_ff * hidden * 4);
    m.end = a.used;
    return m;
}

int moe_ffn_dev(barq_rocm_handle* h, size_t ne, int gt, const void* const* gate, int ut, const void* const* up, int dt,
                const void* const* down, size_t hidden, size_t n_ff, const float* x, size_t rows, const int32_t* ids,
                const float* weights, size_t k, int act, float* out, size_t base) {
    hipStream_t s = h->stream;
    const size_t na = rows * k;
    const bool q8 = act == BARQ_ACT_F32_Q8;
    const MoeArena L = moe_arena(base, ne, hidden, n_ff, na, q8);
    const size_t o_off = L.off, o_tok = L.tok, o_wts = L.wts, o_pos = L.pos, o_xg = L.xg, o_g = L.g, o_u = L.u,
                 o_yg = L.yg, o_q = L.q, o_wf = L.wf;
    BARQ_CHECK(ensure_ws(h, L.end));
    int32_t* offsets = at<int32_t>(h, o_off);
    int32_t* tokens = at<int32_t>(h, o_tok);
    float* wts = at<float>(h, o_wts);
    int32_t* rowpos = at<int32_t>(h, o_pos);
    float* xg = at<float>(h, o_xg);
    float* gb = at<float>(h, o_g);
    float* ub = at<float>(h, o_u);
    float* yg = at<float>(h, o_yg);
    uint8_t* qb = at<uint8_t>(h, o_q);

    const bool device_only = q8 && q8_partner(gt) == BARQ_TYPE_Q8_K && q8_partner(ut) == BARQ_TYPE_Q8_K &&
                             q8_partner(dt) == BARQ_TYPE_Q8_K && barq::kq_supported(gt, n_ff, hidden, na) &&
                             barq::kq_supported(ut, n_ff, hidden, na) && barq::kq_supported(dt, hidden, n_ff, na);
    const bool fused_group = device_only && na <= MOE_FUSED_GROUP_MAX && barq::moe_fused_group_enabled();
    if (fused_group) {
        // grouping and the gather-quantize of the expert rows in one launch
        BARQ_CHECK(launched(barq::moe_group_gather_q8k_launch(ids, weights, rows, k, ne, x, hidden, qb, offsets, tokens,
                                                              wts, rowpos, s), "moe_group_gather"));
    } else {
        BARQ_CHECK(launched(barq::moe_group_launch(ids, weights, rows, k, ne, offsets, tokens, wts, rowpos, s), "moe_group"));
    }
    if (device_only) {
        // Device-only schedule: every kernel reads the expert row ranges from
        // `offsets`, so nothing waits for the host.  Rows past the last
        // assignment are gathered from token 0 and never read back.
        if (!fused_group)
            BARQ_CHECK(launched(barq::quantize_q8_k_gather_launch(x, tokens, na, hidden, qb, s), "quantize_act"));
        const size_t chunk = gt == ut ? 32 : 64;   // expert weight pointers per grouped launch
        std::vector<const void*> wp;
        // Single-token steps (decode): expert-grouped GEMVs, which stream each
        // used expert's weights once at GEMV speed instead of through 32-row
        // MFMA tiles (measured faster for one token only; BARQ_MOE_GEMV=2 also
        // takes them for any step of at most 4 assignments, 0 never).
        const int moe_gemv = barq::moe_gemv_enabled();
        const bool gemv_step = na <= MOE_GEMV_MAX_ASSIGN && (moe_gemv == 2 || (moe_gemv == 1 && rows == 1)) &&
                               barq::moe_gemv_supported(gt, chunk, gt == ut ? 2 : 1, n_ff, hidden) &&
                               barq::moe_gemv_supported(ut, chunk, gt == ut ? 2 : 1, n_ff, hidden) &&
                               barq::moe_gemv_supported(dt, 64, 1, hidden, n_ff);
        if (gemv_step) {
            for (size_t e0 = 0; e0 < ne; e0 += chunk) {
                const size_t c = ne - e0 < chunk ? ne - e0 : chunk;
                if (gt == ut) {
                    wp.assign(gate + e0, gate + e0 + c);
                    wp.insert(wp.end(), up + e0, up + e0 + c);
                    BARQ_CHECK(launched(barq::moe_gemv_launch(gt, wp.data(), c, 2, offsets + e0, na, rows, qb, n_ff, hidden, gb,
                                                              na * n_ff, s), "moe gate/up gemv"));
                } else {
                    BARQ_CHECK(launched(barq::moe_gemv_launch(gt, gate + e0, c, 1, offsets + e0, na, rows, qb, n_ff, hidden, gb, 0, s),
                                        "moe gate gemv"));
                    BARQ_CHECK(launched(barq::moe_gemv_launch(ut, up + e0, c, 1, offsets + e0, na, rows, qb, n_ff, hidden, ub, 0, s),
                                        "moe up gemv"));
                }
            }
            BARQ_CHECK(launched(barq::swiglu_q8_k_launch(gb, ub, na, n_ff, qb, s), "swiglu"));
            for (size_t e0 = 0; e0 < ne; e0 += 64) {
                const size_t c = ne - e0 < 64 ? ne - e0 : 64;
                BARQ_CHECK(launched(barq::moe_gemv_launch(dt, down + e0, c, 1, offsets + e0, na, rows, qb, hidden, n_ff, yg, 0, s),
                                    "moe down gemv"));
            }
            return launched(barq::moe_scatter_launch(yg, ids, weights, rowpos, rows, k, hidden, out, s, 1, 0),
                            "moe_scatter");
        }
        for (size_t e0 = 0; e0 < ne; e0 += chunk) {
            const size_t c = ne - e0 < chunk ? ne - e0 : chunk;
            if (gt == ut) {
                wp.assign(gate + e0, gate + e0 + c);
                wp.insert(wp.end(), up + e0, up + e0 + c);
                BARQ_CHECK(launched(barq::kq_grouped_launch(gt, wp.data(), c, 2, offsets + e0, na, n_ff, hidden, qb, gb,
                                                            na * n_ff, 1, 0, s), "moe gate/up"));
            } else {
                BARQ_CHECK(launched(barq::kq_grouped_launch(gt, gate + e0, c, 1, offsets + e0, na, n_ff, hidden, qb, gb,
                                                            0, 1, 0, s), "moe gate"));
                BARQ_CHECK(launched(barq::kq_grouped_launch(ut, up + e0, c, 1, offsets + e0, na, n_ff, hidden, qb, ub,
                                                            0, 1, 0, s), "moe up"));
            }
        }
        BARQ_CHECK(launched(barq::swiglu_q8_k_launch(gb, ub, na, n_ff, qb, s), "swiglu"));
        // the down projection has only hidden / 128 column tiles per expert:
        // two K slices give every CU two workgroups; the scatter adds them
        // (at most MOE_DOWN_KS partials: the arena holds that many)
        const int ovr = barq::kq_k_slices_override();
        size_t ks = ovr > 0 ? (size_t)ovr : ((n_ff / 256) % 4 == 0 && hidden / 128 * ne < 512 ? 2 : 1);
        if (ks > MOE_DOWN_KS || (n_ff / 256) % (2 * ks) != 0) ks = 1;
        for (size_t e0 = 0; e0 < ne; e0 += 64) {
            const size_t c = ne - e0 < 64 ? ne - e0 : 64;
            BARQ_CHECK(launched(barq::kq_grouped_launch(dt, down + e0, c, 1, offsets + e0, na, hidden, n_ff, qb, yg, 0, ks,
                                                        na * hidden, s), "moe down"));
        }
        return launched(barq::moe_scatter_launch(yg, ids, weights, rowpos, rows, k, hidden, out, s, (int)ks,
                                                 na * hidden), "moe_scatter");
    }
    std::vector<int32_t> off(ne + 1);
    BARQ_HIP(hipMemcpyAsync(off.data(), offsets, (ne + 1) * 4, hipMemcpyDeviceToHost, s));
    BARQ_HIP(hipStreamSynchronize(s));
    const size_t n_assign = (size_t)off[ne];
    BARQ_CHECK(launched(barq::moe_gather_launch(x, tokens, n_assign, hidden, xg, s), "moe_gather"));
    const int in_act = q8 ? q8_partner(gt) : BARQ_ACT_F32;
    if (q8) {
        if (q8_partner(gt) != BARQ_TYPE_Q8_K || q8_partner(ut) != BARQ_TYPE_Q8_K || q8_partner(dt) != BARQ_TYPE_Q8_K)
            return fail(BARQ_E_UNSUPPORTED, "moe_ffn: the Q8 path needs K-quant (Q4_K/Q6_K) expert weights");
        BARQ_CHECK(launched(barq::quantize_q8_k_launch(xg, n_assign, hidden, qb, s), "quantize_act"));
    }
    const size_t xq_row = q8 ? row_bytes_of(BARQ_TYPE_Q8_K, hidden) : hidden * 4;
    const uint8_t* xin = q8 ? qb : reinterpret_cast<const uint8_t*>(xg);
    for (size_t e = 0; e < ne; e++) {
        const size_t r0 = (size_t)off[e], c = (size_t)off[e + 1] - r0;
        if (!c) continue;
        if (q8) {
            // the arena holds this call's data from offset `base`: no workspace
            BARQ_CHECK(matmul_dev(h, gt, gate[e], n_ff, hidden, in_act, xin + r0 * xq_row, c, gb + r0 * n_ff, nullptr));
            BARQ_CHECK(matmul_dev(h, ut, up[e], n_ff, hidden, in_act, xin + r0 * xq_row, c, ub + r0 * n_ff, nullptr));
        } else {
            float* wf = at<float>(h, o_wf);
            BARQ_CHECK(launched(barq::dequant_launch(gt, gate[e], n_ff * hidden, wf, s), "dequantize"));
            BARQ_CHECK(launched(barq::gemm_f32_nt_launch(xg + r0 * hidden, wf, c, hidden, n_ff, gb + r0 * n_ff, s), "gemm_f32_nt"));
            BARQ_CHECK(launched(barq::dequant_launch(ut, up[e], n_ff * hidden, wf, s), "dequantize"));
            BARQ_CHECK(launched(barq::gemm_f32_nt_launch(xg + r0 * hidden, wf, c, hidden, n_ff, ub + r0 * n_ff, s), "gemm_f32_nt"));
        }
    }
    BARQ_CHECK(launched(barq::swiglu_launch(gb, ub, n_assign * n_ff, gb, s), "swiglu"));
    const size_t hq_row = q8 ? row_bytes_of(BARQ_TYPE_Q8_K, n_ff) : n_ff * 4;
    if (q8) BARQ_CHECK(launched(barq::quantize_q8_k_launch(gb, n_assign, n_ff, qb, s), "quantize_act"));
    const uint8_t* hin = q8 ? qb : reinterpret_cast<const uint8_t*>(gb);
    for (size_t e = 0; e < ne; e++) {
        const size_t r0 = (size_t)off[e], c = (size_t)off[e + 1] - r0;
        if (!c) continue;
        if (q8) {
            BARQ_CHECK(matmul_dev(h, dt, down[e], hidden, n_ff, in_act, hin + r0 * hq_row, c, yg + r0 * hidden, nullptr));
        } else {
            float* wf = at<float>(h, o_wf);
            BARQ_CHECK(launched(barq::dequant_launch(dt, down[e], hidden * n_ff, wf, s), "dequantize"));
            BARQ_CHECK(launched(barq::gemm_f32_nt_launch(gb + r0 * n_ff, wf, c, n_ff, hidden, yg + r0 * hidden, s), "gemm_f32_nt"));
        }
    }
    return launched(barq::moe_scatter_launch(yg, ids, weights, rowpos, rows, k, hidden, out, s), "moe_scatter");
}

}  // namespace

int barq_rocm_moe_ffn(barq_rocm_handle* h, size_t ne, int gt, const void* const* gate, int ut, const void* const* up,
                      int dt, const void* const* down, size_t hidden, size_t n_ff, const float* x, size_t rows,
                      const int32_t* ids, const float* weights, size_t k, int act, float* out, int mem) {
    BARQ_CHECK(check_mem(mem));
    if (ne == 0) return fail(BARQ_E_INVALID, "At least one expert function is required");
    if (ne > 256) return fail(BARQ_E_UNSUPPORTED, "moe_ffn: at most 256 experts");
    if (act != BARQ_ACT_F32 && act != BARQ_ACT_F32_Q8) return fail(BARQ_E_UNSUPPORTED, "moe_ffn: act must be BARQ_ACT_F32 or BARQ_ACT_F32_Q8");
    BARQ_CHECK(check_linear(gt, hidden, BARQ_ACT_F32, "moe_ffn gate"));
    BARQ_CHECK(check_linear(ut, hidden, BARQ_ACT_F32, "moe_ffn up"));
    BARQ_CHECK(check_linear(dt, n_ff, BARQ_ACT_F32, "moe_ffn down"));
    if (hidden % 4) return fail(BARQ_E_DIM, "moe_ffn: hidden must be a multiple of 4");
    if (rows == 0) return ok();
    if (k == 0) return fail(BARQ_E_INVALID, "moe_ffn: top_k must be > 0");
    if (!gate || !up || !down || !x || !ids || !weights || !out) return fail(BARQ_E_INVALID, "moe_ffn: null buffer");
    for (size_t e = 0; e < ne; e++)
        if (!gate[e] || !up[e] || !down[e]) return fail(BARQ_E_INVALID, "moe_ffn: null expert weight %zu", e);
    BARQ_CHECK(check_handle(h));
    DeviceGuard g(h);
    if (mem == BARQ_MEM_DEVICE) return moe_ffn_dev(h, ne, gt, gate, ut, up, dt, down, hidden, n_ff, x, rows, ids, weights, k, act, out, 0);
    // host buffers: stage everything into the front of the workspace
    const size_t gb = n_ff * row_bytes_of(gt, hidden), ub = n_ff * row_bytes_of(ut, hidden), db = hidden * row_bytes_of(dt, n_ff);
    Arena a;
    std::vector<size_t> og(ne), ou(ne), od(ne);
    for (size_t e = 0; e < ne; e++) { og[e] = a.add(gb); ou[e] = a.add(ub); od[e] = a.add(db); }
    const size_t ox = a.add(rows * hidden * 4), oi = a.add(rows * k * 4), ow = a.add(rows * k * 4), oo = a.add(rows * hidden * 4);
    // staging region first, then the compute region moe_ffn_dev lays out
    const MoeArena L = moe_arena(a.used, ne, hidden, n_ff, rows * k, act == BARQ_ACT_F32_Q8);
    BARQ_CHECK(ensure_ws(h, L.end));
    for (size_t e = 0; e < ne; e++) {
        BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, og[e]), gate[e], gb, hipMemcpyHostToDevice, h->stream));
        BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, ou[e]), up[e], ub, hipMemcpyHostToDevice, h->stream));
        BARQ_HIP(hipMemcpyAsync(at<uint8_t>(h, od[e]), down[e], db, hipMemcpyHostToDevice, h->stream));
    }
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ox), x, rows * hidden * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<int32_t>(h, oi), ids, rows * k * 4, hipMemcpyHostToDevice, h->stream));
    BARQ_HIP(hipMemcpyAsync(at<float>(h, ow), weights, rows * k * 4, hipMemcpyHostToDevice, h->stream));
    std::vector<const void*> dg(ne), du(ne), dd(ne);
    for (size_t e = 0; e < ne; e++) { dg[e] = at<uint8_t>(h, og[e]); du[e] = at<uint8_t>(h, ou[e]); dd[e] = at<uint8_t>(h, od[e]); }
    BARQ_CHECK(moe_ffn_dev(h, ne, gt, dg.data(), ut, du.data(), dt, dd.data(), hidden, n_ff, at<float>(h, ox), rows,
                           at<int32_t>(h, oi), at<float>(h, ow), k, act, at<float>(h, oo), a.used));
    BARQ_HIP(hipMemcpyAsync(out, at<float>(h, oo), rows * hidden * 4, hipMemcpyDeviceToHost, h->stream));
    BARQ_HIP(hipStreamSynchronize(h->stream));
    return ok();
}

}  // extern "C"
