// barq_rocm_matmul_noalloc: barq_rocm_matmul on device buffers for callers
// that cannot allocate (code under HIP graph capture, serving loops that
// forbid hipMalloc).  Its scratch (activation rows quantized in the call,
// the repacked rows of the 32-element-block GEMM, the K slices' partial
// products) is one fixed array per GPU instead of the handle's growable
// workspace.
#include <mutex>

#include "api_internal.hpp"

// Fixed scratch of the no-allocation matmul.  Every GPU the library runs on
// holds its own copy until the process ends.  Host code never uses this name
// as an address: it uses the per-device pointer looked up by noalloc_init.
static __device__ __align__(256) uint8_t scratch[BARQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_scratch[MAX_DEVICES];   // device address of `scratch` on each device

}  // namespace

int barq::noalloc_init(int device) {
    if (device < 0 || device >= MAX_DEVICES)
        return barq_api::fail(BARQ_E_UNSUPPORTED, "device %d: at most %d devices", device, MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_scratch[device]) return BARQ_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return barq_api::fail(BARQ_E_BACKEND, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                              hipGetErrorString(e));
    g_scratch[device] = p;
    return BARQ_OK;
}

extern "C" int barq_rocm_matmul_noalloc(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k,
                                        int act_type, const void* x, size_t m, float* y) {
    if (!h) return barq_api::fail(BARQ_E_INVALID, "null handle");
    void* p = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (h->device >= 0 && h->device < MAX_DEVICES) p = g_scratch[h->device];
    }
    if (!p) return barq_api::fail(BARQ_E_BACKEND, "matmul_noalloc: no scratch on device %d", h->device);
    return barq_api::matmul_fixed_scratch(h, w_type, w, n_rows, k, act_type, x, m, y, p,
                                          BARQ_NOALLOC_SCRATCH_BYTES, "matmul_noalloc");
}
