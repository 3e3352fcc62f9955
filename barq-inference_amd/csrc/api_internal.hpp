// Internals shared by the C ABI translation units (api.cpp, gguf.cpp,
// attention.cpp).
#pragma once
#include "../../include/barq_rocm.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "common.hpp"

struct barq_rocm_handle {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t switch_ev = nullptr;   // orders the old stream before the new one in set_stream
    void* ws = nullptr;               // device workspace, grown on demand
    size_t ws_size = 0;
    // Workspaces replaced by a larger one: kept until barq_rocm_destroy, since
    // kernels still in flight or HIP graphs captured earlier may use them.
    std::vector<void*> retired;
    barq::Tuning tuning;              // tuning overrides, read at creation
};

namespace barq_api {

// Records the thread's last error message and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int ok() { return BARQ_OK; }

#define BARQ_HIP(expr)                                                                          \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess) return barq_api::fail(BARQ_E_BACKEND, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define BARQ_CHECK(rc_expr)             \
    do {                                \
        int rc_ = (rc_expr);            \
        if (rc_ != BARQ_OK) return rc_; \
    } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Grows the handle's device workspace to at least `bytes` (at least doubling
// it; the old buffer is retired, not freed, until the handle is destroyed).
int ensure_ws(barq_rocm_handle* h, size_t bytes);

// matmul on device buffers with caller-provided scratch of ws_bytes bytes:
// no workspace growth and no allocation.  Fails with BARQ_E_UNSUPPORTED,
// before anything is enqueued, when the call needs more scratch than that.
int matmul_fixed_scratch(barq_rocm_handle* h, int w_type, const void* w, size_t n_rows, size_t k, int act_type,
                         const void* x, size_t m, float* y, void* ws, size_t ws_bytes, const char* what);

// Carves 256-byte aligned slices out of the workspace.
struct Arena {
    size_t used = 0;
    size_t add(size_t bytes) {
        const size_t off = used;
        used = round_up(used + bytes, 256);
        return off;
    }
};

template <class T>
T* at(barq_rocm_handle* h, size_t off) {
    return reinterpret_cast<T*>(static_cast<uint8_t*>(h->ws) + off);
}

inline int check_handle(barq_rocm_handle* h) {
    if (!h) return fail(BARQ_E_INVALID, "null handle");
    return ok();
}

inline int check_mem(int mem) {
    if (mem != BARQ_MEM_HOST && mem != BARQ_MEM_DEVICE) return fail(BARQ_E_INVALID, "mem must be BARQ_MEM_HOST or BARQ_MEM_DEVICE");
    return ok();
}

inline int launched(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(BARQ_E_BACKEND, "%s launch: %s", what, hipGetErrorString(e));
    return ok();
}

// Make the handle's device current for the duration of a call (and, given
// the handle, its tuning snapshot).
struct DeviceGuard {
    int prev = -1;
    bool changed = false;
    barq::TuningScope tune;
    explicit DeviceGuard(int dev, const barq::Tuning* t = nullptr) : tune(t) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) changed = hipSetDevice(dev) == hipSuccess;
    }
    explicit DeviceGuard(const barq_rocm_handle* h) : DeviceGuard(h->device, &h->tuning) {}
    ~DeviceGuard() {
        if (changed) (void)hipSetDevice(prev);
    }
};

}  // namespace barq_api

namespace barq {
// Looks up, once per device, the device address of the fixed scratch array
// behind barq_rocm_matmul_noalloc (the device must be current).
int noalloc_init(int device);
}  // namespace barq
