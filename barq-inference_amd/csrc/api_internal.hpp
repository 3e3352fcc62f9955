// Internals shared by the C ABI translation units (api.cpp, gguf.cpp).
#pragma once
#include "../../include/barq_rocm.h"

#include <hip/hip_runtime.h>

#include <cstddef>

struct barq_rocm_handle {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    void* ws = nullptr;        // device workspace, grown on demand
    size_t ws_size = 0;
};

namespace barq_api {

// Records the thread's last error message and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int ok() { return BARQ_OK; }

// Make the handle's device current for the duration of a call.
struct DeviceGuard {
    int prev = -1;
    bool changed = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) changed = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        if (changed) (void)hipSetDevice(prev);
    }
};

}  // namespace barq_api
