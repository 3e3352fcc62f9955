// The HBM streaming-read floor that bench.py reports beside each one-token
// GEMV: the same bytes read once, with nothing else in the kernel.  Each
// thread reads four 16-byte chunks, every load instruction covering 4 KB of
// consecutive whole lines with the non-temporal hint (of the read patterns
// timed on MI355X for these sizes -- 1 to 16 chunks per thread, 256 or 1024
// threads, buffer->LDS copies of 2-32 KB runs per wave -- the fastest by a
// few percent); the chunks are folded with XOR and stored only when the fold
// equals a constant, so no load can be dropped.
#include "launch.hpp"

namespace barq {

typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* __restrict__ p, size_t n16,
                                                          uint32_t* __restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x;
    u32x4s v[4];
    #pragma unroll
    for (int u = 0; u < 4; u++) {
        const size_t i = base + (size_t)u * 256;
        v[u] = i < n16 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4s*>(p) + i) : u32x4s{0, 0, 0, 0};
    }
    uint32_t a = 0;
    #pragma unroll
    for (int u = 0; u < 4; u++) a ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (a == 0x9E3779B9u) sink[0] = a;
}

hipError_t stream_read_launch(const void* p, size_t bytes, uint32_t* sink, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    const size_t g = (n16 + 1023) / 1024;
    if (g > 0xFFFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)g), dim3(256), 0, s, static_cast<const uint8_t*>(p), n16,
                       sink);
    return hipGetLastError();
}

}  // namespace barq
