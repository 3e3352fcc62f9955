// f32 BLAS arms of barq_core::blas (blas.rs:103-304) for callers that keep
// f32 weights, and the f32 contraction behind the literal (f32-activation)
// matmul and the split-scale quantized_matmul.
//
// The reference sums every output sequentially in k order with unfused
// multiply and add (blas.rs:202-210, 295-301).  These kernels keep that
// order per output and compile with -ffp-contract=off, so their results are
// bit-identical to the reference's CPU fallback, not merely close.
#include "common.hpp"
#include "launch.hpp"

namespace barq {

constexpr int GT = 64;   // output tile
constexpr int GK = 16;   // k tile

// C[m x n] = A[m x k] * B, B is [k x n] (BT = false) or [n x k] (BT = true).
template <bool BT>
__global__ __launch_bounds__(256) void gemm_f32_seq_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                           float* __restrict__ C, int m, int k, int n) {
    __shared__ float As[GK][GT + 1];
    __shared__ float Bs[GK][GT + 1];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int row0 = blockIdx.y * GT, col0 = blockIdx.x * GT;
    float acc[4][4];
    #pragma unroll
    for (int i = 0; i < 4; i++)
        #pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;

    for (int k0 = 0; k0 < k; k0 += GK) {
        const int kt = min(GK, k - k0);
        #pragma unroll
        for (int t = 0; t < 4; t++) {
            const int idx = tid + 256 * t;       // 0..1023
            const int r = idx >> 4, kk = idx & 15;
            const int gr = row0 + r, gk = k0 + kk;
            As[kk][r] = (gr < m && kk < kt) ? A[(size_t)gr * k + gk] : 0.0f;
            if (BT) {
                const int gc = col0 + r;
                Bs[kk][r] = (gc < n && kk < kt) ? B[(size_t)gc * k + gk] : 0.0f;
            } else {
                const int c = idx & 63, kb = idx >> 6;
                const int gc = col0 + c, gkb = k0 + kb;
                Bs[kb][c] = (gc < n && kb < kt) ? B[(size_t)gkb * n + gc] : 0.0f;
            }
        }
        __syncthreads();
        for (int kk = 0; kk < kt; kk++) {
            float a[4], b[4];
            #pragma unroll
            for (int i = 0; i < 4; i++) a[i] = As[kk][ty + 16 * i];
            #pragma unroll
            for (int j = 0; j < 4; j++) b[j] = Bs[kk][tx + 16 * j];
            #pragma unroll
            for (int i = 0; i < 4; i++)
                #pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float p = a[i] * b[j];
                    acc[i][j] = acc[i][j] + p;
                }
        }
        __syncthreads();
    }
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        const int gr = row0 + ty + 16 * i;
        if (gr >= m) continue;
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gc = col0 + tx + 16 * j;
            if (gc < n) C[(size_t)gr * n + gc] = acc[i][j];
        }
    }
}

// y[i] = sum_j a[i*n+j] * x[j], one thread per row, sequential in j.
__global__ __launch_bounds__(256) void gemv_f32_seq_kernel(const float* __restrict__ a, const float* __restrict__ x,
                                                           float* __restrict__ y, int m, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m) return;
    const float* row = a + (size_t)i * n;
    float sum = 0.0f;
    const bool vec = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0) && ((reinterpret_cast<uintptr_t>(x) & 15u) == 0);
    int j = 0;
    if (vec) {
        for (; j + 4 <= n; j += 4) {
            const float4 av = *reinterpret_cast<const float4*>(row + j);
            const float4 xv = *reinterpret_cast<const float4*>(x + j);
            float p;
            p = av.x * xv.x; sum = sum + p;
            p = av.y * xv.y; sum = sum + p;
            p = av.z * xv.z; sum = sum + p;
            p = av.w * xv.w; sum = sum + p;
        }
    }
    for (; j < n; j++) {
        const float p = row[j] * x[j];
        sum = sum + p;
    }
    y[i] = sum;
}

hipError_t gemm_f32_launch(const float* a, const float* b, size_t m, size_t k, size_t n, float* c,
                           hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + GT - 1) / GT), (unsigned)((m + GT - 1) / GT));
    hipLaunchKernelGGL(gemm_f32_seq_kernel<false>, grid, dim3(256), 0, s, a, b, c, (int)m, (int)k, (int)n);
    return hipGetLastError();
}

hipError_t gemm_f32_nt_launch(const float* a, const float* b_nk, size_t m, size_t k, size_t n, float* c,
                              hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + GT - 1) / GT), (unsigned)((m + GT - 1) / GT));
    hipLaunchKernelGGL(gemm_f32_seq_kernel<true>, grid, dim3(256), 0, s, a, b_nk, c, (int)m, (int)k, (int)n);
    return hipGetLastError();
}

hipError_t gemv_f32_plain_launch(const float* a, const float* x, size_t m, size_t n, float* y,
                                 hipStream_t s) {
    if (m == 0) return hipSuccess;
    hipLaunchKernelGGL(gemv_f32_seq_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, a, x, y,
                       (int)m, (int)n);
    return hipGetLastError();
}

}  // namespace barq
