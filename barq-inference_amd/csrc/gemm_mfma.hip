// Batched (M >= 16) Q4_K x Q8_K GEMM on int8 MFMA.
#include "common.hpp"
#include "launch.hpp"

namespace barq {

bool gemm_mfma_supported(int, size_t, size_t) { return false; }

hipError_t gemm_q8k_mfma_launch(int, const void*, size_t, size_t, const void*, size_t, float*, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace barq
