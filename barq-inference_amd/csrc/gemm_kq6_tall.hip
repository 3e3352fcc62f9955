// The Q6_K prompt GEMM on 128 x 128 tiles: four waves, one per SIMD, each
// owning 32 weight columns and all 128 activation rows, so each weight slice's
// Q6_K decode (the costly part of this format) serves four 32 x 32 MFMA row
// tiles instead of two.  Two LDS stages (2 x 65 KB).  Built in its own
// translation unit without -amdgpu-mfma-vgpr-form, which gemm_kq.hip uses:
// with that flag the compiler rejects this instantiation at instruction
// selection (an illegal-operand error on an LDS-aperture compare).
#include "gemm_kq.hpp"

namespace barq {

hipError_t kq6_tall_launch(const KQArgs& a, hipStream_t s) { return kq_launch_t<KQ6, 128, 2, 4, false>(a, s); }

}  // namespace barq
