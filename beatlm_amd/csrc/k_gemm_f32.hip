// The MFMA GEMM instantiated for Math::F32.
#include "k_gemm.inc"

namespace bl {
hipError_t launch_gemm_f32(const GemmArgs &a, int tile, hipStream_t s) { return launch_math<Math::F32>(a, tile, s); }
}  // namespace bl
