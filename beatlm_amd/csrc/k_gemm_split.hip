// The MFMA GEMM instantiated for Math::SPLIT.
#include "k_gemm.inc"

namespace bl {
hipError_t launch_gemm_split(const GemmArgs &a, int tile, hipStream_t s) { return launch_math<Math::SPLIT>(a, tile, s); }
}  // namespace bl
