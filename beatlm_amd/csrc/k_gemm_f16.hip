// The MFMA GEMM and its B packing instantiated for Math::F16.
#include "k_gemm.inc"

namespace bl {
hipError_t launch_gemm_f16(const GemmArgs &a, int tile, hipStream_t s) { return launch_math<Math::F16>(a, tile, s); }
hipError_t launch_pack_f16(const PackArgs &a, hipStream_t s) { return launch_pack<Math::F16>(a, s); }
}  // namespace bl
