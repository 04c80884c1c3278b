// The MFMA GEMM and its B packing instantiated for Math::SPLIT.
#include "k_gemm.inc"

namespace bl {
hipError_t launch_gemm_split(const GemmArgs &a, int tile, hipStream_t s) { return launch_math<Math::SPLIT>(a, tile, s); }
hipError_t launch_pack_split(const PackArgs &a, hipStream_t s) { return launch_pack<Math::SPLIT>(a, s); }
}  // namespace bl
