// The MFMA GEMM and its B packing instantiated for Math::F32.
#include "k_gemm.inc"

namespace bl {
hipError_t launch_gemm_f32(const GemmArgs &a, int tile, hipStream_t s) { return launch_math<Math::F32>(a, tile, s); }
hipError_t launch_pack_f32(const PackArgs &a, hipStream_t s) { return launch_pack<Math::F32>(a, s); }
}  // namespace bl
