// bf16 MFMA grouped GEMM for many tokens per expert (prefill).
#include "common.h"

namespace gtmoe {

int mfma_tile_m() { return 128; }

hipError_t launch_mfma_gateup(const MfmaArgs &, int, int, hipStream_t) { return hipErrorNotSupported; }
hipError_t launch_mfma_down(const MfmaArgs &, int, int, hipStream_t) { return hipErrorNotSupported; }

}  // namespace gtmoe
