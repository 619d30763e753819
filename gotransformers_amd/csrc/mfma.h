// Declarations of the prefill expert kernels (grouped bf16 GEMM on the
// matrix cores) and their host-side launchers.
#pragma once

#include "common.h"

namespace gtmoe {

// Arguments of the grouped MFMA GEMM kernels (bf16 path).
struct MfmaArgs {
    const void *w0;
    const float *s0;
    const float *b0;
    const void *w1;
    const float *s1;
    const float *b1;
    long long w_group_stride;
    long long s_group_stride;
    int n;          // output rows of the weight matrix
    int kp;         // padded K
    int row_bytes;
    int nblocks;
    const uint16_t *a;  // bf16 activations
    int lda;
    long long a_rows;   // rows of the activation buffer (bounds its loads)
    const int32_t *tok;    // gate/up: gather by token; down: nullptr
    const int32_t *count;  // number of m-tiles (the rest of the grid exits)
    const int4 *desc;      // per m-tile: group, first position, positions, 0
    int ntiles_n;          // column tiles (set by the launcher)
    void *out;  // bf16: gate/up hidden rows, down slot outputs
    int ldo;
    float clamp;
};

// The bf16 copy of Float32 rows (panel layout): rows_p rows of kp values.
hipError_t launch_bf16_rows(const void *rows_f32, void *rows_bf16, int rows_p, int kp, hipStream_t s);
hipError_t launch_mfma_gateup(const MfmaArgs &a, int precision, int max_tiles, hipStream_t s);
hipError_t launch_mfma_down(const MfmaArgs &a, int precision, int max_tiles, hipStream_t s);
int mfma_tile_m();

}  // namespace gtmoe
