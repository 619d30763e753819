// The experts' device data layout, and the decode expert kernels' arguments
// and launchers (shared by every kernel file through kernels.h and mfma.h).
//
// Device data layout (all of one layer resident in HBM):
//   expert weights of one role (gate, up or down) for all G = S + E groups
//   (shared experts first, then routed experts) in one allocation, rows
//   padded to kp = ceil(width/64)*64 values (zeros) and grouped in panels of
//   64 rows (rows padded to a multiple of 64 with zero rows):
//     values [G][panel][unit][64 rows][16 B]   a unit is 16 bytes of one
//                 row's codes: 16 Int8 values, 32 FP4 values (even index in
//                 the low nibble) or 4 float32 values; row_bytes / 16 units
//     scales [G][panel][kp/64][64 rows][4]     float32 per 16 values (Int8,
//                 FP4): the scales of four consecutive blocks of a row are
//                 one 16-byte group
//     biases [G][rows]                         float32
//   so one wave-wide 16-byte load (lane = row of a panel) reads 1 KiB of
//   codes contiguously, and one 16-byte scale load covers four blocks.
//   activations are fp32 (or bf16 for the MFMA path) with a row stride of
//   ceil(d/64)*64 resp. ceil(h/64)*64, padding columns zero.
//
// "Positions" number the rows the experts work on: P = T*(S+k).  Positions
// [s*T, (s+1)*T) belong to shared expert s (token = position - s*T);
// positions S*T + q for q in [0, T*k) hold the routed (token, slot) pairs in
// dispatch order (experts ascending, tokens ascending inside an expert).
// goff[G+1] holds the first position of every group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gtmoe {

enum Precision { kFloat64 = 0, kFloat32 = 1, kInt8 = 2, kFP4 = 3 };

constexpr int kValuesPerScale = 16;
constexpr int kPadK = 64;
constexpr int kPanelRows = 64;

inline int pad_k(int width) { return (width + kPadK - 1) / kPadK * kPadK; }
inline int pad_rows(int rows) { return (rows + kPanelRows - 1) / kPanelRows * kPanelRows; }

// Byte offset of 16-byte unit u of row r inside one group's codes.
__host__ __device__ inline size_t panel_unit_offset(int r, int u, int row_bytes)
{
    return (size_t)(r >> 6) * 64 * (size_t)row_bytes + (size_t)u * 1024 + (size_t)(r & 63) * 16;
}

// Index of the scale of block b of row r inside one group's scales.
__host__ __device__ inline size_t panel_scale_index(int r, int b, int nblocks)
{
    return (size_t)(r >> 6) * 64 * (size_t)nblocks + (size_t)(b >> 2) * 256 + (size_t)(r & 63) * 4 + (b & 3);
}

// One weight role of all groups on the device.
struct DeviceMatrix {
    int precision = 0;
    int rows = 0;       // output neurons
    int rows_p = 0;     // rows padded to whole panels
    int width = 0;      // inputs (unpadded)
    int kp = 0;         // padded inputs
    int row_bytes = 0;  // bytes per padded row
    int nblocks = 0;    // kp / 16
    int groups = 0;
    void *values = nullptr;
    float *scales = nullptr;
    float *biases = nullptr;
    // Float32 experts only: the rows rounded to bf16 (nearest even), in the
    // same panel layout with 8 values per 16-byte unit, for the prefill GEMM
    void *bf16 = nullptr;
    size_t group_value_bytes() const { return (size_t)rows_p * row_bytes; }
    size_t group_scales() const { return (size_t)rows_p * nblocks; }
    int bf16_row_bytes() const { return kp * 2; }
    size_t group_bf16_bytes() const { return (size_t)rows_p * bf16_row_bytes(); }
};

// Arguments of the expert GEMV kernels (fp32 path).
struct GemvArgs {
    const void *w0;
    const float *s0;
    const float *b0;
    const void *w1;  // up (gate/up kernel only)
    const float *s1;
    const float *b1;
    long long w_group_stride;  // bytes
    long long s_group_stride;  // floats
    int rows;
    int nblocks;  // kp / 16
    int row_bytes;
    const float *in;
    int ld_in;
    long long in_rows;      // rows of the input buffer (bounds its loads)
    const int32_t *tok;     // gate/up: token of every position; down: nullptr
    const int32_t *count;   // number of token slices (the rest of the grid exits)
    const int4 *desc;       // per slice: group, first position, positions, 0
    float *out;
    int ld_out;
    float clamp;
    // down only, when every output row has at most two contributions (shared
    // experts + routed slots <= 2): instead of writing slot rows, add
    // weight * row into final[token][:] (zeroed beforehand).  Two fp32 terms
    // added onto zero give the same bits in either order.
    float *final_out;        // [T][d] or nullptr
    const int32_t *tok_all;  // token of every position
    const int32_t *chosen;   // [T][k]
    const float *gates32;    // [T][k]
    int T, k, S;
    // Few tokens (self_dispatch): no dispatch tables.  Grid row y < S *
    // shared_slices is a slice of 8 tokens of a shared expert; the next 2E
    // rows are two workgroups per routed expert e (rows y and y + E), which
    // find e's (token, slot) entries in `chosen` and take every other pass
    // of 8.  Rows are indexed directly: shared expert s, token t at s*T + t;
    // routed entry t*k + j at S*T + t*k + j.  list_off: LDS offset of the
    // entry list (set by the launcher; room for T*k entries).
    int self_dispatch, shared_slices, list_off, E;
    // raw: write the bare products, no bias or activation (gate to out, up to
    // raw_up with the same layout); the adapter path's forward
    int raw;
    float *raw_up;
};

// Tokens per work slice of the GEMV path (the dispatch's tile size there).
constexpr int kGemvSlice = 8;
// Up to this many tokens the fp32 path's expert kernels find their own
// tokens in the routing choices and no dispatch launch runs.
constexpr int kSelfDispatchMaxTokens = 64;

// Launchers of the decode expert kernels (each returns the hipError_t of its launch).
hipError_t launch_gemv_gateup(const GemvArgs &a, int precision, int max_slices, hipStream_t s);
hipError_t launch_gemv_down(const GemvArgs &a, int precision, int max_slices, hipStream_t s);

}  // namespace gtmoe
