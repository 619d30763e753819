// Declarations of the routing, combine, adapter and helper kernels and their
// host-side launchers; includes the expert kernels' declarations.
#pragma once

#include "common.h"
#include "mfma.h"

namespace gtmoe {

// One weight role of a group set for the adapter path's transposed product
// (out[p] = sum_r in[p][r] W[r]).  tiles: (group, first position, positions).
struct RowsArgs {
    const void *values;
    const float *scales;
    long long w_group_stride;  // bytes
    long long s_group_stride;  // floats
    int rows, rows_p, kp, row_bytes, nblocks;
    const float *in;
    int ld_in;
    const int32_t *in_tok;  // unused by the transposed product (its input row is the position)
    float *out;
    int ld_out;
    const int4 *tiles;
    int tiles_positions;  // positions the tiles cover (rows of out)
};

// Low-rank adapters of one weight role over G groups (A [G][R][kin], B
// [G][rows][R], scale [G]) applied to P positions (pgroup[p]: group of p, or
// null: group 0; goff[G+1]: first position of every group).
struct LoraArgs {
    const float *A, *B, *scale;
    int R, kin, width, rows, G, P;
    const int32_t *pgroup, *goff;
    // tiles of at most lora_outer_tile_positions() positions of one group
    // (group, first position, positions, 1 if the group has more than one
    // tile else 0), every group's in position order, the first tile of
    // every group (otoff[G + 1]) and the groups of more than one tile
    const int4 *otiles;
    const int32_t *otoff;
    int notiles;
    const int32_t *omulti;
    int nomulti;
};

// Arguments of the few-token routing (input preparation and router logits in
// one launch, top-k or hash routing and the dispatch in a second).
struct FusedArgs {
    const void *x;        // input rows [T][d]: float or double
    const float *norm;    // RMSNorm weights or nullptr
    const float *w;       // router rows [E][kp] (norm folded in when norm != nullptr)
    const double *bias;   // [E]
    const double *balance;
    const int64_t *ids;   // hash routing
    int T, d, kp, E, k, S, bm;
    float *xf;            // prepared rows [T][kp] (fp32) or nullptr
    uint16_t *xb;         // prepared rows [T][kp] (bf16) or nullptr
    double *logits;       // [T][E]
    int32_t *chosen;
    double *gates;
    float *gates32;
    int32_t *load, *offsets, *rows, *pos, *goff, *tok, *tile_off;
    int4 *tile_desc;
    float *zero_out;  // [T][d] rows zeroed by the token's workgroup, or nullptr
    // The previous stack layer's combine, done here before anything else
    // (x is then float): x[t] + shared rows + gate * routed slot rows, in the
    // combine kernel's order and arithmetic, written to x_out (or in place
    // when x_out is null, allowed with one part only).
    const float *pend_slot;    // that layer's fp32 slot outputs, or nullptr: nothing pending
    const int32_t *pend_pos;   // its pos table, or nullptr: slot rows at S*T + t*k + i
    const float *pend_gates;   // [T][k]
    int pend_S, pend_k;
    float *x_out;
    // parts > 1: each token's experts are split over that many workgroups,
    // which publish their logits and count themselves in part_cnt[t] (kept
    // zero between launches); the last to arrive runs the top-k.
    int parts;
    int32_t *part_cnt;
    // read-ahead (not with hash routing): ra_blocks workgroups past the
    // routing and router-warming ones read the first ra_bytes[r] bytes
    // (multiples of 16) of ra[r] and keep nothing, so that the rows the next
    // kernel streams first are in the memory-side cache when it starts
    const void *ra[4];
    size_t ra_bytes[4];
    int ra_blocks;
    int warm_blocks;  // set by the launcher
};

// Workgroups per token of the few-token routing: more than one only for
// batches of up to kMaxSplitRouteTokens tokens and at least 64 experts.
constexpr int kMaxSplitRouteTokens = 256;
int route_fused_parts(int T, int E, bool hash);

// Launchers (each returns the hipError_t of its launch).
hipError_t launch_convert_inputs_f64(const double *x, int T, int d, float *xf, int ldf, uint16_t *xb, int ldb,
                                     hipStream_t s);
hipError_t launch_convert_inputs_f32(const float *x, int T, int d, float *xf, int ldf, uint16_t *xb, int ldb,
                                     hipStream_t s);
hipError_t launch_rmsnorm(const float *x, int T, int d, const float *w, float *xf, int ldf, uint16_t *xb, int ldb,
                          hipStream_t s);
// row_scale (optional, [T]): each row's logits are scale * dot + bias (the
// inverse RMS of a row whose norm weights are folded into w).  xb (optional,
// rows of ldb >= d bf16 values, x unpadded: ldx == d, d % 64 == 0): also
// write x as bf16, as the input conversion would.
// zero (optional): nzero ints cleared by the router kernel, for the top-k
// after it to count into (the chunked dispatch's chunk_cnt).
hipError_t launch_router(const float *x, int ldx, int T, int d, const float *w, int ldw, const double *bias, int E,
                         double *logits, hipStream_t s, const float *row_scale = nullptr, uint16_t *xb = nullptr,
                         int ldb = 0, int32_t *zero = nullptr, int nzero = 0);
// chunk_cnt (optional, zero on entry): the chunked dispatch's per-chunk
// expert counts, added up by the top-k (launch_dispatch then with counted).
hipError_t launch_topk(const double *logits, int T, int E, int k, const double *balance, int32_t *chosen,
                       double *gates, float *gates32, hipStream_t s, int32_t *chunk_cnt = nullptr);
hipError_t launch_hash_route(const int64_t *ids, int T, int E, int k, int32_t *chosen, double *gates,
                             float *gates32, hipStream_t s);
bool fused_route_fits(int T, int k, int kp);
hipError_t launch_route_fused(const FusedArgs &a, bool input_f64, bool hash, bool dispatch, hipStream_t s);
// Dispatch: one workgroup up to 1024 tokens, else (dispatch_chunked) a
// count and a placement launch over chunks of tokens using chunk_cnt
// [dispatch_chunks(T)][E]; counted: the top-k already made the counts, only
// the placement runs.
int dispatch_chunks(int T);
bool dispatch_chunked(int T);
hipError_t launch_dispatch(const int32_t *chosen, int T, int k, int E, int S, int bm, int32_t *load,
                           int32_t *offsets, int32_t *rows, int32_t *pos, int32_t *goff, int32_t *tok,
                           int32_t *tile_off, int4 *tile_desc, int32_t *chunk_cnt, hipStream_t s,
                           bool counted = false);
// The next stack layer's RMSNorm done by the combine (bf16 slot rows, d <=
// 2048, d % 8 == 0, with a residual, fp32 output of stride d): w its norm
// weights [d], xb its bf16 rows [T][ldb], inv the rows' inverse RMS [T].
struct CombineNorm {
    const float *w = nullptr;
    uint16_t *xb = nullptr;
    int ldb = 0;
    float *inv = nullptr;
};
bool combine_norm_fits(int d, bool slot_bf16);
hipError_t launch_combine(int T, int d, int S, int k, const void *slot_out, bool slot_bf16, const int32_t *pos,
                          const float *gates32, const float *residual, float *out32, double *out64, hipStream_t s,
                          const CombineNorm &norm = CombineNorm{});
hipError_t launch_fill_i32(int32_t *p, int n, int32_t v, hipStream_t s);
// Up to kMax device arrays of 4-byte words copied one after the other into
// dst, each part starting at a multiple of 16 words.
struct PackParts {
    static constexpr int kMax = 6;
    const uint32_t *src[kMax];
    int words[kMax];
    int n;
};
hipError_t launch_pack_words(const PackParts &p, uint32_t *dst, hipStream_t s);
// The one-workgroup dispatch (T <= 1024) followed, in the same launch, by the
// gathering of p into dst that launch_pack_words does.
hipError_t launch_dispatch_packed(const int32_t *chosen, int T, int k, int E, int S, int bm, int32_t *load,
                                  int32_t *offsets, int32_t *rows, int32_t *pos, int32_t *goff, int32_t *tok,
                                  int32_t *tile_off, int4 *tile_desc, const PackParts &p, uint32_t *dst,
                                  hipStream_t s);
hipError_t launch_f32_to_f64(const float *x, double *y, long long n, hipStream_t s);

// Adapter path (lora.hip, route.hip).
// out = in W over `chunks` row chunks; partial: chunks * positions * ld_out
// floats of scratch when chunks > 1
hipError_t launch_rows_transposed(const RowsArgs &a, int precision, int ntiles, int tile, int chunks, float *partial,
                                  hipStream_t s);
int rows_transposed_tile(int positions, int groups);
// smallest row chunk worth a workgroup of its own, and workgroups across the
// columns, for tiles of `tile` positions
int rows_transposed_chunk_rows(int tile);
int rows_transposed_colblocks(int nblocks, int tile);
hipError_t launch_lora_down(const LoraArgs &a, const float *in, int ld_in, const int32_t *in_tok, float *u,
                            hipStream_t s);
hipError_t launch_lora_up_bias(const LoraArgs &a, const float *u, float *out, int ld_out, const float *bias,
                               hipStream_t s);
hipError_t launch_lora_up_bias_f64(const LoraArgs &a, const float *u, double *out, int ld_out, const double *bias,
                                   hipStream_t s);
// scratch: a.notiles * a.R * max(a.rows, a.width) floats (unused when no
// group has more than one tile)
hipError_t launch_lora_backward(const LoraArgs &a, const float *grad, int ld_g, const float *u, const float *in,
                                int ld_in, const int32_t *in_tok, float *t, float *dx, int ld_dx, double *dA,
                                double *dB, float *scratch, hipStream_t s);
int lora_outer_tile_positions();
hipError_t launch_swiglu_forward(const float *gpre, const float *upre, int P, int h, int hp, float limit,
                                 float *hidden, hipStream_t s);
hipError_t launch_swiglu_backward(const float *hgrad, const float *gpre, const float *upre, int P, int h, int hp,
                                  float limit, float *ggrad, float *ugrad, hipStream_t s);
hipError_t launch_expert_output_grad(const double *og, int d, int ld, const int32_t *tok, const int32_t *pgroup,
                                     int S, int T, int k, const int32_t *chosen, const double *gates, int P,
                                     float *eg, hipStream_t s);
hipError_t launch_gather_input_grad(const float *dxg, const float *dxu, int ld, int d, int T, int S, int k,
                                    const int32_t *pos, double *dx, hipStream_t s);
hipError_t launch_router_input_grad(const float *lg, int T, int E, const float *w, int ldw, int d, float *dx,
                                    int ld_dx, hipStream_t s);
hipError_t launch_add_rows_f64(const float *src, int ld, int d, int T, double *dst, hipStream_t s);
// Router logit gradients (mixtureofexperts.go:262-282): lg [T][E] float64
// and fp32 copy, zero for the experts a token did not choose.
hipError_t launch_router_backward(const double *og, int d, const float *expert_out, int ld_out,
                                  const int32_t *chosen, const double *gates, const double *logits,
                                  const int32_t *pos, int S, int T, int E, int k, double *lg, float *lgf,
                                  hipStream_t s);
}  // namespace gtmoe
