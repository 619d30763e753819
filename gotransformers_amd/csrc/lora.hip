// Kernels of the adapter path: a forward that keeps what the backward needs,
// and the backward of a mixture whose layers carry low-rank adapters over
// frozen (compressed) weights.
//
//   Layer.Forward with an adapter (perceptron/layer.go:133-162,
//   adapter.go:66-76):  pre = (x W^T + s (x A^T) B^T) + b,  s = alpha / rank
//   (x W^T comes from the decode GEMV kernels in their raw mode)
//   Layer.Backward, base frozen (layer.go:164-210, adapter.go:78-99):
//     dB += s g^T u      (u = x A^T, kept by the forward)
//     t   = s g B
//     dA += t^T x
//     dx  = g W + t A    (g W row by row is Rows.AddScaledRowTo,
//                         lowprecision/rows.go:285-324)
//
// Work is numbered by positions as in the expert kernels: P = T*(S+k), shared
// expert s on positions [s*T, (s+1)*T), the routed (token, slot) pairs after
// them in dispatch order; pgroup[p] is the group of position p, goff[G+1]
// the first position of every group.  A position's input row is in_tok[p]
// (gate/up: the token) or p itself (down: the hidden row) when in_tok is null.
//
// Adapter storage per weight role, all groups in one allocation, zero beyond
// a layer's rank and beyond its widths (so the padding adds nothing):
//   A [G][R][kin] fp32 (Down of the reference, rank x inputs)
//   B [G][rows][R] fp32 (Up, outputs x rank)
//   dA, dB as float64 accumulators of the same shapes (the reference's
//   DownGradients / UpGradients), scale[G] fp32.
// Everything runs in fp32 with the reference's operation order where it has
// one (block sums of a row times the block scale, bias after the adapter).
#include "kernels.h"

namespace gtmoe {

namespace {

constexpr int kTrRows = 128;  // gradient rows staged per step

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// out[p][i] = sum_r grad[p][r] * W[r][i] for the group's rows r: the
// reference's Rows.AddScaledRowTo over every row with scale grad[p][r]
// (target_i += (grad * blockScale) * value).  Lane = one block of 16 columns
// (blockIdx.x * 64 + lane), the TILE positions of tile blockIdx.y, rows
// [blockIdx.z * chunk_rows, +chunk_rows).  The four waves take a quarter of
// every staged run of rows each and request kTrBatch rows' codes and scales
// before their arithmetic (enough bytes in flight to stream the rows at
// decode sizes); their partial sums are added in wave order through LDS.
// With more than one row chunk each writes its partial sums to
// partial[blockIdx.z] (same layout as out) and sum_chunks_kernel adds them
// in chunk order.  Every column of the padded width is written (zero past
// the matrix).
template <int PREC>
__device__ __forceinline__ void load_block_raw(const char *codes, int r, int b, int row_bytes, uint4 (&q)[PREC == kFloat32 ? 4 : 1])
{
    if constexpr (PREC == kInt8) {
        q[0] = *reinterpret_cast<const uint4 *>(codes + panel_unit_offset(r, b, row_bytes));
    } else if constexpr (PREC == kFP4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(codes + panel_unit_offset(r, b >> 1, row_bytes) + 8 * (b & 1));
        q[0] = make_uint4(v.x, v.y, 0u, 0u);
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) q[u] = *reinterpret_cast<const uint4 *>(codes + panel_unit_offset(r, 4 * b + u, row_bytes));
    }
}

template <int PREC>
__device__ __forceinline__ void decode_block(const uint4 (&q)[PREC == kFloat32 ? 4 : 1], float (&w)[16])
{
    if constexpr (PREC == kInt8) {
        const uint32_t d[4] = {q[0].x, q[0].y, q[0].z, q[0].w};
#pragma unroll
        for (int v = 0; v < 16; ++v) w[v] = (float)(int8_t)(d[v >> 2] >> (8 * (v & 3)));
    } else if constexpr (PREC == kFP4) {
        // e2m1 pairs, even value in the low nibble; the conversion's scale
        // operand stays 1.0 (it only takes a power of two)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t d = u ? q[0].y : q[0].x;
            const f32x2 f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
            const f32x2 f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
            const f32x2 f2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
            const f32x2 f3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
            w[8 * u] = f0[0];
            w[8 * u + 1] = f0[1];
            w[8 * u + 2] = f1[0];
            w[8 * u + 3] = f1[1];
            w[8 * u + 4] = f2[0];
            w[8 * u + 5] = f2[1];
            w[8 * u + 6] = f3[0];
            w[8 * u + 7] = f3[1];
        }
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            w[4 * u] = __uint_as_float(q[u].x);
            w[4 * u + 1] = __uint_as_float(q[u].y);
            w[4 * u + 2] = __uint_as_float(q[u].z);
            w[4 * u + 3] = __uint_as_float(q[u].w);
        }
    }
}

constexpr int kTrWaves = 4;
constexpr int kTrBatch = 8;

template <int PREC, int TILE>
__global__ __launch_bounds__(64 * kTrWaves) void rows_transposed_kernel(RowsArgs a, int chunk_rows,
                                                                        float *__restrict__ partial,
                                                                        long long partial_stride)
{
    __shared__ float gs[TILE][kTrRows];
    __shared__ float red[kTrWaves - 1][16][64];
    const int4 td = a.tiles[blockIdx.y];
    const int g = td.x, p0 = td.y, m = td.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.x * 64 + lane;  // block of 16 columns
    const bool live = b < a.nblocks;
    const int bl = live ? b : 0;  // loads of dead lanes stay in bounds and are not used
    const char *codes = reinterpret_cast<const char *>(a.values) + (size_t)g * a.w_group_stride;
    const float *sc = a.scales + (size_t)g * a.s_group_stride;
    float acc[TILE][16];
#pragma unroll
    for (int q = 0; q < TILE; ++q)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[q][v] = 0.f;
    const int nbeg = blockIdx.z * chunk_rows, nend = min(a.rows, nbeg + chunk_rows);
    for (int n0 = nbeg; n0 < nend; n0 += kTrRows) {
        __syncthreads();
        for (int idx = threadIdx.x; idx < TILE * kTrRows; idx += 64 * kTrWaves) {
            const int q = idx / kTrRows, c = idx - q * kTrRows;
            gs[q][c] = q < m && n0 + c < nend ? a.in[(size_t)(p0 + q) * a.ld_in + n0 + c] : 0.f;
        }
        __syncthreads();
        const int nn = min(kTrRows, nend - n0);
        const int ca = wave * nn / kTrWaves, cb = (wave + 1) * nn / kTrWaves;
        for (int c0 = ca; c0 < cb; c0 += kTrBatch) {
            uint4 q[kTrBatch][PREC == kFloat32 ? 4 : 1];
            float s[kTrBatch];
#pragma unroll
            for (int u = 0; u < kTrBatch; ++u) {
                const int r = n0 + min(c0 + u, cb - 1);
                load_block_raw<PREC>(codes, r, bl, a.row_bytes, q[u]);
                s[u] = PREC == kFloat32 ? 1.f : sc[panel_scale_index(r, bl, a.nblocks)];
            }
#pragma unroll
            for (int u = 0; u < kTrBatch; ++u) {
                if (c0 + u >= cb) break;  // wave-uniform
                float w[16];
                decode_block<PREC>(q[u], w);
#pragma unroll
                for (int qq = 0; qq < TILE; ++qq) {
                    const float cs = PREC == kFloat32 ? gs[qq][c0 + u] : gs[qq][c0 + u] * s[u];
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[qq][v] = fmaf(cs, w[v], acc[qq][v]);
                }
            }
        }
    }
    // add the waves' partial sums in wave order, one position at a time
    float *dst = gridDim.z == 1 ? a.out : partial + (size_t)blockIdx.z * partial_stride;
    for (int qq = 0; qq < TILE; ++qq) {
        __syncthreads();
        if (wave > 0) {
#pragma unroll
            for (int v = 0; v < 16; ++v) red[wave - 1][v][lane] = acc[qq][v];
        }
        __syncthreads();
        if (wave == 0 && live && qq < m) {
            float o[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                float t = acc[qq][v];
#pragma unroll
                for (int w2 = 0; w2 < kTrWaves - 1; ++w2) t += red[w2][v][lane];
                o[v] = t;
            }
            float4 *out = reinterpret_cast<float4 *>(dst + (size_t)(p0 + qq) * a.ld_out + 16 * b);
#pragma unroll
            for (int u = 0; u < 4; ++u) out[u] = make_float4(o[4 * u], o[4 * u + 1], o[4 * u + 2], o[4 * u + 3]);
        }
    }
}

// The same product on the matrix cores, for groups of many positions:
// out = G W with G the [positions][rows] gradients and W the group's
// dequantized rows, as fp32 16x16x4 MFMAs (the products keep fp32 operands;
// the only difference from the lane kernel is the summation order and that
// the block scale multiplies the weight, (scale * value), before the
// gradient does).  A workgroup takes kMtPositions positions of one tile,
// kMtBlocks 16-column blocks and the rows [blockIdx.z * chunk_rows,
// +chunk_rows) in steps of one 64-row panel: the block's codes and scales
// are dequantized once into LDS as [column][row] and the gradients staged as
// [position][row], so every lane reads four consecutive rows of its column
// or position with one 16-byte LDS read (the four k of four MFMAs).  Wave w
// owns blocks 2w and 2w+1 for all the positions: 2 x 2 accumulator tiles.
// The next panel's loads are issued before the current panel's MFMAs.
// Rows past the chunk and positions past the tile are staged as zeros.
constexpr int kMtPositions = 32;
constexpr int kMtBlocks = 8;
constexpr int kMtRows = 64;
constexpr int kMtPitch = kMtRows + 4;  // floats; a 16-lane b128 read then touches every bank once

template <int PREC>
__global__ __launch_bounds__(256) void rows_transposed_mfma_kernel(RowsArgs a, int chunk_rows,
                                                                   float *__restrict__ partial,
                                                                   long long partial_stride)
{
    __shared__ __attribute__((aligned(16))) float bs[kMtBlocks * 16][kMtPitch];
    __shared__ __attribute__((aligned(16))) float as[kMtPositions][kMtPitch];
    const int4 td = a.tiles[blockIdx.y];
    const int g = td.x, p0 = td.y, m = td.z;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b0 = blockIdx.x * kMtBlocks;
    const char *codes = reinterpret_cast<const char *>(a.values) + (size_t)g * a.w_group_stride;
    const float *sc = a.scales + (size_t)g * a.s_group_stride;
    const int nbeg = blockIdx.z * chunk_rows, nend = min(a.rows, nbeg + chunk_rows);

    // staging registers of thread (wave, lane): row n0 + lane of blocks
    // b0 + wave + 4 j (j < 2), and row n0 + lane of positions wave + 4 j
    // (j < 8).  Loads are unconditional at clamped indices (the panel's rows
    // past the chunk repeat its last row), and what lies outside is zeroed
    // after the load: the gradients always, the weights through a zero scale
    // (their values are then finite) or, for fp32 rows, directly.
    uint4 q[2][PREC == kFloat32 ? 4 : 1];
    float s[2], x[8];
    bool ok[2];
    auto fetch = [&](int n0) {
        const int rr = min(lane, nend - 1 - n0);  // row inside the panel
        const bool row_ok = n0 + lane < nend;
        const char *pc = codes + (size_t)(n0 >> 6) * 64 * a.row_bytes;
        const float *ps = sc + (size_t)(n0 >> 6) * 64 * a.nblocks;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int b = min(b0 + wave + 4 * j, a.nblocks - 1);
            ok[j] = row_ok && b0 + wave + 4 * j < a.nblocks;
            if constexpr (PREC == kInt8) {
                q[j][0] = *reinterpret_cast<const uint4 *>(pc + (size_t)b * 1024 + rr * 16);
            } else if constexpr (PREC == kFP4) {
                const uint2 v = *reinterpret_cast<const uint2 *>(pc + (size_t)(b >> 1) * 1024 + rr * 16 + 8 * (b & 1));
                q[j][0] = make_uint4(v.x, v.y, 0u, 0u);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    q[j][u] = *reinterpret_cast<const uint4 *>(pc + (size_t)(4 * b + u) * 1024 + rr * 16);
            }
            if constexpr (PREC != kFloat32) {
                const float v = ps[(b >> 2) * 256 + rr * 4 + (b & 3)];
                s[j] = ok[j] ? v : 0.f;
            }
        }
        const float *col = a.in + n0 + rr;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int qq = wave + 4 * j;
            const float v = col[(size_t)(p0 + min(qq, m - 1)) * a.ld_in];
            x[j] = row_ok && qq < m ? v : 0.f;
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int bb = wave + 4 * j;
            float w[16];
            decode_block<PREC>(q[j], w);
#pragma unroll
            for (int v = 0; v < 16; ++v)
                bs[bb * 16 + v][lane] = PREC == kFloat32 ? (ok[j] ? w[v] : 0.f) : s[j] * w[v];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) as[wave + 4 * j][lane] = x[j];
    };

    const int li = lane & 15, kg = lane >> 4;
    f32x4 acc[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nbeg < nend) fetch(nbeg);
    for (int n0 = nbeg; n0 < nend; n0 += kMtRows) {
        __syncthreads();
        stage();
        __syncthreads();
        if (n0 + kMtRows < nend) fetch(n0 + kMtRows);
        const int steps = min(kMtRows, nend - n0 + 15) >> 4;
        for (int st = 0; st < steps; ++st) {
            const int c = 16 * st + 4 * kg;
            f32x4 av[2], bv[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) av[mt] = *reinterpret_cast<const f32x4 *>(&as[16 * mt + li][c]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                bv[nt] = *reinterpret_cast<const f32x4 *>(&bs[16 * (2 * wave + nt) + li][c]);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt][e], bv[nt][e], acc[mt][nt], 0, 0, 0);
        }
    }
    // accumulator register v of lane l: position 4 (l / 16) + v of the
    // 16-position tile, column l % 16 of the block
    float *dst = gridDim.z == 1 ? a.out : partial + (size_t)blockIdx.z * partial_stride;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int b = b0 + 2 * wave + nt;
        if (b >= a.nblocks) continue;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int qq = 16 * mt + 4 * kg + v;
                if (qq < m) dst[(size_t)(p0 + qq) * a.ld_out + 16 * b + li] = acc[mt][nt][v];
            }
    }
}

// out[p][i] = sum over chunks c (in order) of partial[c][p][i], i < cols
__global__ __launch_bounds__(256) void sum_chunks_kernel(const float *__restrict__ partial, long long stride,
                                                         int chunks, int cols, int ld, float *__restrict__ out)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const size_t o = (size_t)blockIdx.y * ld + i;
    if (i >= cols) return;
    float s = partial[o];
    for (int c = 1; c < chunks; ++c) s += partial[(size_t)c * stride + o];
    out[o] = s;
}

__device__ __forceinline__ float wave_sum(float v)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// u[p][j] = sum_i in[row(p)][i] * A[g(p)][j][i]; one wave per (position,
// rank j).  Rows are read as float4 runs over the padded width kin (zeros
// past the width in both operands); the loads are unconditional (clamped
// index, masked sum) so the compiler keeps them all in flight.
__global__ __launch_bounds__(256) void lora_down_kernel(LoraArgs a, const float *__restrict__ in, int ld_in,
                                                        const int32_t *__restrict__ in_tok, float *__restrict__ u)
{
    const int lane = threadIdx.x & 63;
    const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wv >= a.P * a.R) return;  // wave-uniform
    const int p = wv / a.R, j = wv - p * a.R;
    const int g = a.pgroup ? a.pgroup[p] : 0;
    const int row = in_tok ? in_tok[p] : p;
    const float4 *x = reinterpret_cast<const float4 *>(in + (size_t)row * ld_in);
    const float4 *A = reinterpret_cast<const float4 *>(a.A + ((size_t)g * a.R + j) * a.kin);
    const int n4 = a.kin / 4;
    float s = 0.f;
#pragma unroll 4
    for (int i = lane; i < n4 + 63; i += 64) {
        const int c = min(i, n4 - 1);
        const float4 xv = x[c], av = A[c];
        const float d = xv.x * av.x + xv.y * av.y + xv.z * av.z + xv.w * av.w;
        s += i < n4 ? d : 0.f;
    }
    s = wave_sum(s);
    if (lane == 0) u[(size_t)p * a.R + j] = s;
}

// out[p][n] = (out[p][n] + scale[g] * sum_j B[g][n][j] u[p][j]) + bias[n]
// for n < rows (the reference adds the adapter, then the bias).
template <typename OutT>
__global__ __launch_bounds__(256) void lora_up_bias_kernel(LoraArgs a, const float *__restrict__ u,
                                                           OutT *__restrict__ out, int ld_out,
                                                           const float *__restrict__ bias32,
                                                           const double *__restrict__ bias64)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int p = blockIdx.y;
    if (n >= a.rows) return;
    const int g = a.pgroup ? a.pgroup[p] : 0;
    const float *B = a.B + ((size_t)g * a.rows + n) * a.R;
    const float *up = u + (size_t)p * a.R;
    float s = 0.f;
    if ((a.R & 3) == 0) {  // the row's ranks as float4 runs (rows are 16-byte aligned)
        for (int j = 0; j < a.R; j += 4) {
            const float4 b4 = *reinterpret_cast<const float4 *>(B + j);
            s = fmaf(b4.x, up[j], s);
            s = fmaf(b4.y, up[j + 1], s);
            s = fmaf(b4.z, up[j + 2], s);
            s = fmaf(b4.w, up[j + 3], s);
        }
    } else {
        for (int j = 0; j < a.R; ++j) s = fmaf(B[j], up[j], s);
    }
    OutT &o = out[(size_t)p * ld_out + n];
    if constexpr (sizeof(OutT) == 8) {
        o = (o + (double)(a.scale[g] * s)) + bias64[n];
    } else {
        o = (o + a.scale[g] * s) + bias32[(size_t)g * a.rows + n];
    }
}

// The adapter gradients are sums over each group's positions of outer
// products: dB[g] += scale[g] * grad^T u and dA[g] += t^T in.
// lora_outer_kernel sums one tile of at most kOpPositions positions of a
// group (tiles from the host, in position order):
//   sum over the tile's p of U[p][j] * V[row(p)][c]
// for 16 ranks j (chunk blockIdx.z) and 64 columns c (blockIdx.x).  The
// tile's 16 ranks of U are staged in LDS (read back as wave-uniform
// broadcasts), wave w takes positions p0 + w + 4 i with all sixteen of its
// V loads issued together, every lane keeps one column's 16 rank sums, and
// the four waves' sums are added in wave order through LDS.  A group of one
// tile (descriptor .w == 0) adds its sums to the float64 accumulator
// directly (each output has one writer); the tiles of larger groups write
// partial[tile][j][c] and lora_tiles_sum_kernel adds them in tile order, in
// float64, to the accumulator.
constexpr int kOpPositions = 64;

struct OuterArgs {
    const int4 *tiles;
    const float *U;  // [positions][R]
    int R;
    const float *V;  // rows ld_v apart
    int ld_v;
    const int32_t *v_row;  // V's row of every position, or null for the position itself
    int width;             // columns c
    float *partial;        // [tiles][R][width] sums of the tiles of groups with more than one
    const float *scale;    // factor of group g, or null for 1
    double *dst;           // dst[g * gs + j * js + c * cs]
    long long gs, js, cs;
};

__global__ __launch_bounds__(256) void lora_outer_kernel(OuterArgs a)
{
    __shared__ float red[4][16][64];
    __shared__ __attribute__((aligned(16))) float us[kOpPositions][16];
    const int4 td = a.tiles[blockIdx.y];
    const int g = td.x, p0 = td.y, m = td.z;
    const int R = a.R, width = a.width;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = blockIdx.x * 64 + lane, cc = min(c, width - 1);
    const int j0 = blockIdx.z * 16;
    // U rows of the tile, zero past the tile and past the rank (loads at
    // clamped indices, all in flight together)
    float uv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = threadIdx.x + 256 * e, q = i >> 4, jj = i & 15;
        uv[e] = a.U[(size_t)(p0 + min(q, m - 1)) * R + min(j0 + jj, R - 1)];
        if (q >= m || j0 + jj >= R) uv[e] = 0.f;
    }
    int row[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) row[i] = p0 + min(wave + 4 * i, m - 1);
    if (a.v_row) {
#pragma unroll
        for (int i = 0; i < 16; ++i) row[i] = a.v_row[row[i]];
    }
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = a.V[(size_t)row[i] * a.ld_v + cc];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = threadIdx.x + 256 * e;
        us[i >> 4][i & 15] = uv[e];
    }
    __syncthreads();
    float acc[16];
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) acc[jj] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (wave + 4 * i >= m) break;  // wave-uniform; positions past the tile add nothing
        const float4 *u4 = reinterpret_cast<const float4 *>(us[wave + 4 * i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float4 u = u4[e];
            acc[4 * e] = fmaf(u.x, v[i], acc[4 * e]);
            acc[4 * e + 1] = fmaf(u.y, v[i], acc[4 * e + 1]);
            acc[4 * e + 2] = fmaf(u.z, v[i], acc[4 * e + 2]);
            acc[4 * e + 3] = fmaf(u.w, v[i], acc[4 * e + 3]);
        }
    }
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) red[wave][jj][lane] = acc[jj];
    __syncthreads();
    // wave w finishes ranks 4 w .. 4 w + 3
    if (c >= width) return;
    const double f = td.w == 0 && a.scale ? (double)a.scale[g] : 1.0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int jj = 4 * wave + e;
        if (j0 + jj >= R) break;
        const float t = ((red[0][jj][lane] + red[1][jj][lane]) + red[2][jj][lane]) + red[3][jj][lane];
        if (td.w)
            a.partial[((size_t)blockIdx.y * R + j0 + jj) * width + c] = t;
        else
            a.dst[(size_t)g * a.gs + (size_t)(j0 + jj) * a.js + (size_t)c * a.cs] += f * (double)t;
    }
}

// dst[g][j][c] (strides gs, js, cs) += factor * sum over the tiles
// [toff[g], toff[g+1]) in order of partial[tile][j][c], factor = scale[g]
// (or 1 without scales), for the groups g = multi[blockIdx.z]
__global__ __launch_bounds__(256) void lora_tiles_sum_kernel(OuterArgs a, const int32_t *__restrict__ toff,
                                                             const int32_t *__restrict__ multi)
{
    const int c = blockIdx.x * 256 + threadIdx.x, j = blockIdx.y, g = multi[blockIdx.z];
    if (c >= a.width) return;
    double sum = 0.0;
    for (int t = toff[g]; t < toff[g + 1]; ++t) sum += (double)a.partial[((size_t)t * a.R + j) * a.width + c];
    if (a.scale) sum *= (double)a.scale[g];
    a.dst[(size_t)g * a.gs + (size_t)j * a.js + (size_t)c * a.cs] += sum;
}

// dst += the sums of `o` over every group's tiles
void launch_outer(OuterArgs o, const LoraArgs &a, float *scratch, hipStream_t s)
{
    o.partial = scratch;
    hipLaunchKernelGGL(lora_outer_kernel, dim3((o.width + 63) / 64, a.notiles, (o.R + 15) / 16), dim3(256), 0, s, o);
    if (a.nomulti > 0)
        hipLaunchKernelGGL(lora_tiles_sum_kernel, dim3((o.width + 255) / 256, o.R, a.nomulti), dim3(256), 0, s, o,
                           a.otoff, a.omulti);
}

// t[p][j] = scale[g] * sum_n grad[p][n] * B[g][n][j]; one workgroup per
// position and 16 ranks: lane l of wave w takes rows n = 64 (4 i + w) + l,
// reading the gradient once and each row's 16 ranks of B as contiguous
// float4 runs; each wave adds its lanes' partial sums, and the four waves'
// sums are added in wave order through LDS.
constexpr int kTRanks = 16;

__global__ __launch_bounds__(256) void lora_t_kernel(LoraArgs a, const float *__restrict__ grad, int ld_g,
                                                     float *__restrict__ t)
{
    __shared__ float part[4][kTRanks];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nj = (a.R + kTRanks - 1) / kTRanks;
    const int p = blockIdx.x / nj, j0 = (blockIdx.x - p * nj) * kTRanks;
    const int g = a.pgroup ? a.pgroup[p] : 0;
    const float *gr = grad + (size_t)p * ld_g;
    const float *B = a.B + (size_t)g * a.rows * a.R;
    const bool vec = (a.R & 3) == 0 && j0 + kTRanks <= a.R;
    float s[kTRanks];
#pragma unroll
    for (int j = 0; j < kTRanks; ++j) s[j] = 0.f;
#pragma unroll 2
    for (int n = 64 * wave + lane; n < a.rows; n += 256) {
        const float gv = gr[n];
        const float *br = B + (size_t)n * a.R + j0;
        if (vec) {
#pragma unroll
            for (int q = 0; q < kTRanks / 4; ++q) {
                const float4 b4 = *reinterpret_cast<const float4 *>(br + 4 * q);
                s[4 * q] = fmaf(gv, b4.x, s[4 * q]);
                s[4 * q + 1] = fmaf(gv, b4.y, s[4 * q + 1]);
                s[4 * q + 2] = fmaf(gv, b4.z, s[4 * q + 2]);
                s[4 * q + 3] = fmaf(gv, b4.w, s[4 * q + 3]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kTRanks; ++j)
                if (j0 + j < a.R) s[j] = fmaf(gv, br[j], s[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kTRanks; ++j) s[j] = wave_sum(s[j]);
    if (lane < kTRanks) {
        float v = s[0];
#pragma unroll
        for (int j = 1; j < kTRanks; ++j)
            if (lane == j) v = s[j];
        part[wave][lane] = v;
    }
    __syncthreads();
    if (wave == 0 && lane < kTRanks && j0 + lane < a.R)
        t[(size_t)p * a.R + j0 + lane] = a.scale[g] * (((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]);
}

// dx[p][i] += sum_j t[p][j] * A[g][j][i], i < width; thread i takes
// positions pp blockIdx.y .. + pp - 1 and keeps its column of A (up to 16
// ranks) in registers while the group stays the same (pp = 8 when there are
// positions enough to fill the GPU that way, else 1).
__global__ __launch_bounds__(256) void lora_dx_kernel(LoraArgs a, const float *__restrict__ t,
                                                      float *__restrict__ dx, int ld_dx, int pp)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.width) return;
    const int pb = blockIdx.y * pp, pe = min(a.P, pb + pp);
    int gcur = -1;
    float ac[16];
    for (int p = pb; p < pe; ++p) {
        const int g = a.pgroup ? a.pgroup[p] : 0;
        const float *A = a.A + (size_t)g * a.R * a.kin + i;
        if (g != gcur) {  // uniform
#pragma unroll
            for (int j = 0; j < 16; ++j) ac[j] = A[(size_t)min(j, a.R - 1) * a.kin];  // in bounds; j >= R unused
            gcur = g;
        }
        const float *tp = t + (size_t)p * a.R;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (j < a.R) s = fmaf(tp[j], ac[j], s);
        for (int j = 16; j < a.R; ++j) s = fmaf(tp[j], A[(size_t)j * a.kin], s);
        dx[(size_t)p * ld_dx + i] += s;
    }
}

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + __expf(-x)); }

// gate and up activations and their derivatives (activationfunction.go:
// 102-115, moreactivationfunctions.go:207-244); limit > 0 selects the
// clamped pair
__device__ __forceinline__ float gate_act(float x, float limit)
{
    if (limit > 0.f && x > limit) x = limit;
    return x * sigm(x);
}
__device__ __forceinline__ float gate_deriv(float x, float limit)
{
    if (limit > 0.f && x > limit) return 0.f;
    const float s = sigm(x);
    return s + x * s * (1.f - s);
}
__device__ __forceinline__ float up_act(float x, float limit)
{
    if (limit > 0.f) return x > limit ? limit : (x < -limit ? -limit : x);
    return x;
}
__device__ __forceinline__ float up_deriv(float x, float limit)
{
    if (limit > 0.f && (x > limit || x < -limit)) return 0.f;
    return 1.f;
}

// hidden = act_g(gate_pre) * act_u(up_pre) (gatedfeedforward.go:49-57); the
// padding columns [h, hp) are zero
__global__ __launch_bounds__(256) void swiglu_forward_kernel(const float *__restrict__ gpre,
                                                             const float *__restrict__ upre, int h, int hp,
                                                             float limit, float *__restrict__ hidden)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const size_t o = (size_t)blockIdx.y * hp + n;
    if (n >= hp) return;
    hidden[o] = n < h ? gate_act(gpre[o], limit) * up_act(upre[o], limit) : 0.f;
}

// gatedfeedforward.go:59-67 with Layer.Backward's activation step
// (layer.go:175-182): gate_grad = hidden_grad * up_out * act_g'(gate_pre),
// up_grad = hidden_grad * gate_out * act_u'(up_pre)
__global__ __launch_bounds__(256) void swiglu_backward_kernel(const float *__restrict__ hgrad,
                                                              const float *__restrict__ gpre,
                                                              const float *__restrict__ upre, int h, int hp,
                                                              float limit, float *__restrict__ ggrad,
                                                              float *__restrict__ ugrad)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const size_t o = (size_t)blockIdx.y * hp + n;
    if (n >= hp) return;
    float gg = 0.f, ug = 0.f;
    if (n < h) {
        const float gp = gpre[o], upv = upre[o], hg = hgrad[o];
        gg = hg * up_act(upv, limit) * gate_deriv(gp, limit);
        ug = hg * gate_act(gp, limit) * up_deriv(upv, limit);
    }
    ggrad[o] = gg;
    ugrad[o] = ug;
}

// Gradient of every position's expert output: the token's output gradient,
// times the slot's gate for a routed position (mixtureofexperts.go:243-247).
__global__ __launch_bounds__(256) void expert_output_grad_kernel(const double *__restrict__ og, int d, int ld,
                                                                 const int32_t *__restrict__ tok,
                                                                 const int32_t *__restrict__ pgroup, int S, int T,
                                                                 int k, const int32_t *__restrict__ chosen,
                                                                 const double *__restrict__ gates,
                                                                 float *__restrict__ eg)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int p = blockIdx.y;
    if (i >= ld) return;
    const int t = tok[p], g = pgroup[p];
    double w = 1.0;
    if (g >= S)
        for (int j = 0; j < k; ++j)
            if (chosen[(size_t)t * k + j] == g - S) w = gates[(size_t)t * k + j];
    eg[(size_t)p * ld + i] = i < d ? (float)(og[(size_t)t * d + i] * w) : 0.f;
}

// Input gradient of each token: the shared experts' rows, then its routed
// slots in chosen order (mixtureofexperts.go:237-256), each row being the
// gate layer's plus the up layer's input gradient.
__global__ __launch_bounds__(256) void gather_input_grad_kernel(const float *__restrict__ dxg,
                                                                const float *__restrict__ dxu, int ld, int d, int T,
                                                                int S, int k, const int32_t *__restrict__ pos,
                                                                double *__restrict__ dx)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y;
    if (i >= d) return;
    double acc = 0.0;
    for (int s = 0; s < S; ++s) {
        const size_t o = (size_t)(s * T + t) * ld + i;
        acc += (double)(dxg[o] + dxu[o]);
    }
    for (int j = 0; j < k; ++j) {
        const size_t o = (size_t)(S * T + pos[(size_t)t * k + j]) * ld + i;
        acc += (double)(dxg[o] + dxu[o]);
    }
    dx[(size_t)t * d + i] = acc;
}

// dx[t][i] += sum_e lg[t][e] * W[e][i] (the router's base rows, fp32, row
// stride ldw), i < d
__global__ __launch_bounds__(256) void router_input_grad_kernel(const float *__restrict__ lg, int E,
                                                                const float *__restrict__ w, int ldw, int d,
                                                                float *__restrict__ dx, int ld_dx)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y;
    if (i >= d) return;
    float s = 0.f;
    for (int e = 0; e < E; ++e) s = fmaf(lg[(size_t)t * E + e], w[(size_t)e * ldw + i], s);
    dx[(size_t)t * ld_dx + i] = s;
}

__global__ __launch_bounds__(256) void add_rows_f64_kernel(const float *__restrict__ src, int ld, int d, int T,
                                                           double *__restrict__ dst)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int t = blockIdx.y;
    if (i >= d || t >= T) return;
    dst[(size_t)t * d + i] += (double)src[(size_t)t * ld + i];
}

inline dim3 cols_grid(int cols, int rows) { return dim3((cols + 255) / 256, rows); }

}  // namespace

namespace {

template <int PREC>
void launch_transposed_prec(const RowsArgs &a, int tile, dim3 grid, int chunk_rows, float *partial, long long stride,
                            hipStream_t s)
{
    if (tile == kMtPositions)
        hipLaunchKernelGGL((rows_transposed_mfma_kernel<PREC>), grid, dim3(256), 0, s, a, chunk_rows, partial, stride);
    else if (tile == 8)
        hipLaunchKernelGGL((rows_transposed_kernel<PREC, 8>), grid, dim3(64 * kTrWaves), 0, s, a, chunk_rows, partial,
                           stride);
    else
        hipLaunchKernelGGL((rows_transposed_kernel<PREC, 4>), grid, dim3(64 * kTrWaves), 0, s, a, chunk_rows, partial,
                           stride);
}

}  // namespace

hipError_t launch_rows_transposed(const RowsArgs &a, int precision, int ntiles, int tile, int chunks, float *partial,
                                  hipStream_t s)
{
    if (ntiles <= 0) return hipSuccess;
    if (chunks < 1 || (chunks > 1 && !partial) || (tile != 4 && tile != 8 && tile != kMtPositions))
        return hipErrorInvalidValue;
    const bool mfma = tile == kMtPositions;
    int chunk_rows = (a.rows + chunks - 1) / chunks;
    if (mfma) {  // whole panels per chunk, and no empty chunk
        chunk_rows = (chunk_rows + kMtRows - 1) / kMtRows * kMtRows;
        chunks = (a.rows + chunk_rows - 1) / chunk_rows;
    }
    const long long stride = (long long)a.tiles_positions * a.ld_out;
    const dim3 grid(rows_transposed_colblocks(a.nblocks, tile), ntiles, chunks);
    switch (precision) {
    case kInt8: launch_transposed_prec<kInt8>(a, tile, grid, chunk_rows, partial, stride, s); break;
    case kFP4: launch_transposed_prec<kFP4>(a, tile, grid, chunk_rows, partial, stride, s); break;
    case kFloat32: launch_transposed_prec<kFloat32>(a, tile, grid, chunk_rows, partial, stride, s); break;
    default: return hipErrorInvalidValue;
    }
    if (chunks > 1)
        hipLaunchKernelGGL(sum_chunks_kernel, dim3((a.kp + 255) / 256, a.tiles_positions), dim3(256), 0, s, partial,
                           stride, chunks, a.kp, a.ld_out, a.out);
    return hipGetLastError();
}

// Positions per workgroup of the transposed product: the matrix-core kernel's
// 32 once the groups average 16 positions, eight once they average eight
// (each decoded weight then feeds twice the multiply-adds), else four.
int rows_transposed_tile(int positions, int groups)
{
    return positions >= 16 * groups ? kMtPositions : positions >= 8 * groups ? 8 : 4;
}
int lora_outer_tile_positions() { return kOpPositions; }
int rows_transposed_chunk_rows(int tile) { return tile == kMtPositions ? kMtRows : 32 * kTrWaves; }
int rows_transposed_colblocks(int nblocks, int tile)
{
    return tile == kMtPositions ? (nblocks + kMtBlocks - 1) / kMtBlocks : (nblocks + 63) / 64;
}

hipError_t launch_lora_down(const LoraArgs &a, const float *in, int ld_in, const int32_t *in_tok, float *u,
                            hipStream_t s)
{
    if (a.P <= 0 || a.R <= 0) return hipSuccess;
    const int waves = a.P * a.R;
    hipLaunchKernelGGL(lora_down_kernel, dim3((waves + 3) / 4), dim3(256), 0, s, a, in, ld_in, in_tok, u);
    return hipGetLastError();
}

hipError_t launch_lora_up_bias(const LoraArgs &a, const float *u, float *out, int ld_out, const float *bias,
                               hipStream_t s)
{
    if (a.P <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_up_bias_kernel<float>, cols_grid(a.rows, a.P), dim3(256), 0, s, a, u, out, ld_out, bias,
                       nullptr);
    return hipGetLastError();
}

hipError_t launch_lora_up_bias_f64(const LoraArgs &a, const float *u, double *out, int ld_out, const double *bias,
                                   hipStream_t s)
{
    if (a.P <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_up_bias_kernel<double>, cols_grid(a.rows, a.P), dim3(256), 0, s, a, u, out, ld_out,
                       nullptr, bias);
    return hipGetLastError();
}

hipError_t launch_lora_backward(const LoraArgs &a, const float *grad, int ld_g, const float *u, const float *in,
                                int ld_in, const int32_t *in_tok, float *t, float *dx, int ld_dx, double *dA,
                                double *dB, float *scratch, hipStream_t s)
{
    if (a.P <= 0 || a.R <= 0) return hipSuccess;
    if (a.notiles <= 0 || !a.otiles || !a.otoff || (a.nomulti > 0 && (!a.omulti || !scratch)))
        return hipErrorInvalidValue;
    // dB += scale grad^T u: columns are B's rows n, the sums land at dB[g][n][j]
    launch_outer(OuterArgs{a.otiles, u, a.R, grad, ld_g, nullptr, a.rows, nullptr, a.scale, dB,
                           (long long)a.rows * a.R, 1LL, (long long)a.R},
                 a, scratch, s);
    hipLaunchKernelGGL(lora_t_kernel, dim3(a.P * ((a.R + kTRanks - 1) / kTRanks)), dim3(256), 0, s, a, grad, ld_g, t);
    // dA += t^T in: columns are the inputs i, the sums land at dA[g][j][i]
    launch_outer(OuterArgs{a.otiles, t, a.R, in, ld_in, in_tok, a.width, nullptr, nullptr, dA, (long long)a.R * a.kin,
                           (long long)a.kin, 1LL},
                 a, scratch, s);
    const int pp = (long long)((a.width + 255) / 256) * (a.P / 8) >= 1024 ? 8 : 1;
    hipLaunchKernelGGL(lora_dx_kernel, dim3((a.width + 255) / 256, (a.P + pp - 1) / pp), dim3(256), 0, s, a, t, dx,
                       ld_dx, pp);
    return hipGetLastError();
}

hipError_t launch_swiglu_forward(const float *gpre, const float *upre, int P, int h, int hp, float limit,
                                 float *hidden, hipStream_t s)
{
    if (P <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_forward_kernel, cols_grid(hp, P), dim3(256), 0, s, gpre, upre, h, hp, limit, hidden);
    return hipGetLastError();
}

hipError_t launch_swiglu_backward(const float *hgrad, const float *gpre, const float *upre, int P, int h, int hp,
                                  float limit, float *ggrad, float *ugrad, hipStream_t s)
{
    if (P <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_backward_kernel, cols_grid(hp, P), dim3(256), 0, s, hgrad, gpre, upre, h, hp, limit,
                       ggrad, ugrad);
    return hipGetLastError();
}

hipError_t launch_expert_output_grad(const double *og, int d, int ld, const int32_t *tok, const int32_t *pgroup,
                                     int S, int T, int k, const int32_t *chosen, const double *gates, int P,
                                     float *eg, hipStream_t s)
{
    if (P <= 0) return hipSuccess;
    hipLaunchKernelGGL(expert_output_grad_kernel, cols_grid(ld, P), dim3(256), 0, s, og, d, ld, tok, pgroup, S, T, k,
                       chosen, gates, eg);
    return hipGetLastError();
}

hipError_t launch_gather_input_grad(const float *dxg, const float *dxu, int ld, int d, int T, int S, int k,
                                    const int32_t *pos, double *dx, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_input_grad_kernel, cols_grid(d, T), dim3(256), 0, s, dxg, dxu, ld, d, T, S, k, pos, dx);
    return hipGetLastError();
}

hipError_t launch_router_input_grad(const float *lg, int T, int E, const float *w, int ldw, int d, float *dx,
                                    int ld_dx, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(router_input_grad_kernel, cols_grid(d, T), dim3(256), 0, s, lg, E, w, ldw, d, dx, ld_dx);
    return hipGetLastError();
}

hipError_t launch_add_rows_f64(const float *src, int ld, int d, int T, double *dst, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(add_rows_f64_kernel, cols_grid(d, T), dim3(256), 0, s, src, ld, d, T, dst);
    return hipGetLastError();
}

}  // namespace gtmoe
