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
#include "common.h"

namespace gtmoe {

namespace {

constexpr int kTrRows = 128;  // gradient rows staged per step

__device__ __forceinline__ float fp4_value(uint32_t code)
{
    const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    const float v = mag[code & 7];
    return (code & 8) ? -v : v;
}

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
        const uint32_t d[2] = {q[0].x, q[0].y};
#pragma unroll
        for (int v = 0; v < 16; ++v) w[v] = fp4_value(d[v >> 3] >> (4 * (v & 7)));
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

// dB[g][n][j] += scale[g] * sum_{p in g} grad[p][n] * u[p][j]
__global__ __launch_bounds__(256) void lora_grad_up_kernel(LoraArgs a, const float *__restrict__ grad, int ld_g,
                                                           const float *__restrict__ u, double *__restrict__ dB)
{
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int g = blockIdx.y;
    if (idx >= a.rows * a.R) return;
    const int n = idx / a.R, j = idx - n * a.R;
    float s = 0.f;
#pragma unroll 8
    for (int p = a.goff[g]; p < a.goff[g + 1]; ++p) s = fmaf(grad[(size_t)p * ld_g + n], u[(size_t)p * a.R + j], s);
    dB[(size_t)g * a.rows * a.R + idx] += (double)(a.scale[g] * s);
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

// dA[g][j][i] += sum_{p in g} t[p][j] * in[row(p)][i], i < width
__global__ __launch_bounds__(256) void lora_grad_down_kernel(LoraArgs a, const float *__restrict__ t,
                                                             const float *__restrict__ in, int ld_in,
                                                             const int32_t *__restrict__ in_tok,
                                                             double *__restrict__ dA)
{
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int g = blockIdx.y;
    if (idx >= a.R * a.width) return;
    const int j = idx / a.width, i = idx - j * a.width;
    float s = 0.f;
#pragma unroll 8
    for (int p = a.goff[g]; p < a.goff[g + 1]; ++p) {
        const int row = in_tok ? in_tok[p] : p;
        s = fmaf(t[(size_t)p * a.R + j], in[(size_t)row * ld_in + i], s);
    }
    dA[((size_t)g * a.R + j) * a.kin + i] += (double)s;
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
    if (tile == 8)
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
    if (chunks < 1 || (chunks > 1 && !partial) || (tile != 4 && tile != 8)) return hipErrorInvalidValue;
    const int chunk_rows = (a.rows + chunks - 1) / chunks;
    const long long stride = (long long)a.tiles_positions * a.ld_out;
    const dim3 grid((a.nblocks + 63) / 64, ntiles, chunks);
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

// Positions per workgroup of the transposed product: eight once the groups
// average eight positions (each decoded weight then feeds twice the
// multiply-adds), else four.
int rows_transposed_tile(int positions, int groups) { return positions >= 8 * groups ? 8 : 4; }
int rows_transposed_chunk_rows() { return 32 * kTrWaves; }

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
                                double *dB, hipStream_t s)
{
    if (a.P <= 0 || a.R <= 0) return hipSuccess;
    hipLaunchKernelGGL(lora_grad_up_kernel, cols_grid(a.rows * a.R, a.G), dim3(256), 0, s, a, grad, ld_g, u, dB);
    hipLaunchKernelGGL(lora_t_kernel, dim3(a.P * ((a.R + kTRanks - 1) / kTRanks)), dim3(256), 0, s, a, grad, ld_g, t);
    hipLaunchKernelGGL(lora_grad_down_kernel, cols_grid(a.R * a.width, a.G), dim3(256), 0, s, a, t, in, ld_in,
                       in_tok, dA);
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
