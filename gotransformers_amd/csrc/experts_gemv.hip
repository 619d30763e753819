// fp32 expert kernels for few tokens per expert (decode): a dequantizing
// GEMV that streams each weight row from HBM once per group of tokens.
//
// Work split: grid (ceil(rows/16), token slices of all groups); every wave
// owns 4 consecutive output rows of one group (expert) for one slice of at
// most 8 of its tokens.  A row's K values are covered by the 64
// lanes in 16-value blocks -- lane l takes blocks l, l+64, ... -- so each
// load instruction of a wave reads one contiguous run of the row (1 KiB of
// Int8, 512 B of FP4), coalesced, together with the matching fp32 scales.
// Per block the lane forms the 16-term partial sum of every token it holds,
// scales it once (the reference's DotRow order, lowprecision/rows.go:
// 207-257), and accumulates.  The per-lane partials of all (row, matrix,
// token) values are then summed across the wave by a transposing butterfly
// that halves the live values at every exchange.
//
// Gate/up fuse the SwiGLU epilogue (feedforward/gatedfeedforward.go:49-57):
// hidden = act_g(gate + b_g) * act_u(up + b_u).  Down adds its bias.
#include "common.h"

#include <utility>

namespace gtmoe {

namespace {

template <int PREC>
struct RawBlock;
template <>
struct RawBlock<kInt8> {
    uint4 v;
};
template <>
struct RawBlock<kFP4> {
    uint2 v;
};
template <>
struct RawBlock<kFloat32> {
    float4 v[4];
};

template <int PREC>
__device__ __forceinline__ void load_raw(RawBlock<PREC> &r, const char *row, int b);
template <>
__device__ __forceinline__ void load_raw<kInt8>(RawBlock<kInt8> &r, const char *row, int b)
{
    r.v = *reinterpret_cast<const uint4 *>(row + (size_t)b * 16);
}
template <>
__device__ __forceinline__ void load_raw<kFP4>(RawBlock<kFP4> &r, const char *row, int b)
{
    r.v = *reinterpret_cast<const uint2 *>(row + (size_t)b * 8);
}
template <>
__device__ __forceinline__ void load_raw<kFloat32>(RawBlock<kFloat32> &r, const char *row, int b)
{
    const float4 *p = reinterpret_cast<const float4 *>(row + (size_t)b * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = p[i];
}

template <int PREC>
__device__ __forceinline__ void zero_raw(RawBlock<PREC> &r)
{
    r = RawBlock<PREC>{};
}

// Codes of one block as floats (Int8 values, FP4 magnitudes with sign, or
// the float32 weights themselves); the scale is applied by the caller.
__device__ __forceinline__ void decode(const RawBlock<kInt8> &r, float (&w)[16])
{
    const uint32_t d[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) w[4 * i + j] = (float)(int)(int8_t)(d[i] >> (8 * j));
}
__device__ __forceinline__ void decode(const RawBlock<kFP4> &r, float (&w)[16])
{
    // e2m1 codes, even value in the low nibble; the hardware conversion
    // with scale 1.0 yields exactly {0, .5, 1, 1.5, 2, 3, 4, 6} with sign.
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const uint32_t d[2] = {r.v.x, r.v.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const f32x2 f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 0);
        const f32x2 f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 1);
        const f32x2 f2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 2);
        const f32x2 f3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 3);
        w[8 * i + 0] = f0[0];
        w[8 * i + 1] = f0[1];
        w[8 * i + 2] = f1[0];
        w[8 * i + 3] = f1[1];
        w[8 * i + 4] = f2[0];
        w[8 * i + 5] = f2[1];
        w[8 * i + 6] = f3[0];
        w[8 * i + 7] = f3[1];
    }
}
__device__ __forceinline__ void decode(const RawBlock<kFloat32> &r, float (&w)[16])
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[4 * i + 0] = r.v[i].x;
        w[4 * i + 1] = r.v[i].y;
        w[4 * i + 2] = r.v[i].z;
        w[4 * i + 3] = r.v[i].w;
    }
}

// Sum N per-lane values over the 64 lanes of a wave.  Afterwards lane l
// holds in v[0] the total of value index l / (64 / N).
//
// Every exchange halves the live values: the lower lanes of a pair keep
// values [0, half) and send [half, 2*half), the upper lanes the reverse.
// The pair loop is expanded at compile time (index sequences) so the array
// elements stay in registers; a runtime-indexed form lets the compiler fold
// the per-lane choice into a register-file index, which costs a compare and
// select per element.
template <int I, int HALF, int OFF>
__device__ __forceinline__ void exchange_pair(float *v, bool upper)
{
    const float lo = v[I], hi = v[I + HALF];
    if constexpr (OFF == 32 || OFF == 16) {
        // gfx950 v_permlane{32,16}_swap: lanes of the upper half of each
        // 2*OFF group trade `lo` for their partner's `hi`; afterwards every
        // lane's two registers hold the pair it keeps, whichever half it is in
        const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false)
                                 : __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
        v[I] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        const float send = upper ? lo : hi;
        const float keep = upper ? hi : lo;
        v[I] = keep + __shfl_xor(send, OFF);
    }
}

template <int HALF, int OFF, int... I>
__device__ __forceinline__ void exchange_all(float *v, bool upper, std::integer_sequence<int, I...>)
{
    (exchange_pair<I, HALF, OFF>(v, upper), ...);
}

template <int HALF, int OFF>
__device__ __forceinline__ void halve(float *v, int lane)
{
    if constexpr (HALF >= 1) {
        exchange_all<HALF, OFF>(v, (lane & OFF) != 0, std::make_integer_sequence<int, HALF>{});
        halve<HALF / 2, OFF / 2>(v, lane);
    }
}

template <int N>
__device__ __forceinline__ void wave_transpose_reduce(float (&v)[N], int lane)
{
    halve<N / 2, 32>(v, lane);
    for (int off = 32 / N; off > 0; off >>= 1) v[0] += __shfl_xor(v[0], off);
}

template <int N>
struct Log2 {
    static constexpr int value = 1 + Log2<N / 2>::value;
};
template <>
struct Log2<1> {
    static constexpr int value = 0;
};

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

}  // namespace

// Weight blocks (and their scales) of RIF rows starting at row rb, for each
// matrix and each of the lane's NB blocks.
template <int PREC, int NB, int RIF, int MATS>
__device__ __forceinline__ void load_rows(const GemvArgs &a, int rb, int lane, const char *wb0, const char *wb1,
                                          const float *sb0, const float *sb1, RawBlock<PREC> (&raw)[RIF][MATS][NB],
                                          float (&sc)[RIF][MATS][NB])
{
#pragma unroll
    for (int rr = 0; rr < RIF; ++rr) {
        const int r = rb + rr;
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt) {
            const char *row = (mt == 0 ? wb0 : wb1) + (size_t)r * a.row_bytes;
            const float *srow = (mt == 0 ? sb0 : sb1) + (size_t)r * a.nblocks;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int b = lane + 64 * j;
                if (r < a.rows && b < a.nblocks) {
                    load_raw<PREC>(raw[rr][mt][j], row, b);
                    sc[rr][mt][j] = (PREC == kFloat32) ? 1.0f : srow[b];
                } else {
                    zero_raw<PREC>(raw[rr][mt][j]);
                    sc[rr][mt][j] = 0.f;
                }
            }
        }
    }
}

// Dot products of the TC held tokens with RIF loaded rows, reduced across
// the wave, with the epilogue (SwiGLU or bias) written to the output.
template <int PREC, int NB, int TC, int RIF, bool GATEUP>
__device__ __forceinline__ void process_rows(const GemvArgs &a, int p0, int M, int c0, int rb, int lane,
                                             const float (&xr)[TC][NB][16],
                                             const RawBlock<PREC> (&raw)[RIF][GATEUP ? 2 : 1][NB],
                                             const float (&sc)[RIF][GATEUP ? 2 : 1][NB], const float *bb0,
                                             const float *bb1)
{
    constexpr int MATS = GATEUP ? 2 : 1;
    constexpr int NV = RIF * MATS * TC;  // values reduced per exchange round
    constexpr int SHIFT = 6 - Log2<NV>::value;
    static_assert(NV <= 64, "too many values per lane");
    float part[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) part[i] = 0.f;
#pragma unroll
    for (int rr = 0; rr < RIF; ++rr)
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                float w[16];
                decode(raw[rr][mt][j], w);
#pragma unroll
                for (int c = 0; c < TC; ++c) {
                    float bs = 0.f;
#pragma unroll
                    for (int q = 0; q < 16; ++q) bs = fmaf(xr[c][j][q], w[q], bs);
                    float &acc = part[(rr * MATS + mt) * TC + c];
                    acc = fmaf(bs, sc[rr][mt][j], acc);
                }
            }
    wave_transpose_reduce<NV>(part, lane);
    const int v = lane >> SHIFT;
    const bool writer = (lane & ((1 << SHIFT) - 1)) == 0;
    const int c = v % TC;
    const int m = c0 + c;
    if (GATEUP) {
        const float other = __shfl_xor(part[0], TC << SHIFT);
        const int mt = (v / TC) % 2;
        const int rr = v / (2 * TC);
        const int r = rb + rr;
        if (writer && mt == 0 && m < M && r < a.rows) {
            float gv = part[0] + bb0[r];
            float uv = other + bb1[r];
            if (a.clamp > 0.f) {
                gv = fminf(gv, a.clamp);                   // ClampedSiLU: x > L -> silu(L)
                uv = fminf(fmaxf(uv, -a.clamp), a.clamp);  // ClampedLinear
            }
            a.out[(size_t)(p0 + m) * a.ld_out + r] = silu(gv) * uv;
        }
    } else {
        const int rr = v / TC;
        const int r = rb + rr;
        if (writer && m < M && r < a.rows) a.out[(size_t)(p0 + m) * a.ld_out + r] = part[0] + bb0[r];
    }
}

// One chunk of TC tokens (positions p0+c0 .. p0+c0+TC-1, those >= M masked)
// of a group against the NIT*RIF rows of this wave.  The tokens sit in
// registers; the rows go through RIF at a time with the weights of the next
// RIF rows loading while the current ones are computed (two register
// buffers), so the wave keeps loads in flight through its compute.
template <int PREC, int NB, int TC, int RIF, int NIT, bool GATEUP>
__device__ __forceinline__ void gemv_chunk(const GemvArgs &a, int p0, int M, int c0, int r0, int lane,
                                           const char *wb0, const char *wb1, const float *sb0, const float *sb1,
                                           const float *bb0, const float *bb1)
{
    static_assert(NIT == 1 || NIT % 2 == 0, "row steps come alone or in pairs");
    constexpr int MATS = GATEUP ? 2 : 1;
    RawBlock<PREC> raw0[RIF][MATS][NB], raw1[RIF][MATS][NB];
    float sc0[RIF][MATS][NB], sc1[RIF][MATS][NB];
    load_rows<PREC, NB, RIF, MATS>(a, r0, lane, wb0, wb1, sb0, sb1, raw0, sc0);

    float xr[TC][NB][16];
#pragma unroll
    for (int c = 0; c < TC; ++c) {
        const int m = c0 + c;
        const int src = (m < M) ? (GATEUP ? a.tok[p0 + m] : p0 + m) : 0;
        const float *xrow = a.in + (size_t)src * a.ld_in;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int b = lane + 64 * j;
            if (m < M && b < a.nblocks) {
                const float4 *p = reinterpret_cast<const float4 *>(xrow + (size_t)b * 16);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = p[q];
                    xr[c][j][4 * q + 0] = v.x;
                    xr[c][j][4 * q + 1] = v.y;
                    xr[c][j][4 * q + 2] = v.z;
                    xr[c][j][4 * q + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) xr[c][j][q] = 0.f;
            }
        }
    }

    if constexpr (NIT == 1) {
        process_rows<PREC, NB, TC, RIF, GATEUP>(a, p0, M, c0, r0, lane, xr, raw0, sc0, bb0, bb1);
        return;
    }
#pragma unroll
    for (int it = 0; it < NIT; it += 2) {
        load_rows<PREC, NB, RIF, MATS>(a, r0 + (it + 1) * RIF, lane, wb0, wb1, sb0, sb1, raw1, sc1);
        process_rows<PREC, NB, TC, RIF, GATEUP>(a, p0, M, c0, r0 + it * RIF, lane, xr, raw0, sc0, bb0, bb1);
        if (it + 2 < NIT) load_rows<PREC, NB, RIF, MATS>(a, r0 + (it + 2) * RIF, lane, wb0, wb1, sb0, sb1, raw0, sc0);
        process_rows<PREC, NB, TC, RIF, GATEUP>(a, p0, M, c0, r0 + (it + 1) * RIF, lane, xr, raw1, sc1, bb0, bb1);
    }
}

// One wave = NIT*RIF output rows of one group over one slice of at most
// tslice of the group's tokens (blockIdx.y enumerates the slices of all
// groups; the dispatch wrote their prefix and the slice -> group table).
// Inside the slice, tokens go through in chunks whose width follows the count
// left (TCMAX, then 2, then 1), so a group with one or two tokens does no work
// for absent ones.
template <int PREC, int NB, int TCMAX, int RIF, int NIT, bool GATEUP>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a)
{
    constexpr int RPW = NIT * RIF;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int item = blockIdx.y;
    if (item >= a.slice_off[a.groups]) return;
    const int g = a.group_of[item];
    const int r0 = (blockIdx.x * 4 + wave) * RPW;
    if (r0 >= a.rows) return;
    const int first = (item - a.slice_off[g]) * a.tslice;
    const int p0 = a.goff[g] + first;
    const int M = min(a.goff[g + 1] - a.goff[g] - first, a.tslice);
    if (M <= 0) return;

    const char *wb0 = reinterpret_cast<const char *>(a.w0) + (size_t)g * a.w_group_stride;
    const char *wb1 = GATEUP ? reinterpret_cast<const char *>(a.w1) + (size_t)g * a.w_group_stride : nullptr;
    const float *sb0 = a.s0 + (size_t)g * a.s_group_stride;
    const float *sb1 = GATEUP ? a.s1 + (size_t)g * a.s_group_stride : nullptr;
    const float *bb0 = a.b0 + (size_t)g * a.rows;
    const float *bb1 = GATEUP ? a.b1 + (size_t)g * a.rows : nullptr;

    int c0 = 0;
    if constexpr (TCMAX >= 4) {
        for (; M - c0 >= 3; c0 += 4)
            gemv_chunk<PREC, NB, 4, RIF, NIT, GATEUP>(a, p0, M, c0, r0, lane, wb0, wb1, sb0, sb1, bb0, bb1);
    }
    if constexpr (TCMAX >= 2) {
        for (; M - c0 >= 2; c0 += 2)
            gemv_chunk<PREC, NB, 2, RIF, NIT, GATEUP>(a, p0, M, c0, r0, lane, wb0, wb1, sb0, sb1, bb0, bb1);
    }
    for (; c0 < M; ++c0)
        gemv_chunk<PREC, NB, 1, RIF, NIT, GATEUP>(a, p0, M, c0, r0, lane, wb0, wb1, sb0, sb1, bb0, bb1);
}

namespace {

// Shapes per K width: NB blocks of 16 per lane, TCMAX tokens in registers,
// RIF rows per pipeline step, NIT steps per wave.
template <bool GATEUP, int PREC>
hipError_t launch_prec(const GemvArgs &a, int max_slices, hipStream_t s)
{
    const int nb = (a.nblocks + 63) / 64;
    constexpr bool F32 = PREC == kFloat32;
    auto grid = [&](int rows_per_wave) {
        return dim3((a.rows + 4 * rows_per_wave - 1) / (4 * rows_per_wave), max_slices);
    };
    if (nb <= 1) {
        if constexpr (F32) hipLaunchKernelGGL((gemv_kernel<PREC, 1, 4, 1, 4, GATEUP>), grid(4), dim3(256), 0, s, a);
        else hipLaunchKernelGGL((gemv_kernel<PREC, 1, 4, 4, 1, GATEUP>), grid(4), dim3(256), 0, s, a);
    } else if (nb <= 2) {
        if constexpr (F32) hipLaunchKernelGGL((gemv_kernel<PREC, 2, 2, 1, 4, GATEUP>), grid(4), dim3(256), 0, s, a);
        else hipLaunchKernelGGL((gemv_kernel<PREC, 2, 2, 1, 4, GATEUP>), grid(4), dim3(256), 0, s, a);
    } else if (nb <= 4) {
        hipLaunchKernelGGL((gemv_kernel<PREC, 4, 1, 1, 4, GATEUP>), grid(4), dim3(256), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool GATEUP>
hipError_t launch_any(const GemvArgs &a, int precision, int max_slices, hipStream_t s)
{
    if (max_slices <= 0) return hipSuccess;
    switch (precision) {
    case kInt8: return launch_prec<GATEUP, kInt8>(a, max_slices, s);
    case kFP4: return launch_prec<GATEUP, kFP4>(a, max_slices, s);
    case kFloat32: return launch_prec<GATEUP, kFloat32>(a, max_slices, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemv_gateup(const GemvArgs &a, int precision, int max_slices, hipStream_t s)
{
    return launch_any<true>(a, precision, max_slices, s);
}

hipError_t launch_gemv_down(const GemvArgs &a, int precision, int max_slices, hipStream_t s)
{
    return launch_any<false>(a, precision, max_slices, s);
}

}  // namespace gtmoe
