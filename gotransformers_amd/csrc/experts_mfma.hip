// bf16 MFMA grouped GEMM for many tokens per expert (prefill).
//
// One workgroup computes a 128-position x 128-column tile of one group
// (expert) with v_mfma_f32_32x32x16_bf16, fp32 accumulation:
//   gate/up  A = activations gathered by token (bf16), B = 64 gate rows and
//            the same 64 up rows of the expert, dequantized in registers
//            (Int8 code or e2m1 code times its fp32 block scale, rounded to
//            bf16) and staged in LDS; the epilogue applies the SwiGLU
//            (feedforward/gatedfeedforward.go:49-57) and writes bf16 hidden
//            rows.
//   down     A = hidden rows (bf16, contiguous per group), B = 128 down rows;
//            the epilogue adds the bias and writes fp32 slot outputs.
// Four waves, each a 64 x 64 sub-tile = 2 x 2 MFMA 32x32 tiles; for gate/up
// a wave's two column tiles are gate and up of the same 32 neurons, so both
// values of a neuron land in the same lane.  K advances in steps of 32 (two
// scale blocks) through double-buffered LDS; global loads of the next step
// are in flight during the MFMAs of the current one.
//
// Tiles: blockIdx.x enumerates the m-tiles of all groups (the dispatch
// kernel wrote their count and a (group, first position, positions)
// descriptor per tile; blocks past the last tile exit), blockIdx.y the
// column tiles.
#include "common.h"

namespace gtmoe {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128;
constexpr int BK = 32;
constexpr int BC = 128;     // columns of B staged per tile
constexpr int LDSK = 40;    // LDS row stride in bf16 (32 + 8 padding)

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi)
{
    const __bf16 a = (__bf16)lo, b = (__bf16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Sixteen weights (one scale block) at block index b of a row, times the
// block scale, as 16 bf16 in 8 dwords.  `row` points at the row's first
// 16-byte unit in its panel (units of a row are 1 KiB apart), `srow` at its
// first scale group.
template <int PREC>
__device__ __forceinline__ void dequant16(const char *row, const float *srow, int b, uint32_t (&out)[8])
{
    float w[16];
    const float s = PREC == kFloat32 ? 1.0f : srow[(size_t)(b >> 2) * 256 + (b & 3)];
    if constexpr (PREC == kInt8) {
        const uint4 q = *reinterpret_cast<const uint4 *>(row + (size_t)b * 1024);
        const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) w[4 * i + j] = (float)(int)(int8_t)(d[i] >> (8 * j)) * s;
    } else if constexpr (PREC == kFP4) {
        const uint2 q = *reinterpret_cast<const uint2 *>(row + (size_t)(b >> 1) * 1024 + (b & 1) * 8);
        const uint32_t d[2] = {q.x, q.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x2 f;
                switch (j) {
                case 0: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 0); break;
                case 1: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 1); break;
                case 2: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 2); break;
                default: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d[i], 1.0f, 3); break;
                }
                w[8 * i + 2 * j] = f[0] * s;
                w[8 * i + 2 * j + 1] = f[1] * s;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = *reinterpret_cast<const float4 *>(row + (size_t)(4 * b + i) * 1024);
            w[4 * i + 0] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = pack_bf16(w[2 * i], w[2 * i + 1]);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

}  // namespace

template <int PREC, bool GATEUP>
__global__ __launch_bounds__(256) void mfma_gemm_kernel(MfmaArgs a)
{
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDSK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BC][LDSK];

    const int tile = blockIdx.x;
    const int ntiles = *a.count;
    const int4 dsc = a.desc[tile];  // in bounds for every tile of the grid
    if (tile >= ntiles) return;
    const int g = dsc.x;
    const int p0 = dsc.y;  // first position of the tile
    const int M = dsc.z;   // positions in the tile
    constexpr int m0 = 0;
    constexpr int NEURONS = GATEUP ? BC / 2 : BC;  // output neurons per tile
    const int n0 = blockIdx.y * NEURONS;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // this thread's share of the global loads: one 16-wide K half of one
    // A row and of one B column per step
    const int lr = tid >> 1, lh = tid & 1;
    const int am = m0 + lr;
    const bool a_ok = am < M;
    const uint16_t *arow = a.a + (size_t)(a_ok ? (GATEUP ? a.tok[p0 + am] : p0 + am) : 0) * a.lda;
    const int bmat = GATEUP ? (lr >= NEURONS) : 0;
    const int bn = n0 + (GATEUP ? (lr & (NEURONS - 1)) : lr);
    const bool b_ok = bn < a.n;
    const int brw = b_ok ? bn : 0;
    const char *brow = reinterpret_cast<const char *>(bmat ? a.w1 : a.w0) + (size_t)g * a.w_group_stride +
                       panel_unit_offset(brw, 0, a.row_bytes);
    const float *bsrow = PREC == kFloat32 ? nullptr
                                          : (bmat ? a.s1 : a.s0) + (size_t)g * a.s_group_stride +
                                                panel_scale_index(brw, 0, a.nblocks);

    uint4 av[2];
    uint32_t bv[8];
    auto load_global = [&](int k0) {
        if (a_ok) {
            const uint4 *p = reinterpret_cast<const uint4 *>(arow + k0 + lh * 16);
            av[0] = p[0];
            av[1] = p[1];
        } else {
            av[0] = make_uint4(0, 0, 0, 0);
            av[1] = make_uint4(0, 0, 0, 0);
        }
        if (b_ok) {
            dequant16<PREC>(brow, bsrow, k0 / 16 + lh, bv);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) bv[i] = 0;
        }
    };
    auto store_lds = [&](int buf) {
        uint4 *pa = reinterpret_cast<uint4 *>(&As[buf][lr][lh * 16]);
        pa[0] = av[0];
        pa[1] = av[1];
        uint4 *pb = reinterpret_cast<uint4 *>(&Bs[buf][lr][lh * 16]);
        pb[0] = make_uint4(bv[0], bv[1], bv[2], bv[3]);
        pb[1] = make_uint4(bv[4], bv[5], bv[6], bv[7]);
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // column base of the wave's two B tiles
    const int col0 = GATEUP ? wn * 32 : wn * 64;
    const int col1 = GATEUP ? NEURONS + wn * 32 : wn * 64 + 32;
    const int frow = lane & 31, fk = (lane >> 5) * 8;

    load_global(0);
    store_lds(0);
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < a.kp; k0 += BK) {
        const bool more = k0 + BK < a.kp;
        if (more) load_global(k0 + BK);
#pragma unroll
        for (int ks = 0; ks < BK; ks += 16) {
            bf16x8 af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(&As[buf][wm * 64 + i * 32 + frow][ks + fk]);
            bfr[0] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][col0 + frow][ks + fk]);
            bfr[1] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][col1 + frow][ks + fk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (more) store_lds(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // epilogue: lane holds column (lane & 31) of each 32x32 tile, rows
    // 8*(r/4) + 4*(lane/32) + r%4 for accumulator register r
    const int ccol = lane & 31, rq = (lane >> 5) * 4;
    if constexpr (GATEUP) {
        const int n = n0 + wn * 32 + ccol;
        if (n < a.n) {
            const float bg = a.b0[(size_t)g * a.n + n], bu = a.b1[(size_t)g * a.n + n];
            uint16_t *out = reinterpret_cast<uint16_t *>(a.out);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + rq + (r & 3);
                    if (m < M) {
                        float gv = acc[i][0][r] + bg;
                        float uv = acc[i][1][r] + bu;
                        if (a.clamp > 0.f) {
                            gv = fminf(gv, a.clamp);
                            uv = fminf(fmaxf(uv, -a.clamp), a.clamp);
                        }
                        const __bf16 h = (__bf16)(silu(gv) * uv);
                        out[(size_t)(p0 + m) * a.ldo + n] = __builtin_bit_cast(uint16_t, h);
                    }
                }
        }
    } else {
        float *out = reinterpret_cast<float *>(a.out);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + ccol;
            if (n >= a.n) continue;
            const float bd = a.b0[(size_t)g * a.n + n];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + rq + (r & 3);
                    if (m < M) out[(size_t)(p0 + m) * a.ldo + n] = acc[i][j][r] + bd;
                }
        }
    }
}

int mfma_tile_m() { return BM; }

namespace {

template <bool GATEUP>
hipError_t launch_mfma(const MfmaArgs &a, int precision, int max_tiles, hipStream_t s)
{
    if (max_tiles <= 0) return hipSuccess;
    if (a.kp % BK != 0) return hipErrorInvalidValue;
    constexpr int NEURONS = GATEUP ? BC / 2 : BC;
    dim3 grid(max_tiles, (a.n + NEURONS - 1) / NEURONS);
    switch (precision) {
    case kInt8: hipLaunchKernelGGL((mfma_gemm_kernel<kInt8, GATEUP>), grid, dim3(256), 0, s, a); break;
    case kFP4: hipLaunchKernelGGL((mfma_gemm_kernel<kFP4, GATEUP>), grid, dim3(256), 0, s, a); break;
    case kFloat32: hipLaunchKernelGGL((mfma_gemm_kernel<kFloat32, GATEUP>), grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_mfma_gateup(const MfmaArgs &a, int precision, int max_tiles, hipStream_t s)
{
    return launch_mfma<true>(a, precision, max_tiles, s);
}

hipError_t launch_mfma_down(const MfmaArgs &a, int precision, int max_tiles, hipStream_t s)
{
    return launch_mfma<false>(a, precision, max_tiles, s);
}

}  // namespace gtmoe
