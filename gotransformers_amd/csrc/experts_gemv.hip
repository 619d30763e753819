// Expert kernels for few tokens per expert (decode): a dequantizing GEMV
// that streams each weight row from HBM once per slice of at most 8 tokens,
// with the multiply-adds on the matrix cores at fp32-level accuracy.
//
// Work split: grid (panels of 64 output rows, token slices of all groups);
// a workgroup's NW waves share one panel and split its K range between them
// (NW = 4 or 8).
// Lane l of a wave owns row l of the panel, so with the panel layout of the
// weights every 16-byte load of the wave reads 1 KiB of codes contiguously.
//
// Arithmetic: v_mfma_f32_4x4x4_16b_bf16 holds 16 independent 4x4x4
// products; block b of it multiplies 4 tokens (A, broadcast from lanes 0-3)
// by 4 k-values of rows 4b..4b+3 (B, one row per lane), so a wave computes
// 4 tokens x 64 rows per instruction and lane l ends up holding row l's dot
// products for the 4 tokens -- no cross-lane reduction.  Weight codes are
// exact in bf16 (Int8 magnitudes <= 127, e2m1 values); the tokens are split
// as x = hi + lo with hi = bf16(x) and lo = bf16(x - hi), which represents
// x to about 2^-17 relative, and both halves go through the MFMA with fp32
// accumulation.  Four chained instructions cover one 16-value scale block;
// the block sum is then scaled once into an fp32 accumulator, the order of
// the reference's DotRow (lowprecision/rows.go:207-257).  float32 weights
// are split the same way (three products: hi*hi, lo*hi, hi*lo) and need no
// block scaling.
//
// Gate/up fuse the SwiGLU epilogue (feedforward/gatedfeedforward.go:49-57):
// hidden = act_g(gate + b_g) * act_u(up + b_u).  Down adds its bias.
#include "common.h"

namespace gtmoe {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Per precision: 16-byte units and scale blocks per pipeline chunk.
template <int PREC>
struct Chunk;
template <>
struct Chunk<kInt8> {
    static constexpr int U = 2, CB = 2;  // 32 values
};
template <>
struct Chunk<kFP4> {
    static constexpr int U = 1, CB = 2;  // 32 values
};
template <>
struct Chunk<kFloat32> {
    static constexpr int U = 4, CB = 1;  // 16 values
};

template <int PREC, int MATS>
struct ChunkRegs {
    uint4 c[MATS][Chunk<PREC>::U];
    float s[MATS][Chunk<PREC>::CB];
};

// Chunks in flight per wave (register ring): about 4 KiB of codes per wave
// (measured best; deeper rings lose more to occupancy than they gain).
template <int PREC, int MATS>
constexpr int ring_depth()
{
    return Chunk<PREC>::U * MATS >= 4 ? 1 : 2;
}

template <int I>
__device__ __forceinline__ uint32_t comp(const uint4 &v)
{
    return I == 0 ? v.x : I == 1 ? v.y : I == 2 ? v.z : v.w;
}

__device__ __forceinline__ s16x4 as_s16x4(uint32_t lo, uint32_t hi)
{
    const u32x2 v = {lo, hi};
    return __builtin_bit_cast(s16x4, v);
}

// bf16 bits of two floats that bf16 holds exactly (small integers): their
// upper halves, packed.
__device__ __forceinline__ uint32_t upper_halves(float lo, float hi)
{
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (nearest even) and packed, lo in the low half:
// one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16_rne_pair(float lo, float hi)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// x = hi + lo for two values: hi = bf16(x) rounded to nearest, lo = bf16 of
// the (exact) remainder.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t &hi, uint32_t &lo)
{
    hi = bf16_rne_pair(x0, x1);
    const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
    lo = bf16_rne_pair(x0 - h0, x1 - h1);
}

// B operand of step S (k-values 4S..4S+3) of block J of a chunk.
template <int PREC, int J, int S>
__device__ __forceinline__ s16x4 weights_step(const uint4 (&c)[Chunk<PREC>::U])
{
    if constexpr (PREC == kInt8) {
        const uint32_t d = comp<S>(c[J]);
        const float f0 = (float)(int)(int8_t)d, f1 = (float)(int)(int8_t)(d >> 8);
        const float f2 = (float)(int)(int8_t)(d >> 16), f3 = (float)(int)(int8_t)(d >> 24);
        return as_s16x4(upper_halves(f0, f1), upper_halves(f2, f3));
    } else {
        // FP4: block J is half J&1 of unit J/2; step S is bytes 2S, 2S+1 of
        // it, and each byte holds two values, the even one in the low nibble
        const uint32_t d = comp<(J & 1) * 2 + (S >> 1)>(c[J >> 1]);
        const auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, 1.0f, (S & 1) * 2);
        const auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, 1.0f, (S & 1) * 2 + 1);
        return as_s16x4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
    }
}
template <int S>
__device__ __forceinline__ void weights_step_f32(const uint4 (&c)[Chunk<kFloat32>::U], s16x4 &hi, s16x4 &lo)
{
    const uint4 v = c[S];
    uint32_t h01, l01, h23, l23;
    split_pair(__uint_as_float(v.x), __uint_as_float(v.y), h01, l01);
    split_pair(__uint_as_float(v.z), __uint_as_float(v.w), h23, l23);
    hi = as_s16x4(h01, h23);
    lo = as_s16x4(l01, l23);
}

__device__ __forceinline__ f32x4 mfma4(s16x4 a, s16x4 b, f32x4 c)
{
    // CBSZ = 4, ABID = 0: block 0's A (lanes 0-3, the tokens) is used by
    // all 16 blocks
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 4, 0, 0);
}

// x * sigmoid(x) with the hardware exp and reciprocal (about 1 ulp each)
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// The staged tokens: for every group of 8 k-values, NT tokens' bf16 hi
// values (16 bytes each), then the same for lo.  Lane reads of one token's
// 16 bytes for tokens 4q..4q+3 are contiguous and shared by the other lanes.
template <int NT>
struct Staged {
    const uint4 *hi;
    const uint4 *lo;
    __device__ __forceinline__ void read(int g8, int t, uint4 &h, uint4 &l) const
    {
        h = hi[g8 * NT + t];
        l = lo[g8 * NT + t];
    }
};

// Codes (and scales) of chunk ch of the lane's row, for every matrix.  A
// chunk of CB blocks starts at block ch*CB; its scales are CB consecutive
// floats of the row's 4-block scale group.
template <int PREC, int MATS>
__device__ __forceinline__ void load_chunk(ChunkRegs<PREC, MATS> &r, const char *const (&w)[MATS],
                                           const float *const (&sc)[MATS], int ch)
{
    constexpr int U = Chunk<PREC>::U, CB = Chunk<PREC>::CB;
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            r.c[m][u] = *reinterpret_cast<const uint4 *>(w[m] + (size_t)(ch * U + u) * 1024);
        if constexpr (PREC != kFloat32) {
            const int b = ch * CB;
            const float *p = sc[m] + (size_t)(b >> 2) * 256 + (b & 3);
            if constexpr (CB == 4) {
                const float4 v = *reinterpret_cast<const float4 *>(p);
                r.s[m][0] = v.x;
                r.s[m][1] = v.y;
                r.s[m][2] = v.z;
                r.s[m][3] = v.w;
            } else if constexpr (CB == 2) {
                const float2 v = *reinterpret_cast<const float2 *>(p);
                r.s[m][0] = v.x;
                r.s[m][1] = v.y;
            } else {
                r.s[m][0] = *p;
            }
        }
    }
}

// One step of one block: A operands of the NQ token quads for k-values
// 4S..4S+3, against every matrix.
template <int PREC, int MATS, int NQ, int J, int S>
__device__ __forceinline__ void block_step(const ChunkRegs<PREC, MATS> &r, const uint4 (&ah)[NQ],
                                           const uint4 (&al)[NQ], f32x4 (&blk)[MATS][NQ])
{
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const s16x4 xh = (S & 1) ? as_s16x4(ah[q].z, ah[q].w) : as_s16x4(ah[q].x, ah[q].y);
        const s16x4 xl = (S & 1) ? as_s16x4(al[q].z, al[q].w) : as_s16x4(al[q].x, al[q].y);
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            if constexpr (PREC == kFloat32) {
                s16x4 wh, wl;
                weights_step_f32<S>(r.c[m], wh, wl);
                blk[m][q] = mfma4(xh, wh, blk[m][q]);
                blk[m][q] = mfma4(xl, wh, blk[m][q]);
                blk[m][q] = mfma4(xh, wl, blk[m][q]);
            } else {
                const s16x4 w = weights_step<PREC, J, S>(r.c[m]);
                blk[m][q] = mfma4(xh, w, blk[m][q]);
                blk[m][q] = mfma4(xl, w, blk[m][q]);
            }
        }
    }
}

template <int PREC, int MATS, int NQ, int J>
__device__ __forceinline__ void chunk_block(const ChunkRegs<PREC, MATS> &r, const Staged<4 * NQ> &xs, int g8,
                                            int tl, f32x4 (&acc)[MATS][NQ])
{
    f32x4 blk[MATS][NQ];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int q = 0; q < NQ; ++q) blk[m][q] = PREC == kFloat32 ? acc[m][q] : f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 ah[NQ], al[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) xs.read(g8, 4 * q + tl, ah[q], al[q]);
    block_step<PREC, MATS, NQ, J, 0>(r, ah, al, blk);
    block_step<PREC, MATS, NQ, J, 1>(r, ah, al, blk);
#pragma unroll
    for (int q = 0; q < NQ; ++q) xs.read(g8 + 1, 4 * q + tl, ah[q], al[q]);
    block_step<PREC, MATS, NQ, J, 2>(r, ah, al, blk);
    block_step<PREC, MATS, NQ, J, 3>(r, ah, al, blk);
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            if constexpr (PREC == kFloat32) {
                acc[m][q] = blk[m][q];
            } else {
                const float s = r.s[m][J];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[m][q][i] = fmaf(blk[m][q][i], s, acc[m][q][i]);
            }
        }
}

template <int PREC, int MATS, int NQ>
__device__ __forceinline__ void compute_chunk(const ChunkRegs<PREC, MATS> &r, const Staged<4 * NQ> &xs, int ch,
                                              int tl, f32x4 (&acc)[MATS][NQ])
{
    constexpr int CB = Chunk<PREC>::CB;
    const int g8 = ch * CB * 2;  // groups of 8 k-values
    chunk_block<PREC, MATS, NQ, 0>(r, xs, g8, tl, acc);
    if constexpr (CB > 1) chunk_block<PREC, MATS, NQ, 1>(r, xs, g8 + 2, tl, acc);
    if constexpr (CB > 2) {
        chunk_block<PREC, MATS, NQ, 2>(r, xs, g8 + 4, tl, acc);
        chunk_block<PREC, MATS, NQ, 3>(r, xs, g8 + 6, tl, acc);
    }
}

// One slice of M <= 4*NQ tokens of group g against panel `panel`.
template <int PREC, bool GATEUP, int NW, int NQ>
__device__ __forceinline__ void run_slice(const GemvArgs &a, char *lds, int g, int p0, int M, int panel)
{
    constexpr int NT = 4 * NQ;
    constexpr int MATS = GATEUP ? 2 : 1;
    constexpr int CB = Chunk<PREC>::CB;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kp = a.nblocks * 16;
    const int ng8 = kp / 8;

    // this wave's chunks of K; the first chunks' loads (and the epilogue's
    // biases) are issued before the token rows are staged
    const int nch = a.nblocks / CB;
    const int c0 = wave * nch / NW, c1 = (wave + 1) * nch / NW;
    const char *w[MATS];
    const float *sc[MATS];
    const size_t wpanel = (size_t)panel * 64 * a.row_bytes + (size_t)lane * 16;
    const size_t spanel = (size_t)panel * 64 * a.nblocks + (size_t)lane * 4;
    w[0] = reinterpret_cast<const char *>(a.w0) + (size_t)g * a.w_group_stride + wpanel;
    sc[0] = PREC == kFloat32 ? nullptr : a.s0 + (size_t)g * a.s_group_stride + spanel;
    if constexpr (GATEUP) {
        w[1] = reinterpret_cast<const char *>(a.w1) + (size_t)g * a.w_group_stride + wpanel;
        sc[1] = PREC == kFloat32 ? nullptr : a.s1 + (size_t)g * a.s_group_stride + spanel;
    }
    constexpr int kDepth = ring_depth<PREC, MATS>();
    ChunkRegs<PREC, MATS> r[kDepth];
#pragma unroll
    for (int i = 0; i < kDepth; ++i)
        if (c0 + i < c1) load_chunk<PREC, MATS>(r[i], w, sc, c0 + i);
    const int row = panel * 64 + lane;
    const bool writer = wave < 4 && row < a.rows;
    float bias[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) bias[m] = writer ? (m == 0 ? a.b0 : a.b1)[(size_t)g * a.rows + row] : 0.f;

    // stage the slice's token rows as bf16 hi / lo
    uint4 *xhi = reinterpret_cast<uint4 *>(lds);
    uint4 *xlo = xhi + (size_t)ng8 * NT;
    for (int idx = tid; idx < NT * ng8; idx += blockDim.x) {
        const int t = idx / ng8, g8 = idx - t * ng8;
        uint4 h = make_uint4(0, 0, 0, 0), l = make_uint4(0, 0, 0, 0);
        if (t < M) {
            const int src = GATEUP ? a.tok[p0 + t] : p0 + t;
            const float4 *p = reinterpret_cast<const float4 *>(a.in + (size_t)src * a.ld_in) + 2 * g8;
            const float4 v0 = p[0], v1 = p[1];
            split_pair(v0.x, v0.y, h.x, l.x);
            split_pair(v0.z, v0.w, h.y, l.y);
            split_pair(v1.x, v1.y, h.z, l.z);
            split_pair(v1.z, v1.w, h.w, l.w);
        }
        xhi[g8 * NT + t] = h;
        xlo[g8 * NT + t] = l;
    }
    __syncthreads();

    const Staged<NT> xs{xhi, xlo};
    const int tl = lane & 3;

    f32x4 acc[MATS][NQ];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int q = 0; q < NQ; ++q) acc[m][q] = f32x4{0.f, 0.f, 0.f, 0.f};

    // ring of kDepth chunk buffers: once chunk ch is computed, its buffer
    // takes chunk ch + kDepth
    for (int ch = c0; ch < c1; ch += kDepth) {
#pragma unroll
        for (int j = 0; j < kDepth; ++j) {
            if (ch + j < c1) {
                compute_chunk<PREC, MATS, NQ>(r[j], xs, ch + j, tl, acc);
                if (ch + j + kDepth < c1) load_chunk<PREC, MATS>(r[j], w, sc, ch + j + kDepth);
            }
        }
    }

    // sum the NW partial K ranges through LDS; wave v < 4 then finishes
    // tokens 4q + v of every quad
    __syncthreads();  // all reads of the staged tokens are done
    float *red = reinterpret_cast<float *>(lds);
    auto slot = [&](int wv, int m, int q, int i) { return (((wv * MATS + m) * NQ + q) * 4 + i) * 64 + lane; };
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[slot(wave, m, q, i)] = acc[m][q][i];
    __syncthreads();
    if (!writer) return;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int t = 4 * q + wave;
        if (t >= M) continue;
        float v[MATS];
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            float s = 0.f;
#pragma unroll
            for (int wv = 0; wv < NW; ++wv) s += red[slot(wv, m, q, wave)];
            v[m] = s;
        }
        float *out = a.out + (size_t)(p0 + t) * a.ld_out + row;
        if constexpr (GATEUP) {
            float gv = v[0] + bias[0];
            float uv = v[1] + bias[MATS - 1];
            if (a.clamp > 0.f) {
                gv = fminf(gv, a.clamp);                   // ClampedSiLU: x > L -> silu(L)
                uv = fminf(fmaxf(uv, -a.clamp), a.clamp);  // ClampedLinear
            }
            *out = silu(gv) * uv;
        } else {
            *out = v[0] + bias[0];
        }
    }
}

}  // namespace

// blockIdx.x = panel of 64 output rows, blockIdx.y = token slice (the
// dispatch wrote the slice count and a (group, first position, positions)
// descriptor per slice; slices past the last exit).
template <int PREC, bool GATEUP, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_kernel(GemvArgs a)
{
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int item = blockIdx.y;
    const int nslices = *a.count;
    const int4 dsc = a.desc[item];  // in bounds for every slice of the grid
    if (item >= nslices) return;    // workgroup-uniform
    const int g = dsc.x, p0 = dsc.y, M = dsc.z;
    if (M <= 0) return;  // workgroup-uniform
    if (M <= 4) run_slice<PREC, GATEUP, NW, 1>(a, lds, g, p0, M, blockIdx.x);
    else run_slice<PREC, GATEUP, NW, 2>(a, lds, g, p0, M, blockIdx.x);
}

namespace {

// LDS: the staged tokens (2 x 2 bytes per k-value and token) or the
// cross-wave partial sums, whichever is larger.
size_t gemv_lds_bytes(int nblocks, bool gateup, int nw)
{
    const size_t staged = (size_t)nblocks * 16 * 2 * 2 * kGemvSlice;
    const size_t red = (size_t)nw * (gateup ? 2 : 1) * 2 * 4 * 64 * sizeof(float);
    return staged > red ? staged : red;
}

template <int PREC, bool GATEUP, int NW>
hipError_t launch_nw(const GemvArgs &a, int max_slices, hipStream_t s)
{
    const size_t lds = gemv_lds_bytes(a.nblocks, GATEUP, NW);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_kernel<PREC, GATEUP, NW>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((a.rows + 63) / 64, max_slices);
    hipLaunchKernelGGL((gemv_kernel<PREC, GATEUP, NW>), grid, dim3(64 * NW), lds, s, a);
    return hipGetLastError();
}

// Waves per workgroup: eight when K holds at least two chunks per wave,
// else four (the epilogue's waves).
template <int PREC>
int waves_for(const GemvArgs &a)
{
    const int nch = a.nblocks / Chunk<PREC>::CB;
    return nch >= 16 ? 8 : 4;
}

template <bool GATEUP, int PREC>
hipError_t launch_prec(const GemvArgs &a, int max_slices, hipStream_t s)
{
    static_assert(kGemvSlice <= 8, "at most two token quads per slice");
    if (a.nblocks % Chunk<PREC>::CB) return hipErrorInvalidValue;
    if (waves_for<PREC>(a) == 8) return launch_nw<PREC, GATEUP, 8>(a, max_slices, s);
    return launch_nw<PREC, GATEUP, 4>(a, max_slices, s);
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
