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
#include <algorithm>

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

// Chunks in flight per wave (register ring): three for FP4 gate/up, whose
// chunks are half the bytes of Int8's (C5 decode gate/up 1183 -> 1158 us per
// step), two otherwise (a third chunk measured slower for Int8).
template <int PREC, int MATS, int NQ>
constexpr int ring_depth()
{
    return PREC == kFP4 && MATS == 2 ? 3 : 2;
}

// One weight matrix's panel as buffer resources: the panel's codes (64 rows
// side by side in 16-byte units) and its scales.  The resources live in
// scalar registers; a lane addresses its row with one 32-bit offset and a
// chunk with a scalar offset, so the loads cost one vector register of
// address in all, and a load past the panel returns zeros.
struct PanelSrc {
    __amdgpu_buffer_rsrc_t codes;
    __amdgpu_buffer_rsrc_t scales;
};

// descriptor word 3 for raw (untyped) buffer access on CDNA
constexpr int kRawBufferWord3 = 0x00020000;

template <int I>
__device__ __forceinline__ uint32_t comp(const uint4 &v)
{
    return I == 0 ? v.x : I == 1 ? v.y : I == 2 ? v.z : v.w;
}

__device__ __forceinline__ uint32_t comp_rt(const uint4 &v, int i)
{
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
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
// floats of the row's 4-block scale group.  vo = lane * 16; ch is uniform
// across the wave.
template <int PREC, int MATS>
__device__ __forceinline__ void load_chunk(ChunkRegs<PREC, MATS> &r, const PanelSrc (&src)[MATS], uint32_t vo, int ch)
{
    constexpr int U = Chunk<PREC>::U, CB = Chunk<PREC>::CB;
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            r.c[m][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src[m].codes, vo,
                                                                                        (ch * U + u) * 1024, 0));
        if constexpr (PREC != kFloat32) {
            const int b = ch * CB;
            const int so = (b >> 2) * 1024 + (b & 3) * 4;
            if constexpr (CB == 4) {
                const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(src[m].scales, vo, so, 0));
                r.s[m][0] = v.x;
                r.s[m][1] = v.y;
                r.s[m][2] = v.z;
                r.s[m][3] = v.w;
            } else if constexpr (CB == 2) {
                const float2 v = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(src[m].scales, vo, so, 0));
                r.s[m][0] = v.x;
                r.s[m][1] = v.y;
            } else {
                r.s[m][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src[m].scales, vo, so, 0));
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

// Where the M rows of a slice come from: positions p0 .. p0 + M - 1 of the
// dispatch (kByPosition), the routed (token, slot) entries list[0 .. M) of one
// expert, entry i = token * k + slot (kByEntry), or tokens t0 .. t0 + M - 1 of
// shared expert s (kShared).
enum { kByPosition = 0, kByEntry = 1, kShared = 2 };
struct SliceSrc {
    int mode;
    int p0;
    const int *list;
    int t0, s;
};

// input row (token row for gate/up, hidden row for down) and output row of
// slice token t
template <bool GATEUP, int MODE>
__device__ __forceinline__ int slice_in_row(const GemvArgs &a, const SliceSrc &sl, int t)
{
    if constexpr (MODE == kByPosition) return GATEUP ? a.tok[sl.p0 + t] : sl.p0 + t;
    else if constexpr (MODE == kByEntry) return GATEUP ? sl.list[t] / a.k : a.S * a.T + sl.list[t];
    else return GATEUP ? sl.t0 + t : sl.s * a.T + sl.t0 + t;
}
template <int MODE>
__device__ __forceinline__ int slice_out_row(const GemvArgs &a, const SliceSrc &sl, int t)
{
    if constexpr (MODE == kByPosition) return sl.p0 + t;
    else if constexpr (MODE == kByEntry) return a.S * a.T + sl.list[t];
    else return sl.s * a.T + sl.t0 + t;
}

// One slice of M <= 4*NQ tokens of group g against panels panel0 ..
// panel0 + PPW - 1: the NW waves are PPW sets of WPP = NW / PPW, set pi on
// panel panel0 + pi, its waves splitting K; the sets share the staged tokens.
template <int PREC, bool GATEUP, int NW, int NQ, int MODE, int PPW>
__device__ __forceinline__ void run_slice(const GemvArgs &a, char *lds, int g, const SliceSrc &sl, int M,
                                          int panel0)
{
    static_assert(NW % PPW == 0, "whole sets of waves per panel");
    constexpr int WPP = NW / PPW;
    constexpr int NT = 4 * NQ;
    constexpr int MATS = GATEUP ? 2 : 1;
    constexpr int CB = Chunk<PREC>::CB;
    // the empty asm hides where tid comes from, so that a caller's loop over
    // slices cannot hoist the lane-dependent set-up out of the loop and keep
    // it live across the main loop (that costs about 16 VGPRs)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kp = a.nblocks * 16;
    const int ng8 = kp / 8;

    // this wave's panel and chunks of K; the first chunks' loads (and the
    // epilogue's biases) are issued before the token rows are staged
    const int pi = wave / WPP, kw = wave - pi * WPP;
    const int panel = panel0 + pi;
    const bool in_matrix = panel * 64 < a.rows;  // the last workgroup's sets may lie past the rows
    const int nch = a.nblocks / CB;
    const int c0 = kw * nch / WPP, c1 = (kw + 1) * nch / WPP;
    PanelSrc src[MATS];
    {
        const size_t wpanel = (size_t)panel * 64 * a.row_bytes;
        const int wbytes = in_matrix ? 64 * a.row_bytes : 0;  // past the rows: every load reads zeros
        src[0].codes = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char *>(reinterpret_cast<const char *>(a.w0)) + (size_t)g * a.w_group_stride + wpanel, 0, wbytes,
            kRawBufferWord3);
        if constexpr (GATEUP)
            src[1].codes = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char *>(reinterpret_cast<const char *>(a.w1)) + (size_t)g * a.w_group_stride + wpanel, 0,
                wbytes, kRawBufferWord3);
        if constexpr (PREC != kFloat32) {
            const size_t spanel = (size_t)panel * 64 * a.nblocks;
            const int sbytes = in_matrix ? 64 * a.nblocks * 4 : 0;
            src[0].scales = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(a.s0) + (size_t)g * a.s_group_stride + spanel, 0, sbytes, kRawBufferWord3);
            if constexpr (GATEUP)
                src[1].scales = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<float *>(a.s1) + (size_t)g * a.s_group_stride + spanel, 0, sbytes, kRawBufferWord3);
        }
    }
    const uint32_t vo = (uint32_t)lane * 16;

    // The slice's tokens for this wave's K range (groups of 8 k-values
    // [g0, g0 + gn)) are staged as bf16 hi / lo by the PPW waves that share
    // the range: one wave (PPW = 1) needs no workgroup barrier before its
    // main loop.  Item i of a lane is token lane % NT (64 is a multiple of
    // NT) at group g0 + idx / NT, idx = lane + 64 (pi + PPW i): the lanes'
    // 16-byte LDS stores are contiguous.  The token loads are issued before
    // the weight prefetch, the conversion after it, so the wait for the
    // tokens overlaps the first weight chunks' latency.  Padding tokens
    // (t >= M) read past the input buffer and get zeros.
    const int g0 = c0 * CB * 2, gn = (c1 - c0) * CB * 2;
    const int items = NT * gn;
    const int ipl = (items + 64 * PPW - 1) / (64 * PPW);  // items per lane
    auto item = [&](int i) { return lane + 64 * (pi + PPW * i); };
    const int t = lane % NT;
    uint32_t rowoff = 0x80000000u;  // past the buffer: zeros
    if (t < M) rowoff = (uint32_t)slice_in_row<GATEUP, MODE>(a, sl, t) * (uint32_t)a.ld_in * 4u;
    const __amdgpu_buffer_rsrc_t xin = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.in), 0, (int)(a.in_rows * a.ld_in * 4), kRawBufferWord3);
    auto token_off = [&](int idx) {
        return idx < items ? rowoff + (uint32_t)(g0 + idx / NT) * 32u : 0x80000000u;
    };
    auto stage = [&](int idx, const float4 &v0, const float4 &v1, uint4 *xhi, uint4 *xlo) {
        uint4 h, l;
        split_pair(v0.x, v0.y, h.x, l.x);
        split_pair(v0.z, v0.w, h.y, l.y);
        split_pair(v1.x, v1.y, h.z, l.z);
        split_pair(v1.z, v1.w, h.w, l.w);
        const int at = (g0 + idx / NT) * NT + t;
        xhi[at] = h;
        xlo[at] = l;
    };
    // the first kEarly items per lane go ahead of the weight prefetch (all
    // of them up to 2 KiB of K per wave); any others are staged after it
    constexpr int kEarly = 2;
    float4 xv[kEarly][2];
#pragma unroll
    for (int i = 0; i < kEarly; ++i) {
        if (i < ipl) {  // wave-uniform
            const uint32_t off = token_off(item(i));
            xv[i][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xin, off, 0, 0));
            xv[i][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xin, off, 16, 0));
        }
    }

    // the epilogue's biases are requested before the ring, so that the loads
    // in flight at the main loop's entry are the ring's alone, in ring order,
    // as on its back edge
    const int row = panel * 64 + lane;
    const bool writer = kw < 4 && row < a.rows;
    float bias[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) bias[m] = writer ? (m == 0 ? a.b0 : a.b1)[(size_t)g * a.rows + row] : 0.f;

    constexpr int kDepth = ring_depth<PREC, MATS, NQ>();
    // Every load of the ring is issued unconditionally, so that the compiler
    // can count the loads in flight and wait for one chunk at a time (loads
    // under a branch make it wait for all of them).  Past the wave's last
    // chunk the ring re-loads that chunk: cache hits, never used.
    const int clast = c1 > c0 ? c1 - 1 : c0;
    ChunkRegs<PREC, MATS> r[kDepth];
#pragma unroll
    for (int i = 0; i < kDepth; ++i) {
        // the scheduling barriers keep the ring's loads in ring order here
        // and in the loop: the compiler's wait before each chunk must hold
        // for the loads in flight both at the loop's entry and on its back
        // edge, so a different order here (say all codes, then all scales)
        // would make it wait for the next chunk's loads as well
        __builtin_amdgcn_sched_barrier(0);
        load_chunk<PREC, MATS>(r[i], src, vo, min(c0 + i, clast));
    }
    __builtin_amdgcn_sched_barrier(0);

    uint4 *xhi = reinterpret_cast<uint4 *>(lds);
    uint4 *xlo = xhi + (size_t)ng8 * NT;
#pragma unroll
    for (int i = 0; i < kEarly; ++i) {
        const int idx = item(i);
        if (i < ipl && idx < items) stage(idx, xv[i][0], xv[i][1], xhi, xlo);
    }
    for (int i = kEarly; i < ipl; ++i) {
        const int idx = item(i);
        const uint32_t off = token_off(idx);
        const float4 v0 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xin, off, 0, 0));
        const float4 v1 = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xin, off, 16, 0));
        if (idx < items) stage(idx, v0, v1, xhi, xlo);
    }
    // With one panel the wave reads back only what it wrote; LDS operations
    // of a wave are performed in order, so a wait for its own stores is
    // enough.  With several, every wave waits for its own stores and then
    // for the other waves at a bare barrier (no wait for the weight loads in
    // flight).  The fences keep the compiler from moving LDS accesses across.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    if constexpr (PPW == 1) __builtin_amdgcn_wave_barrier();
    else __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const Staged<NT> xs{xhi, xlo};
    const int tl = lane & 3;

    f32x4 acc[MATS][NQ];
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int q = 0; q < NQ; ++q) acc[m][q] = f32x4{0.f, 0.f, 0.f, 0.f};

    // ring of kDepth chunk buffers: once chunk ch is computed, its buffer
    // takes chunk ch + kDepth.  The loop body computes every buffer with no
    // branch, so the loads in flight on its back edge are exactly the ring's
    // and the compiler waits, before each chunk, for that chunk's loads only
    // (with a conditional compute in the body it also waited for the next
    // buffer's loads, leaving about one chunk in flight); the last
    // c1 - ch < kDepth chunks, already in the ring, are computed after it.
    int ch = c0;
    for (; ch + kDepth <= c1; ch += kDepth) {
#pragma unroll
        for (int j = 0; j < kDepth; ++j) {
            compute_chunk<PREC, MATS, NQ>(r[j], xs, ch + j, tl, acc);
            __builtin_amdgcn_sched_barrier(0);
            load_chunk<PREC, MATS>(r[j], src, vo, min(ch + j + kDepth, clast));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int j = 0; j + 1 < kDepth; ++j)
        if (ch + j < c1) compute_chunk<PREC, MATS, NQ>(r[j], xs, ch + j, tl, acc);

    // sum the partial K ranges of each panel through LDS; wave kw < 4 of the
    // panel's set then finishes tokens 4q + v of every quad, v = kw, kw +
    // WPP, ... < 4
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
    for (int tq = kw; tq < 4; tq += WPP)
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int t = 4 * q + tq;
        if (t >= M) continue;
        float v[MATS];
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            float s = 0.f;
#pragma unroll
            for (int wv = 0; wv < WPP; ++wv) s += red[slot(pi * WPP + wv, m, q, tq)];
            v[m] = s;
        }
        const size_t orow = (size_t)slice_out_row<MODE>(a, sl, t) * a.ld_out;
        float *out = a.out + orow + row;
        if (a.raw) {  // the bare products (the adapter path adds its terms and the bias)
            *out = v[0];
            if constexpr (GATEUP) a.raw_up[orow + row] = v[MATS - 1];
        } else if constexpr (GATEUP) {
            float gv = v[0] + bias[0];
            float uv = v[1] + bias[MATS - 1];
            if (a.clamp > 0.f) {
                gv = fminf(gv, a.clamp);                   // ClampedSiLU: x > L -> silu(L)
                uv = fminf(fmaxf(uv, -a.clamp), a.clamp);  // ClampedLinear
            }
            *out = silu(gv) * uv;
        } else if (a.final_out) {
            // the combine of mixtureofexperts.go:192-205 for at most two
            // contributions per row: shared experts with weight 1, a routed
            // expert with its token's gate for it
            int tk;
            float wgt = 1.0f;
            if constexpr (MODE == kByEntry) {
                tk = sl.list[t] / a.k;
                wgt = a.gates32[sl.list[t]];
            } else if constexpr (MODE == kShared) {
                tk = sl.t0 + t;
            } else {
                tk = a.tok_all[sl.p0 + t];
                if (g >= a.S) {
                    const int e = g - a.S;
                    for (int j = 0; j < a.k; ++j)
                        if (a.chosen[(size_t)tk * a.k + j] == e) wgt = a.gates32[(size_t)tk * a.k + j];
                }
            }
            __hip_atomic_fetch_add(a.final_out + (size_t)tk * a.rows + row, wgt * (v[0] + bias[0]), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        } else {
            *out = v[0] + bias[0];
        }
    }
}

}  // namespace

// blockIdx.x = panel of 64 output rows, blockIdx.y = token slice (the
// dispatch wrote the slice count and a (group, first position, positions)
// descriptor per slice; slices past the last exit).
template <int PREC, bool GATEUP, int NW, bool SELF, int PPW>
__global__ __launch_bounds__(64 * NW) void gemv_kernel(GemvArgs a)
{
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int y = blockIdx.y;
    if constexpr (!SELF) {
        const int nslices = *a.count;
        const int4 dsc = a.desc[y];  // in bounds for every slice of the grid
        if (y >= nslices) return;    // workgroup-uniform
        const SliceSrc sl{kByPosition, dsc.y, nullptr, 0, 0};
        if (dsc.z <= 0) return;  // workgroup-uniform
        const int panel0 = blockIdx.x * PPW;
        if (dsc.z <= 4) run_slice<PREC, GATEUP, NW, 1, kByPosition, PPW>(a, lds, dsc.x, sl, dsc.z, panel0);
        else run_slice<PREC, GATEUP, NW, 2, kByPosition, PPW>(a, lds, dsc.x, sl, dsc.z, panel0);
        return;
    } else {
        const int nsh = a.S * a.shared_slices;
        if (y < nsh) {  // 8 tokens of a shared expert
            const int s = y / a.shared_slices;
            const SliceSrc sl{kShared, 0, nullptr, (y - s * a.shared_slices) * kGemvSlice, s};
            const int m = min(kGemvSlice, a.T - sl.t0);
            const int panel0 = blockIdx.x * PPW;
            if (m <= 4) run_slice<PREC, GATEUP, NW, 1, kShared, PPW>(a, lds, s, sl, m, panel0);
            else run_slice<PREC, GATEUP, NW, 2, kShared, PPW>(a, lds, s, sl, m, panel0);
            return;
        }
        // routed expert e: its entries in token order (the order of the
        // reference's rowsForExpert, mixtureofexperts.go:175-180), found by
        // wave 0 with ballots over `chosen` (four loads in flight per
        // round); this workgroup takes passes par, par + 2, ... of 8
        // entries.  Rows [nsh, nsh + E) are the first halves, [nsh + E,
        // nsh + 2E) the second, so the second halves (mostly without work at
        // decode loads) are dispatched after every first half.
        const int e = (y - nsh) % a.E, par = (y - nsh) / a.E;  // y < nsh + 2E
        int *list = reinterpret_cast<int *>(lds + a.list_off);
        int *count = list + a.T * a.k;
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            const int n = a.T * a.k;
            int c = 0;
            for (int b0 = 0; b0 < n; b0 += 256) {
                int ch[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) ch[j] = a.chosen[min(b0 + j * 64 + lane, n - 1)];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = b0 + j * 64 + lane;
                    const bool hit = i < n && ch[j] == e;
                    const unsigned long long bal = __ballot(hit);
                    if (hit) list[c + __popcll(bal & ((1ull << lane) - 1ull))] = i;
                    c += __popcll(bal);
                }
            }
            if (lane == 0) *count = c;
        }
        __syncthreads();
        const int c = __builtin_amdgcn_readfirstlane(*count);
        for (int first = par * kGemvSlice; first < c; first += 2 * kGemvSlice) {
            const SliceSrc sl{kByEntry, 0, list + first, 0, 0};
            const int m = min(kGemvSlice, c - first);
            int g = a.S + e, panel0 = blockIdx.x * PPW;
            asm volatile("" : "+s"(g), "+s"(panel0));  // as for tid in run_slice
            if (m <= 4) run_slice<PREC, GATEUP, NW, 1, kByEntry, PPW>(a, lds, g, sl, m, panel0);
            else run_slice<PREC, GATEUP, NW, 2, kByEntry, PPW>(a, lds, g, sl, m, panel0);
            __syncthreads();  // the next pass re-stages the LDS
        }
    }
}

// A few tokens (T <= kFewTokens, self-dispatching): only k T routed
// (token, slot) pairs and S T shared (expert, token) pairs have work, so
// each pair's rows are spread over the whole GPU.  A workgroup takes R rows
// of one pair (R divides the 64-row panel) and all of K; lane l of each of
// its 4 waves owns row l % R and unit phase l / R, so a load of the wave
// reads R rows' 16-byte units side by side (R x 16 contiguous bytes per
// phase).  Phase p of the workgroup takes units p, p + 4 * 64 / R, ... of
// its rows.  The pair's input row is staged once in LDS as fp32.  Per
// 16-value block: the codes times the input values, summed in order with
// fp32 FMAs, then times the block's scale into the lane's sum (the order of
// lowprecision/rows.go:207-257 within a block); the lanes' sums are added
// across phases and waves.  Same epilogues as gemv_kernel.
template <int PREC, bool GATEUP, int R>
__global__ __launch_bounds__(256) void gemv_few_kernel(GemvArgs a)
{
    constexpr int MATS = GATEUP ? 2 : 1;
    constexpr int PH = 64 / R;       // unit phases per wave
    constexpr int STRIDE = 4 * PH;   // units between a lane's units
    constexpr int VPU = PREC == kInt8 ? 16 : 32;  // values per 16-byte unit
    extern __shared__ __attribute__((aligned(16))) char lds[];
    float *xs = reinterpret_cast<float *>(lds);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // token t = blockIdx.z; blockIdx.y = shared expert s < S (row s T + t
    // of the self-dispatch layout), else routed slot j = blockIdx.y - S
    // (entry t k + j, row S T + t k + j).  The input row (the token, or the
    // pair's hidden row) is requested first: it does not depend on the
    // routing.
    const int t = blockIdx.z, yy = blockIdx.y;
    const int n0 = blockIdx.x * R;
    const int K = a.nblocks * 16;
    const int entry = t * a.k + yy - a.S;  // routed pairs only
    const int y = yy < a.S ? yy * a.T + t : a.S * a.T + entry;
    const int in_row = GATEUP ? t : y;
    const int out_row = y;
    const float4 *xin = reinterpret_cast<const float4 *>(a.in + (size_t)in_row * a.ld_in);
    // K <= 4096: four float4 per thread, loaded unconditionally (the index
    // clamped) and stored unconditionally into a 16 KiB row buffer (the
    // copies past K are never read): with a store under a branch the
    // compiler moved each load into the branch, behind the weight loads and
    // with a wait of its own
    float4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = xin[min(tid + 256 * i, K / 4 - 1)];
    int g = yy;
    float wgt = 1.0f;
    if (yy >= a.S) {
        g = a.S + a.chosen[entry];
        wgt = a.gates32[entry];
    }
    g = __builtin_amdgcn_readfirstlane(g);
    const int nunits = a.row_bytes / 16;
    const int r = lane % R;
    const int n = n0 + r;
    const int panel = n0 >> 6, prow = (n0 & 63) + r;

    PanelSrc src[MATS];
    {
        const size_t wpanel = (size_t)panel * 64 * a.row_bytes;
        const int wbytes = 64 * a.row_bytes;
        const size_t spanel = (size_t)panel * 64 * a.nblocks;
        const int sbytes = 64 * a.nblocks * 4;
#pragma unroll
        for (int m = 0; m < MATS; ++m) {
            const void *w = m == 0 ? a.w0 : a.w1;
            const float *sc = m == 0 ? a.s0 : a.s1;
            src[m].codes = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char *>(reinterpret_cast<const char *>(w)) + (size_t)g * a.w_group_stride + wpanel, 0,
                wbytes, kRawBufferWord3);
            src[m].scales = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(sc) + (size_t)g * a.s_group_stride + spanel, 0, sbytes, kRawBufferWord3);
        }
    }
    constexpr int UB = 4;  // units of a lane in flight together
    float sum[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) sum[m] = 0.f;
    const int ulanes = nunits / STRIDE;  // units per lane (the launcher checks the division)

    // unit u = U0 + q of the lane: U0 = wave PH + j STRIDE (uniform, a
    // multiple of 4) and q = lane / R; its first scale block b = u BPU sits
    // at (b / 4) 1024 + (b % 4) 4 + row 16 in the panel's scales
    constexpr int BPU = VPU / 16;  // scale blocks per unit
    const int q = lane / R;
    const uint32_t cvo = (uint32_t)prow * 16u + (uint32_t)q * 1024u;
    const uint32_t svo = (uint32_t)prow * 16u + (uint32_t)((q * BPU) >> 2) * 1024u + (uint32_t)((q * BPU) & 3) * 4u;
    uint4 c[UB][MATS];
    float sc[UB][MATS][BPU];
    // the lane's units j0 .. j0 + UB - 1 (past its last unit: the last unit
    // again, never used)
    auto load_units = [&](int j0) {
#pragma unroll
        for (int i = 0; i < UB; ++i) {
            const int U0 = wave * PH + min(j0 + i, ulanes - 1) * STRIDE;
#pragma unroll
            for (int m = 0; m < MATS; ++m) {
                c[i][m] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src[m].codes, cvo,
                                                                                         U0 * 1024, 0));
                const int soff = (U0 * BPU / 4) * 1024;
                if constexpr (BPU == 1) {
                    sc[i][m][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src[m].scales, svo,
                                                                                                soff, 0));
                } else {
                    const float2 v = __builtin_bit_cast(
                        float2, __builtin_amdgcn_raw_buffer_load_b64(src[m].scales, svo, soff, 0));
                    sc[i][m][0] = v.x;
                    sc[i][m][1] = v.y;
                }
            }
        }
    };
    load_units(0);
    // the input row into LDS (K fp32 values, K a multiple of 64)
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<float4 *>(xs)[tid + 256 * i] = xv[i];
    __syncthreads();
    for (int j0 = 0;;) {
#pragma unroll
        for (int i = 0; i < UB; ++i) {
            if (j0 + i >= ulanes) break;  // wave-uniform
            const int u = wave * PH + (j0 + i) * STRIDE + q;
            const float4 *xq = reinterpret_cast<const float4 *>(xs + u * VPU);
#pragma unroll
            for (int blk = 0; blk < BPU; ++blk) {
                float xb[16];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float4 v = xq[blk * 4 + h];
                    xb[4 * h] = v.x;
                    xb[4 * h + 1] = v.y;
                    xb[4 * h + 2] = v.z;
                    xb[4 * h + 3] = v.w;
                }
#pragma unroll
                for (int m = 0; m < MATS; ++m) {
                    float acc = 0.f;
                    if constexpr (PREC == kInt8) {
#pragma unroll
                        for (int h = 0; h < 4; ++h) {
                            const uint32_t d = comp_rt(c[i][m], h);
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                acc = fmaf((float)(int)(int8_t)(d >> (8 * e)), xb[4 * h + e], acc);
                        }
                    } else {
                        // FP4: block blk is dwords 2 blk, 2 blk + 1; each byte
                        // holds two values, the even one in the low nibble
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const uint32_t d = comp_rt(c[i][m], 2 * blk + h);
                            const f32x2 f[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0),
                                                __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1),
                                                __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2),
                                                __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3)};
#pragma unroll
                            for (int sel = 0; sel < 4; ++sel) {
                                acc = fmaf(f[sel].x, xb[8 * h + 2 * sel], acc);
                                acc = fmaf(f[sel].y, xb[8 * h + 2 * sel + 1], acc);
                            }
                        }
                    }
                    sum[m] = fmaf(acc, sc[i][m][blk], sum[m]);
                }
            }
        }
        j0 += UB;
        if (j0 >= ulanes) break;
        load_units(j0);
    }
    // across the phases of the wave, then across the waves in wave order
#pragma unroll
    for (int m = 0; m < MATS; ++m)
#pragma unroll
        for (int off = R; off < 64; off <<= 1) sum[m] += __shfl_xor(sum[m], off);
    __syncthreads();  // every read of the staged row is done
    float *red = xs;  // [4][MATS][R]
    if (lane < R)
#pragma unroll
        for (int m = 0; m < MATS; ++m) red[(wave * MATS + m) * R + lane] = sum[m];
    __syncthreads();
    if (wave != 0 || lane >= R || n >= a.rows) return;
    float v[MATS];
#pragma unroll
    for (int m = 0; m < MATS; ++m) {
        float t = 0.f;
#pragma unroll
        for (int wv = 0; wv < 4; ++wv) t += red[(wv * MATS + m) * R + lane];
        v[m] = t;
    }
    const float b0 = a.b0[(size_t)g * a.rows + n];
    if constexpr (GATEUP) {
        float gv = v[0] + b0;
        float uv = v[1] + a.b1[(size_t)g * a.rows + n];
        if (a.clamp > 0.f) {
            gv = fminf(gv, a.clamp);                   // ClampedSiLU: x > L -> silu(L)
            uv = fminf(fmaxf(uv, -a.clamp), a.clamp);  // ClampedLinear
        }
        a.out[(size_t)out_row * a.ld_out + n] = silu(gv) * uv;
    } else if (a.final_out) {
        // at most two contributions per output row (see gemv_kernel)
        __hip_atomic_fetch_add(a.final_out + (size_t)t * a.rows + n, wgt * (v[0] + b0), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
        a.out[(size_t)out_row * a.ld_out + n] = v[0] + b0;
    }
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

template <int PREC, bool GATEUP, int NW, int PPW = 1>
hipError_t launch_nw(const GemvArgs &a0, int max_slices, hipStream_t s)
{
    GemvArgs a = a0;
    size_t lds = gemv_lds_bytes(a.nblocks, GATEUP, NW);
    if (a.self_dispatch) {
        // the routed expert's entry list and its length after the slice's LDS
        a.list_off = (int)((lds + 15) / 16 * 16);
        lds = (size_t)a.list_off + ((size_t)a.T * a.k + 1) * sizeof(int);
    }
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const void *fn = a.self_dispatch ? reinterpret_cast<const void *>(&gemv_kernel<PREC, GATEUP, NW, true, PPW>)
                                     : reinterpret_cast<const void *>(&gemv_kernel<PREC, GATEUP, NW, false, PPW>);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const dim3 grid((a.rows + 64 * PPW - 1) / (64 * PPW), max_slices);
    if (a.self_dispatch)
        hipLaunchKernelGGL((gemv_kernel<PREC, GATEUP, NW, true, PPW>), grid, dim3(64 * NW), lds, s, a);
    else hipLaunchKernelGGL((gemv_kernel<PREC, GATEUP, NW, false, PPW>), grid, dim3(64 * NW), lds, s, a);
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
    // a self-dispatching gate/up launch whose experts nearly all have tokens,
    // over K <= 32 chunks: four waves per workgroup (eight chunks each) fit
    // every busy workgroup at once; eight would leave some for a second round
    if (GATEUP && a.self_dispatch && a.nblocks / Chunk<PREC>::CB <= 32 && a.T * a.k >= a.E)
        return launch_nw<PREC, GATEUP, 4>(a, max_slices, s);
    // Down over many workgroups: two panels per workgroup, which stages its
    // tokens once for both (the staging was a fifth of the C5 decode down
    // kernel: 30.0 -> 27.6 us per layer).  With fewer busy workgroups than
    // two rounds' worth at the halved count the grid would no longer fill
    // the GPU (a C2-sized layer: 14.5 -> 17.9 us), so those keep one panel.
    if (!GATEUP && waves_for<PREC>(a) == 8 && a.rows >= 128) {
        const long long busy = a.self_dispatch ? (long long)a.S * a.shared_slices + std::min(a.E, a.T * a.k)
                                               : (long long)max_slices;
        if ((long long)(a.rows / 128) * busy >= 1024) return launch_nw<PREC, GATEUP, 8, 2>(a, max_slices, s);
    }
    if (waves_for<PREC>(a) == 8) return launch_nw<PREC, GATEUP, 8>(a, max_slices, s);
    return launch_nw<PREC, GATEUP, 4>(a, max_slices, s);
}

// Up to this many tokens the few-token kernel runs: it streams an expert's
// weights once per (token, slot) pair, where gemv_kernel streams them once per
// slice of up to 8 tokens, and measured faster up to 6 tokens (C2 and a C5
// block; about even at 8).
constexpr int kFewTokens = 6;
// LDS of the few-token kernel: its row buffer, four float4 per thread
constexpr size_t kFewRowBytes = 4 * 256 * sizeof(float4);

template <bool GATEUP, int PREC, int R>
hipError_t launch_few(const GemvArgs &a, hipStream_t s)
{
    const size_t lds = kFewRowBytes;  // the token row (K <= 4096 values); >= the reduction's 4 x 2 x R floats
    const dim3 grid((a.rows + R - 1) / R, a.S + a.k, a.T);
    hipLaunchKernelGGL((gemv_few_kernel<PREC, GATEUP, R>), grid, dim3(256), lds, s, a);
    return hipGetLastError();
}

// A few tokens through a layer wide enough that gemv_kernel runs eight waves
// over a panel (at least 16 chunks of K): the few-token kernel, with R = 16
// rows per workgroup when that still gives 256 workgroups, else 8.  Int8 and
// FP4 rows whose 16-byte units divide evenly among a workgroup's unit
// phases.  Returns false (nothing launched) otherwise.
template <bool GATEUP>
bool launch_few_tokens(const GemvArgs &a, int precision, hipStream_t s, hipError_t &e)
{
    if (!a.self_dispatch || a.T < 1 || a.T > kFewTokens || a.raw || (precision != kInt8 && precision != kFP4))
        return false;
    if (a.nblocks / Chunk<kInt8>::CB < 16 || a.nblocks * 16 > 4096) return false;
    const int nunits = a.row_bytes / 16;
    const int R = (long long)(a.rows / 16) * (a.S + a.k) * a.T >= 256 ? 16 : 8;
    if (a.row_bytes % 16 != 0 || nunits % (4 * (64 / R)) != 0) return false;
    if (precision == kInt8)
        e = R == 16 ? launch_few<GATEUP, kInt8, 16>(a, s) : launch_few<GATEUP, kInt8, 8>(a, s);
    else
        e = R == 16 ? launch_few<GATEUP, kFP4, 16>(a, s) : launch_few<GATEUP, kFP4, 8>(a, s);
    return true;
}

template <bool GATEUP>
hipError_t launch_any(const GemvArgs &a, int precision, int max_slices, hipStream_t s)
{
    if (max_slices <= 0) return hipSuccess;
    hipError_t e1 = hipSuccess;
    if (launch_few_tokens<GATEUP>(a, precision, s, e1)) return e1;
    // the input rows are read through a buffer resource with 32-bit offsets
    if (a.in_rows <= 0 || a.in_rows * a.ld_in * 4 > 0x7fffffffLL) return hipErrorInvalidValue;
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
