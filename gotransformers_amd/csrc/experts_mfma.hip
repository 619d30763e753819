// bf16 MFMA grouped GEMM for many tokens per expert (prefill).
//
// One workgroup computes a 128-position x 256-column tile of one group
// (expert) with v_mfma_f32_32x32x16_bf16, fp32 accumulation:
//   gate/up  A = activations gathered by token (bf16), B = 128 gate rows and
//            the same 128 up rows of the expert, dequantized (Int8 code or
//            e2m1 code times its fp32 block scale, rounded to bf16); the
//            epilogue applies the SwiGLU (feedforward/gatedfeedforward.go:
//            49-57) and writes bf16 hidden rows.
//   down     A = hidden rows (bf16, contiguous per group), B = 256 down rows;
//            the epilogue adds the bias and writes bf16 slot outputs.
// Four waves split the columns: each wave owns all 128 positions x 64
// columns (4 x 2 MFMA tiles of 32 x 32; for gate/up its two column tiles are
// gate and up of the same 32 neurons, so both values of a neuron land in
// the same lane).  The MFMAs take the weights as their first operand, so an
// accumulator tile is the output's transpose: a lane holds one position and
// four runs of four consecutive neurons, which leave as 8-byte pieces.  The activations reach LDS by LDS-DMA loads (three
// buffers, K steps of 64, two steps ahead) and are read by all four waves;
// each weight value is loaded and dequantized exactly once per workgroup, by
// the wave that uses it, straight from the panel layout into MFMA operand
// registers (three register stages, three steps ahead): lane l holds column
// l%32 and, for each pair of 16-value MFMA steps, one whole scale block
// (block 2p + l/32 of the K step; FP4: 2(l/32) + p, so that its two blocks
// of a step are one 16-byte unit), whose first and second halves feed the
// two steps.  The activations are read from LDS in the same permuted K
// order.  A tile multiplies only the 32-row blocks that hold positions, and
// the epilogue stages the tile's bf16 outputs in LDS so that they leave in
// 16-byte row pieces.
//
// Tiles: the m-tiles of all groups (the dispatch kernel wrote their count
// and a (group, first position, positions) descriptor per tile; blocks past
// the last tile exit) times the column tiles, in a 1-D grid ordered for the
// XCDs: the hardware hands block b to XCD x = b % 8, and XCD x takes the
// x-th eighth of the m-tiles, in order, each with its NT column tiles back
// to back (block b: m-tile x * ceil(tiles / 8) + j / NT, column tile j % NT,
// j = b / 8).  An m-tile's activation rows and an expert's weights (its
// m-tiles are consecutive) are then read from HBM once per XCD that needs
// them and found in that XCD's L2 by the other tiles.
#include <type_traits>

#include "mfma.h"

namespace gtmoe {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;    // positions per tile
constexpr int BN = 256;    // weight rows per tile (gate/up: 128 neurons x 2)
constexpr int BK = 64;     // K per pipeline step (4 scale blocks)

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (nearest even) and packed, lo in the low half:
// one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// x * sigmoid(x) with the hardware exp and reciprocal (about 1 ulp each)
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Codes of the two scale blocks a lane dequantizes per K step, per column
// tile, and the scales of the row's four blocks of the step (the lane uses
// blocks 2p + h: one 16-byte load serves both halves of the wave).
template <int PREC>
struct BRaw;
template <>
struct BRaw<kInt8> {
    uint4 q[2];
    float s[4];
};
template <>
struct BRaw<kFP4> {
    uint4 u;  // the lane's whole unit of the step: its blocks for pairs 0 and 1
    float s[4];
};
template <>
struct BRaw<kFloat32> {
    uint4 q[2][2];  // Float32 experts: the block's 16 values from the rows' bf16 copy
};

// descriptor word 3 for raw (untyped) buffer access on CDNA
constexpr int kRawBufferWord3 = 0x00020000;

// One group's weight matrix as buffer resources (codes and scales in the
// panel layout).  Loads past the group read zeros: column tiles past the
// matrix need no clamping.
struct GroupSrc {
    __amdgpu_buffer_rsrc_t codes;
    __amdgpu_buffer_rsrc_t scales;
};

// Codes of the lane's block of pair p of K step m (m = k0 / 64, h = lane / 32,
// the lane's half): Int8 and Float32 take block 4m + 2p + h; FP4 takes block
// 4m + 2h + p, so that a lane's two blocks of a step are one 16-byte unit,
// loaded with pair 0.  vo: the lane's byte offset of its row (plus its
// half's share) in the codes; the rest is scalar.
template <int PREC>
__device__ __forceinline__ void load_block(BRaw<PREC> &r, int i, const GroupSrc &src, uint32_t vo, int m, int p)
{
    if constexpr (PREC == kInt8) {
        // unit b; vo carries h * 1024
        r.q[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.codes, vo, (4 * m + 2 * p) * 1024, 0));
    } else if constexpr (PREC == kFP4) {
        // unit 2m + h (blocks 4m + 2h and 4m + 2h + 1); vo carries h * 1024
        if (p == 0) r.u = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.codes, vo, 2 * m * 1024, 0));
    } else {
        // Float32 experts read their rows' bf16 copy (8 values per unit):
        // units 2b, 2b + 1; vo carries 2h * 1024
#pragma unroll
        for (int u = 0; u < 2; ++u)
            r.q[i][u] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(src.codes, vo, ((4 * m + 2 * p) * 2 + u) * 1024, 0));
    }
}

// The four block scales (4m .. 4m + 3) of the lane's row for K step m; vs:
// the row's byte offset in the scales.
template <int PREC>
__device__ __forceinline__ void load_scales(BRaw<PREC> &r, const GroupSrc &src, uint32_t vs, int m)
{
    if constexpr (PREC != kFloat32) {
        const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(src.scales, vs, m * 1024, 0));
        r.s[0] = v.x;
        r.s[1] = v.y;
        r.s[2] = v.z;
        r.s[3] = v.w;
    }
}

// The lane's half of the wave (its block of a pair is 2p + half).
__device__ __forceinline__ bool lane_half() { return (threadIdx.x & 32) != 0; }

// Values 8h..8h+7 of block i as bf16 (times the block scale).
template <int PREC>
__device__ __forceinline__ bf16x8 dequant_half(const BRaw<PREC> &r, int i, int h)
{
    u32x4 o;
    if constexpr (PREC == kInt8) {
        const uint32_t d0 = h ? r.q[i].z : r.q[i].x, d1 = h ? r.q[i].w : r.q[i].y;
        const float s = lane_half() ? r.s[2 * i + 1] : r.s[2 * i];  // constant indices: no scratch
        o[0] = pack_bf16((float)(int)(int8_t)d0 * s, (float)(int)(int8_t)(d0 >> 8) * s);
        o[1] = pack_bf16((float)(int)(int8_t)(d0 >> 16) * s, (float)(int)(int8_t)(d0 >> 24) * s);
        o[2] = pack_bf16((float)(int)(int8_t)d1 * s, (float)(int)(int8_t)(d1 >> 8) * s);
        o[3] = pack_bf16((float)(int)(int8_t)(d1 >> 16) * s, (float)(int)(int8_t)(d1 >> 24) * s);
    } else if constexpr (PREC == kFP4) {
        // e2m1 pairs, even value in the low nibble (the conversion's own
        // scale operand only takes a power of two, so it stays 1.0 and the
        // block scale is applied in fp32)
        const uint32_t d = i == 0 ? (h ? r.u.y : r.u.x) : (h ? r.u.w : r.u.z);
        const float s = lane_half() ? r.s[2 + i] : r.s[i];  // block 2 half + i of the step
        const f32x2 f0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
        const f32x2 f1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
        const f32x2 f2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
        const f32x2 f3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
        o[0] = pack_bf16(f0[0] * s, f0[1] * s);
        o[1] = pack_bf16(f1[0] * s, f1[1] * s);
        o[2] = pack_bf16(f2[0] * s, f2[1] * s);
        o[3] = pack_bf16(f3[0] * s, f3[1] * s);
    } else {
        // already bf16 (the fp32 rows rounded to nearest even at upload, as
        // pack_bf16 rounds): no arithmetic
        return __builtin_bit_cast(bf16x8, r.q[i][h]);
    }
    return __builtin_bit_cast(bf16x8, o);
}

// The output tile in LDS: two halves of 64 rows, one activation buffer each,
// of 128 bf16 columns, row stride OLD (68 words: the rows m and m + 4 that
// one ds_write covers fall on disjoint banks).  An activation buffer holds
// one K step of the tile (128 rows of 128 bytes) or one output half.
constexpr int OLD = 136;
constexpr int kBufBytes = 64 * OLD * 2 > BM * BK * 2 ? 64 * OLD * 2 : BM * BK * 2;

// Rows [0, M) of the LDS output tile (row m at os[m / 64] + (m % 64) OLD)
// to out rows p0 + m; tile column c goes to output column col_of(c) (groups
// of 8 tile columns map to 8 consecutive output columns).  Thread t stores
// the 16-byte pieces t + 256 i (row piece / 16, columns 8 (piece % 16) ..).
// Widths or strides that are not multiples of 8 columns take 2-byte stores.
template <typename ColOf>
__device__ __forceinline__ void store_tile(const MfmaArgs &a, const uint16_t *os0, const uint16_t *os1, int p0, int M,
                                           ColOf col_of)
{
    uint16_t *out = reinterpret_cast<uint16_t *>(a.out);
    const int tid = threadIdx.x;
    if (a.n % 8 == 0 && a.ldo % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
#pragma unroll
        for (int i = 0; i < BM * 16 / 256; ++i) {
            const int piece = tid + 256 * i;
            const int m = piece >> 4, c = (piece & 15) * 8;
            const int n = col_of(c);
            const uint16_t *os = i < BM * 8 / 256 ? os0 : os1;  // rows 16 i + tid / 16
            if (m < M && n < a.n)
                *reinterpret_cast<uint4 *>(out + (size_t)(p0 + m) * a.ldo + n) =
                    *reinterpret_cast<const uint4 *>(os + (m & 63) * OLD + c);
        }
    } else {
        for (int e = tid; e < BM * 128; e += 256) {
            const int m = e >> 7, c = e & 127;
            const int n = col_of(c);
            if (m < M && n < a.n) out[(size_t)(p0 + m) * a.ldo + n] = (m < 64 ? os0 : os1)[(m & 63) * OLD + c];
        }
    }
}

template <int S>
__device__ __forceinline__ char *pick(char *b0, char *b1, char *b2)
{
    return S == 0 ? b0 : S == 1 ? b1 : b2;
}

}  // namespace

// One tile whose positions lie in its first MI 32-row blocks (M <= 32 MI):
// the blocks past them are neither loaded nor multiplied.  b0, b1, b2: the
// three activation buffers (kBufBytes of LDS each, separate arrays, so that
// the compiler tells their accesses apart).
template <int PREC, bool GATEUP, int MI>
__device__ __forceinline__ void gemm_tile(const MfmaArgs &a, char *b0, char *b1, char *b2, int g, int p0, int M,
                                          int ntile)
{
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, h = lane >> 5;

    // activations go from memory straight into LDS (16-byte LDS-DMA loads,
    // no registers): per K step, row block i < MI of the tile is four wave
    // loads, wave w taking rows 32 i + 8 w .. + 7, lane l writing 16 bytes
    // at row 32 i + 8 w + l / 8, slot l % 8 of the step's buffer.  A row is
    // 128 bytes (64 bf16 of K); slot s of row R holds K values
    // 8 (s ^ (R / 2) % 8) .. + 7.  The LDS has 64 four-byte banks and serves
    // a 16-byte read 16 lanes at a time: rows R and R + 1 fall on opposite
    // halves of the banks and the swizzle spreads the 8 rows of each parity
    // among a 16-row run over the 8 slots, so an operand read (16 rows, one
    // K chunk) touches every bank once.  Rows past M read past the buffer
    // and get zeros.
    const __amdgpu_buffer_rsrc_t asrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(a.a), 0, (int)(a.a_rows * a.lda * 2), kRawBufferWord3);
    // (R / 2) % 8 == (4 (w % 2) + l / 16) for this lane's rows R
    const int arow = lane >> 3, achunk = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    // gate/up gathers rows by token: the MI token numbers are loaded together,
    // the position clamped into the tile (a load under the r < M condition
    // made the compiler wait for each before issuing the next); the row
    // offsets are formed in the prologue, after the first weight loads
    uint32_t aoff[MI];
    int arow_src[MI];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int r = 32 * i + 8 * wave + arow;
        arow_src[i] = GATEUP ? a.tok[p0 + min(r, M - 1)] : p0 + r;
    }
    auto form_aoff = [&]() {
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int r = 32 * i + 8 * wave + arow;
            aoff[i] = r < M ? ((uint32_t)arow_src[i] * (uint32_t)a.lda + achunk * 8) * 2u : 0x80000000u;
        }
    };

    // weights: the wave's two column tiles (gate/up: the same 32 neurons of
    // gate and up; down: 64 consecutive rows), a group's matrices as buffer
    // resources; columns past n read zeros and are not written
    GroupSrc bsrc[2];
    uint32_t bvo[2], bvs[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = GATEUP ? ntile * (BN / 2) + wave * 32 + col : ntile * BN + wave * 64 + j * 32 + col;
        const void *w = GATEUP ? (j ? a.w1 : a.w0) : a.w0;
        const float *sc = GATEUP ? (j ? a.s1 : a.s0) : a.s0;
        bsrc[j].codes = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char *>(reinterpret_cast<const char *>(w)) + (size_t)g * a.w_group_stride, 0,
            (int)a.w_group_stride, kRawBufferWord3);
        const uint32_t rowoff = (uint32_t)(n / 64) * 64u * (uint32_t)a.row_bytes + (uint32_t)(n % 64) * 16u;
        if constexpr (PREC == kInt8) bvo[j] = rowoff + h * 1024u;
        else if constexpr (PREC == kFP4) bvo[j] = rowoff + h * 1024u;
        else bvo[j] = rowoff + h * 2048u;
        if constexpr (PREC != kFloat32) {
            bsrc[j].scales = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(sc) + (size_t)g * a.s_group_stride, 0,
                                                             (int)(a.s_group_stride * 4), kRawBufferWord3);
            bvs[j] = ((uint32_t)(n / 64) * 64u * (uint32_t)a.nblocks + (uint32_t)(n % 64) * 4u) * 4u;
        } else {
            bsrc[j].scales = bsrc[j].codes;
            bvs[j] = 0;
        }
    }

    // Accumulator tile (i, j) holds output[position 32 i + col][neuron
    // nbase[j] + nn(r)] in register r, nn(r) = 8 (r / 4) + 4 h + r % 4 (the
    // weights are the MFMA's first operand).  The accumulators start at the
    // neurons' biases: the epilogue has nothing to load.  The biases are
    // requested here and copied in after the prologue, whose counted waits
    // cover them (they are the oldest loads).
    int nbase[2];
    floatx16 binit[2], acc[MI][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        nbase[j] = GATEUP ? ntile * (BN / 2) + wave * 32 : ntile * BN + wave * 64 + j * 32;
        const float *bias = (GATEUP && j ? a.b1 : a.b0) + (size_t)g * a.n;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = nbase[j] + 8 * q + 4 * h;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (a.n % 4 == 0) {
                if (n < a.n) v = *reinterpret_cast<const float4 *>(bias + n);
            } else {
                if (n < a.n) v.x = bias[n];
                if (n + 1 < a.n) v.y = bias[n + 1];
                if (n + 2 < a.n) v.z = bias[n + 2];
                if (n + 3 < a.n) v.w = bias[n + 3];
            }
            binit[j][4 * q] = v.x;
            binit[j][4 * q + 1] = v.y;
            binit[j][4 * q + 2] = v.z;
            binit[j][4 * q + 3] = v.w;
        }
    }

    // Software pipeline: during step k the activations of step k + 2 are
    // on their way into LDS buffer (k + 2) % 3 (buffer (k + 2) % 3 was read
    // in step k - 1, before the barrier that ended it) and the weights of
    // step k + NS into register stage k % NS (its pair 1 is dequantized at
    // the start of step k): NS = 3 stages, or 2 for Float32 experts, whose
    // bf16 rows make stages a third larger than Int8's codes and scales.
    // The loop is unrolled by three (six for two stages) so the buffer and
    // stage indices are constants; every load is
    // issued unconditionally (steps past the end re-load the last step:
    // cache hits, never used), so that each step issues the same VMEM
    // instructions in the same order: MI activation loads, then NB weight
    // loads.  Step k ends once the activations of step k + 1 have landed:
    // each wave waits until at most the VMEM instructions issued after its
    // own loads of them are pending (2 NB + MI: one step's weights, then the
    // activations and the weights of step k) and the barrier makes every
    // wave's rows visible.  Scheduling barriers keep that order.
    const int nsteps = a.kp / BK;
    constexpr int NS = PREC == kFloat32 ? 2 : 3;
    constexpr int UNROLL = NS == 3 ? 3 : 6;
    BRaw<PREC> bq[NS][2];  // [stage][column tile]
    constexpr int NB = PREC == kInt8 ? 6 : PREC == kFP4 ? 4 : 8;
    constexpr int VM = 2 * NB + MI;
    static_assert(VM < 64, "vmcnt holds six bits");
    // s_waitcnt vmcnt(n) lgkmcnt(0), expcnt not waited for
    constexpr auto vm_wait = [](int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); };
    constexpr int kStepWait = vm_wait(VM);
    // after the prologue's activations of step 0: the weights of step 1 and
    // the activations of step 1, and with three stages the weights of step 2
    constexpr int kPrologueWait = vm_wait(NS == 3 ? VM : NB + MI);
    auto dma_a = [&](char *buf, int step) {
        const int k0 = min(step, nsteps - 1) * BK;
#pragma unroll
        for (int i = 0; i < MI; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                asrc, (__attribute__((address_space(3))) void *)(buf + (32 * i + 8 * wave) * 128), 16, aoff[i],
                k0 * 2, 0, 0);
    };
    auto load_b = [&](BRaw<PREC> (&q)[2], int step) {
        const int m = min(step, nsteps - 1);
        // pair p of the step: this lane's block is 2p + h (FP4: 2h + p)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int p = 0; p < 2; ++p) load_block<PREC>(q[j], p, bsrc[j], bvo[j], m, p);
            load_scales<PREC>(q[j], bsrc[j], bvs[j], m);
        }
    };
    auto end_step = [&](auto wait_tag) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(decltype(wait_tag)::value);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    // The K step is done in two halves (pair p = 0, 1: 16 MFMAs each, K
    // values of scale blocks 2p and 2p + 1).  While the MFMAs of one half run,
    // the same wave dequantizes the B operands of the next half, so the VALU
    // work hides under the matrix cores: the scheduling groups below ask for
    // one MFMA, then a share of the VALU instructions (four with all four
    // row blocks), in turn.
    auto dequant_pair = [&](const BRaw<PREC> (&q)[2], int p, bf16x8 (&out)[2][2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) out[j][s2] = dequant_half<PREC>(q[j], p, s2);
    };
    auto mfma_pair = [&](const char *buf, int p, const bf16x8 (&bfp)[2][2]) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            // k-values of this MFMA step: lanes of half h carry values
            // 8s2..8s2+7 of block 2p + h (FP4: 2h + p) of the K step, which
            // is K chunk 2 block + s2, in slot chunk ^ (row / 2) % 8
            const int chunk = 2 * (PREC == kFP4 ? 2 * h + p : 2 * p + h) + s2;
            const int so = 16 * (chunk ^ ((col >> 1) & 7));
            bf16x8 af[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i) af[i] = *reinterpret_cast<const bf16x8 *>(buf + (32 * i + col) * 128 + so);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfp[j][s2], af[i], acc[i][j], 0, 0, 0);
        }
    };
    auto interleave = [&]() {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            __builtin_amdgcn_sched_group_barrier(0x100, MI, 0);  // the LDS reads of the A operands
#pragma unroll
            for (int m = 0; m < 2 * MI; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, (16 + MI - 1) / MI, 0);  // VALU
            }
        }
    };
    bf16x8 bfa[2][2], bfb[2][2];  // B operands of the current and the next half step
    // step k of the pipeline (U = k % UNROLL); bfa holds pair 0 of step k.
    // The last steps, after the loop, wait for all their loads instead: the
    // compiler drops their weight loads (nothing reads them), which leaves
    // fewer instructions behind the activations than the loop's count.
    auto step = [&](auto u_tag, int k, auto wait_tag) {
        constexpr int U = decltype(u_tag)::value;
        constexpr int A0 = U % 3, A2 = (U + 2) % 3, B0 = U % NS, B1 = (U + 1) % NS;
        const char *rd = pick<A0>(b0, b1, b2);
        dma_a(pick<A2>(b0, b1, b2), k + 2);
        __builtin_amdgcn_sched_barrier(0);
        mfma_pair(rd, 0, bfa);
        dequant_pair(bq[B0], 1, bfb);
        interleave();
        __builtin_amdgcn_sched_barrier(0);
        load_b(bq[B0], k + NS);
        mfma_pair(rd, 1, bfb);
        dequant_pair(bq[B1], 0, bfa);  // pair 0 of step k + 1 (past the end: unused)
        interleave();
        end_step(wait_tag);
    };
    const std::integral_constant<int, kStepWait> loop_wait;
    const std::integral_constant<int, (7 << 4)> full_wait;  // vmcnt(0) lgkmcnt(0)

    // prologue: after the activations of step 1 come as many VMEM
    // instructions as after those of step k + 1 in the loop (with three
    // stages the weights of step 2, with two those of step 1)
    load_b(bq[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    form_aoff();
    dma_a(b0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NS == 3) {
        load_b(bq[1], 1);
        __builtin_amdgcn_sched_barrier(0);
        dma_a(b1, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_b(bq[NS - 1], 2);
    } else {
        dma_a(b1, 1);
        __builtin_amdgcn_sched_barrier(0);
        load_b(bq[1], 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    dequant_pair(bq[0], 0, bfa);
    end_step(std::integral_constant<int, kPrologueWait>{});
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = binit[j];
    int k = 0;
    for (; k + UNROLL <= nsteps; k += UNROLL) {
        step(std::integral_constant<int, 0>{}, k, loop_wait);
        step(std::integral_constant<int, 1>{}, k + 1, loop_wait);
        step(std::integral_constant<int, 2>{}, k + 2, loop_wait);
        if constexpr (UNROLL == 6) {
            step(std::integral_constant<int, 3>{}, k + 3, loop_wait);
            step(std::integral_constant<int, 4>{}, k + 4, loop_wait);
            step(std::integral_constant<int, 5>{}, k + 5, loop_wait);
        }
    }
    if (k < nsteps) step(std::integral_constant<int, 0>{}, k, full_wait);
    if (k + 1 < nsteps) step(std::integral_constant<int, 1>{}, k + 1, full_wait);
    if constexpr (UNROLL == 6) {
        if (k + 2 < nsteps) step(std::integral_constant<int, 2>{}, k + 2, full_wait);
        if (k + 3 < nsteps) step(std::integral_constant<int, 3>{}, k + 3, full_wait);
        if (k + 4 < nsteps) step(std::integral_constant<int, 4>{}, k + 4, full_wait);
    }
    // the loads past the last step land before any wave reuses the buffers
    end_step(full_wait);

    // epilogue: the tile's bf16 outputs are put in LDS (free now: every wave
    // is past its last read of the activations and every load has landed),
    // four neurons of a position per 8-byte write, and leave in 16-byte
    // stores of whole row pieces.  Lane holds position 32 i + col of row
    // block i and neurons nn(r) of each column tile; rows past the tile's M
    // are computed from zero activations and not stored.  Row block i goes
    // to half i / 2, LDS column wave * 32 + nn.
    uint16_t *os0 = reinterpret_cast<uint16_t *>(b0), *os1 = reinterpret_cast<uint16_t *>(b1);
    auto put4 = [&](int i, int q, uint32_t lo, uint32_t hi) {  // neurons 8 q + 4 h .. + 3
        uint16_t *os = i < 2 ? os0 : os1;
        const int m = (i & 1) * 32 + col;
        *reinterpret_cast<uint2 *>(os + m * OLD + wave * 32 + 8 * q + 4 * h) = make_uint2(lo, hi);
    };
    if constexpr (GATEUP) {
        auto emit_all = [&](auto clamp_tag) {
            constexpr bool CL = decltype(clamp_tag)::value;
            auto swiglu = [&](float gv, float uv) {
                if constexpr (CL) {
                    gv = fminf(gv, a.clamp);                   // ClampedSiLU: x > L -> silu(L)
                    uv = fminf(fmaxf(uv, -a.clamp), a.clamp);  // ClampedLinear
                }
                return silu(gv) * uv;
            };
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 4 * q;
                    put4(i, q,
                         pack_bf16(swiglu(acc[i][0][r], acc[i][1][r]), swiglu(acc[i][0][r + 1], acc[i][1][r + 1])),
                         pack_bf16(swiglu(acc[i][0][r + 2], acc[i][1][r + 2]),
                                   swiglu(acc[i][0][r + 3], acc[i][1][r + 3])));
                }
        };
        if (a.clamp > 0.f) emit_all(std::true_type{});
        else emit_all(std::false_type{});
        __syncthreads();
        // tile column c is hidden column ntile * 128 + c
        store_tile(a, os0, os1, p0, M, [&](int c) { return ntile * (BN / 2) + c; });
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // one column tile of every wave per pass: tile column c is output
            // column ntile * 256 + (c / 32) * 64 + j * 32 + c % 32
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 4 * q;
                    put4(i, q, pack_bf16(acc[i][j][r], acc[i][j][r + 1]), pack_bf16(acc[i][j][r + 2], acc[i][j][r + 3]));
                }
            __syncthreads();
            store_tile(a, os0, os1, p0, M, [&](int c) { return ntile * BN + (c >> 5) * 64 + j * 32 + (c & 31); });
            if (j == 0) __syncthreads();  // the next pass rewrites the LDS tile
        }
    }
}

template <int PREC, bool GATEUP>
__global__ __launch_bounds__(256, 2) void mfma_gemm_kernel(MfmaArgs a)
{
    __shared__ __attribute__((aligned(16))) char buf0[kBufBytes];
    __shared__ __attribute__((aligned(16))) char buf1[kBufBytes];
    __shared__ __attribute__((aligned(16))) char buf2[kBufBytes];

    const int j8 = blockIdx.x >> 3;
    const int ntiles = *a.count;
    const int per_xcd = (ntiles + 7) >> 3;
    const int tile = (blockIdx.x & 7) * per_xcd + j8 / a.ntiles_n;
    const int ntile = j8 % a.ntiles_n;
    if (j8 / a.ntiles_n >= per_xcd || tile >= ntiles) return;
    const int4 dsc = a.desc[tile];
    const int g = dsc.x;
    const int p0 = dsc.y;  // first position of the tile
    const int M = dsc.z;   // positions in the tile
    // an expert's last tile is usually partly filled: multiply only the
    // 32-row blocks that hold positions (fewer than three run as two: the
    // dequantization, the same for any M, then bounds the time anyway)
    if (M > 96)
        gemm_tile<PREC, GATEUP, 4>(a, buf0, buf1, buf2, g, p0, M, ntile);
    else if (M > 64)
        gemm_tile<PREC, GATEUP, 3>(a, buf0, buf1, buf2, g, p0, M, ntile);
    else
        gemm_tile<PREC, GATEUP, 2>(a, buf0, buf1, buf2, g, p0, M, ntile);
}

int mfma_tile_m() { return BM; }

// One 16-byte unit of the bf16 copy per thread: fp32 units 2u and 2u + 1 of
// a row (8 values), rounded as pack_bf16 rounds.  Threads run down the rows
// of a unit, so reads and writes are contiguous within each panel.
__global__ __launch_bounds__(256) void bf16_rows_kernel(const char *__restrict__ src, char *__restrict__ dst,
                                                        int rows_p, int kp)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const int units = kp / 8;
    if (idx >= (long long)rows_p * units) return;
    const int r = (int)(idx % rows_p), u = (int)(idx / rows_p);
    const uint4 a = *reinterpret_cast<const uint4 *>(src + panel_unit_offset(r, 2 * u, kp * 4));
    const uint4 b = *reinterpret_cast<const uint4 *>(src + panel_unit_offset(r, 2 * u + 1, kp * 4));
    uint4 o;
    o.x = pack_bf16(__uint_as_float(a.x), __uint_as_float(a.y));
    o.y = pack_bf16(__uint_as_float(a.z), __uint_as_float(a.w));
    o.z = pack_bf16(__uint_as_float(b.x), __uint_as_float(b.y));
    o.w = pack_bf16(__uint_as_float(b.z), __uint_as_float(b.w));
    *reinterpret_cast<uint4 *>(dst + panel_unit_offset(r, u, kp * 2)) = o;
}

hipError_t launch_bf16_rows(const void *rows_f32, void *rows_bf16, int rows_p, int kp, hipStream_t s)
{
    if (rows_p <= 0 || kp <= 0 || kp % 8 != 0) return hipErrorInvalidValue;
    const long long n = (long long)rows_p * (kp / 8);
    hipLaunchKernelGGL(bf16_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       static_cast<const char *>(rows_f32), static_cast<char *>(rows_bf16), rows_p, kp);
    return hipGetLastError();
}

namespace {

template <bool GATEUP>
hipError_t launch_mfma(const MfmaArgs &a, int precision, int max_tiles, hipStream_t s)
{
    if (max_tiles <= 0) return hipSuccess;
    if (a.kp % BK != 0) return hipErrorInvalidValue;
    // activations and each group's weights are read through buffer resources
    // with 32-bit offsets
    if (a.a_rows <= 0 || a.a_rows * a.lda * 2 > 0x7fffffffLL || a.w_group_stride > 0x7fffffffLL ||
        a.s_group_stride * 4 > 0x7fffffffLL)
        return hipErrorInvalidValue;
    constexpr int COLS = GATEUP ? BN / 2 : BN;  // output columns per tile
    MfmaArgs b = a;
    b.ntiles_n = (a.n + COLS - 1) / COLS;
    const dim3 grid((unsigned)((max_tiles + 7) / 8 * 8 * b.ntiles_n));
    switch (precision) {
    case kInt8: hipLaunchKernelGGL((mfma_gemm_kernel<kInt8, GATEUP>), grid, dim3(256), 0, s, b); break;
    case kFP4: hipLaunchKernelGGL((mfma_gemm_kernel<kFP4, GATEUP>), grid, dim3(256), 0, s, b); break;
    case kFloat32: hipLaunchKernelGGL((mfma_gemm_kernel<kFloat32, GATEUP>), grid, dim3(256), 0, s, b); break;
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
