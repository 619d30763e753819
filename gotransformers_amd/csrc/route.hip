// Routing kernels: fp32 router logits, float64 affinity / top-k / gates with
// the reference's tie-break, hash routing, and the stable dispatch.
//
// Built with -ffp-contract=off: the affinity and gate arithmetic must round
// exactly like the float64 CPU restatement (mixtureofexperts.go:153-173), so
// nothing here may be fused unless written as an explicit fmaf.
#include "kernels.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace gtmoe {

// ---------------------------------------------------------------------------
// float64 exp / log1p, the fdlibm methods that Go's portable math.Exp and
// math.Log1p follow (activationfunction.Softplus calls them,
// moreactivationfunctions.go:8-16).  Same operation sequence as the CPU
// restatement, so results agree to the bit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double bits_f64(unsigned long long u) { return __longlong_as_double((long long)u); }

__device__ double go_exp(double x)
{
    const double ln2_hi = bits_f64(0x3fe62e42fee00000ULL);
    const double ln2_lo = bits_f64(0x3dea39ef35793c76ULL);
    const double log2e = bits_f64(0x3ff71547652b82feULL);
    const double overflow = 7.09782712893383973096e+02;
    const double underflow = -7.45133219101941108420e+02;
    const double near_zero = 1.0 / (double)(1 << 28);
    const double p1 = bits_f64(0x3fc5555555555555ULL);
    const double p2 = bits_f64(0xbf66c16c16bebd93ULL);
    const double p3 = bits_f64(0x3f11566aaf25de2cULL);
    const double p4 = bits_f64(0xbebbbd41c5d26bf1ULL);
    const double p5 = bits_f64(0x3e66376972bea4d0ULL);

    if (isnan(x) || (isinf(x) && x > 0)) return x;
    if (isinf(x)) return 0;
    if (x > overflow) return INFINITY;
    if (x < underflow) return 0;
    if (-near_zero < x && x < near_zero) return 1 + x;

    int k = 0;
    if (x < 0) k = (int)(log2e * x - 0.5);
    else if (x > 0) k = (int)(log2e * x + 0.5);
    double hi = x - (double)k * ln2_hi;
    double lo = (double)k * ln2_lo;
    double r = hi - lo;
    double t = r * r;
    double c = r - t * (p1 + t * (p2 + t * (p3 + t * (p4 + t * p5))));
    double y = 1 - ((lo - (r * c) / (2 - c)) - hi);
    return ldexp(y, k);
}

__device__ double go_log1p(double x)
{
    const double sqrt2m1 = bits_f64(0x3fda827999fcef34ULL);
    const double sqrt2halfm1 = bits_f64(0xbfd2bec333018866ULL);
    const double small = 1.0 / (double)(1 << 29);
    const double tiny = 1.0 / (double)(1ULL << 54);
    const double two53 = (double)(1ULL << 53);
    const double ln2_hi = bits_f64(0x3fe62e42fee00000ULL);
    const double ln2_lo = bits_f64(0x3dea39ef35793c76ULL);
    const double lp1 = bits_f64(0x3fe5555555555593ULL);
    const double lp2 = bits_f64(0x3fd999999997fa04ULL);
    const double lp3 = bits_f64(0x3fd2492494229359ULL);
    const double lp4 = bits_f64(0x3fcc71c51d8e78afULL);
    const double lp5 = bits_f64(0x3fc7466496cb03deULL);
    const double lp6 = bits_f64(0x3fc39a09d078c69fULL);
    const double lp7 = bits_f64(0x3fc2f112df3e5244ULL);

    if (x < -1 || isnan(x)) return NAN;
    if (x == -1) return -INFINITY;
    if (isinf(x)) return INFINITY;

    double absx = fabs(x);
    double f = 0;
    unsigned long long iu = 0;
    int k = 1;
    if (absx < sqrt2m1) {
        if (absx < small) {
            if (absx < tiny) return x;
            return x - x * x * 0.5;
        }
        if (x > sqrt2halfm1) {
            k = 0;
            f = x;
            iu = 1;
        }
    }
    double c = 0;
    if (k != 0) {
        double u;
        if (absx < two53) {
            u = 1.0 + x;
            iu = (unsigned long long)__double_as_longlong(u);
            k = (int)((iu >> 52) - 1023);
            if (k > 0) c = 1.0 - (u - x);
            else c = x - (u - 1.0);
            c /= u;
        } else {
            u = x;
            iu = (unsigned long long)__double_as_longlong(u);
            k = (int)((iu >> 52) - 1023);
            c = 0;
        }
        iu &= 0x000fffffffffffffULL;
        if (iu < 0x0006a09e667f3bcdULL) {
            u = bits_f64(iu | 0x3ff0000000000000ULL);
        } else {
            k++;
            u = bits_f64(iu | 0x3fe0000000000000ULL);
            iu = (0x0010000000000000ULL - iu) >> 2;
        }
        f = u - 1.0;
    }
    double hfsq = 0.5 * f * f;
    double s, r, z;
    if (iu == 0) {
        if (f == 0) {
            if (k == 0) return 0;
            c += (double)k * ln2_lo;
            return (double)k * ln2_hi + c;
        }
        r = hfsq * (1.0 - 0.66666666666666666 * f);
        if (k == 0) return f - r;
        return (double)k * ln2_hi - ((r - ((double)k * ln2_lo + c)) - f);
    }
    s = f / (2.0 + f);
    z = s * s;
    r = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + r));
    return (double)k * ln2_hi - ((hfsq - (s * (hfsq + r) + ((double)k * ln2_lo + c))) - f);
}

// affinity = sqrt(softplus(logit)) (mixtureofexperts.go:80-82)
__device__ double affinity(double logit)
{
    double sp;
    if (logit > 20) sp = logit;
    else if (logit < -20) sp = go_exp(logit);
    else sp = go_log1p(go_exp(logit));
    return sqrt(sp);
}

// ---------------------------------------------------------------------------
// Router logits: logits[t][e] = double(sum_i x[t][i] * w[e][i]) + bias[e].
// ---------------------------------------------------------------------------

// zero[0 .. nzero) cleared by the whole grid (any grid shape): the chunked
// dispatch's per-chunk expert counts, which the top-k after the router adds
// up (the clearing must be a kernel, not a memset, where the launch may be
// captured into a graph).
__device__ __forceinline__ void clear_counts(int32_t *__restrict__ zero, int nzero)
{
    if (zero == nullptr) return;
    const int wg = blockIdx.y * gridDim.x + blockIdx.x;
    const int stride = gridDim.x * gridDim.y * blockDim.x;
    for (int i = wg * blockDim.x + threadIdx.x; i < nzero; i += stride) zero[i] = 0;
}

// Few tokens: one wave per (token, expert) dot product; lanes read float4
// runs of the zero-padded rows (x row stride ldx, router row stride ldw, both
// multiples of 64 floats) and reduce across the wave.
__global__ __launch_bounds__(256) void router_small_kernel(const float *__restrict__ x, int ldx, int T, int kp,
                                                           const float *__restrict__ w, int ldw,
                                                           const double *__restrict__ bias, int E,
                                                           double *__restrict__ logits,
                                                           const float *__restrict__ row_scale,
                                                           int32_t *__restrict__ zero, int nzero)
{
    clear_counts(zero, nzero);
    const int lane = threadIdx.x & 63;
    const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (pair >= T * E) return;  // wave-uniform
    const int t = pair / E, e = pair - t * E;
    const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)t * ldx);
    const float4 *wr = reinterpret_cast<const float4 *>(w + (size_t)e * ldw);
    float acc = 0.f;
    for (int i = lane; i < kp / 4; i += 64) {
        const float4 a = xr[i], b = wr[i];
        acc = fmaf(a.x, b.x, acc);
        acc = fmaf(a.y, b.y, acc);
        acc = fmaf(a.z, b.z, acc);
        acc = fmaf(a.w, b.w, acc);
    }
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (row_scale) acc = row_scale[t] * acc;
    if (lane == 0) logits[(size_t)t * E + e] = (double)acc + bias[e];
}

// Many tokens: fp32 matrix cores.  A workgroup computes 32 tokens x 32 NE
// experts with v_mfma_f32_32x32x2_f32 (fp32 products, fp32 accumulation),
// so a token row is read once for NE expert tiles; its NW waves take an
// NW-th of K each and add their partial tiles through LDS in wave order.
// Lane l supplies row l%32 (token resp. expert of each tile) at k-offset
// 8*(l/32) + s of every 16-value step for the 8 chained instructions s, so a
// lane's operands are two float4 loads per row and step; the loads of the
// next kRouterAhead steps are in flight while a step multiplies.  Rows past
// T or E read the last valid row and are not written.
typedef float floatx16 __attribute__((ext_vector_type(16)));
constexpr long long kRouterWaves = 2048;  // two waves per SIMD of 256 CUs
constexpr int kRouterAhead = 3;            // steps whose loads are in flight

template <int NE, int NW>
__global__ __launch_bounds__(64 * NW) void router_mfma_kernel(const float *__restrict__ x, int ldx, int T, int kp,
                                                              const float *__restrict__ w, int ldw,
                                                              const double *__restrict__ bias, int E,
                                                              double *__restrict__ logits,
                                                              const float *__restrict__ row_scale,
                                                              int32_t *__restrict__ zero, int nzero)
{
    __shared__ float red[NW][16 * NE][64];
    clear_counts(zero, nzero);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 32, e0 = blockIdx.y * 32 * NE;
    const int r = lane & 31, h = lane >> 5;
    const float *xr = x + (size_t)min(t0 + r, T - 1) * ldx + 8 * h;
    const float *wr[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) wr[j] = w + (size_t)min(e0 + 32 * j + r, E - 1) * ldw + 8 * h;
    const int n16 = kp / 16;
    const int k0 = wave * n16 / NW, k1 = (wave + 1) * n16 / NW;
    floatx16 acc[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.f;
    // a ring of kRouterAhead steps' operands: step kb's loads are issued
    // kRouterAhead steps before it multiplies (past the last step the ring
    // re-loads that step, unused)
    struct Ops {
        float4 xa, xb, wa[NE], wb[NE];
    };
    auto load = [&](Ops &o, int kb) {
        o.xa = *reinterpret_cast<const float4 *>(xr + kb * 16);
        o.xb = *reinterpret_cast<const float4 *>(xr + kb * 16 + 4);
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            o.wa[j] = *reinterpret_cast<const float4 *>(wr[j] + kb * 16);
            o.wb[j] = *reinterpret_cast<const float4 *>(wr[j] + kb * 16 + 4);
        }
    };
    Ops ring[kRouterAhead];
    if (k0 < k1) {
#pragma unroll
        for (int i = 0; i < kRouterAhead; ++i) load(ring[i], min(k0 + i, k1 - 1));
    }
    for (int kb = k0; kb < k1; kb += kRouterAhead) {
#pragma unroll
        for (int i = 0; i < kRouterAhead; ++i) {
            if (kb + i >= k1) break;  // wave-uniform
            Ops &o = ring[i];
            const float xs[8] = {o.xa.x, o.xa.y, o.xa.z, o.xa.w, o.xb.x, o.xb.y, o.xb.z, o.xb.w};
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int j = 0; j < NE; ++j) {
                    const float ws = s < 4 ? (&o.wa[j].x)[s] : (&o.wb[j].x)[s - 4];
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[s], ws, acc[j], 0, 0, 0);
                }
            load(o, min(kb + i + kRouterAhead, k1 - 1));
        }
    }
#pragma unroll
    for (int j = 0; j < NE; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[wave][16 * j + i][lane] = acc[j][i];
    __syncthreads();
    // accumulator register i of tile j in lane l is token row
    // 8*(i/4) + 4*(l/32) + i%4, expert 32 j + l%32; wave q finishes the
    // registers 16 j + i = q, q + NW, ...
    for (int ji = wave; ji < 16 * NE; ji += NW) {
        const int j = ji >> 4, i = ji & 15;
        const int t = t0 + 8 * (i >> 2) + 4 * h + (i & 3), e = e0 + 32 * j + r;
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < NW; ++q) v += red[q][ji][lane];
        if (t < T && e < E) {
            if (row_scale) v = row_scale[t] * v;
            logits[(size_t)t * E + e] = (double)v + bias[e];
        }
    }
}

// Many tokens, staged through LDS: a workgroup computes 32 tokens x 32 NE
// experts with v_mfma_f32_32x32x2_f32 as router_mfma_kernel does, but the
// token and router rows reach LDS in 64-value chunks by 16-byte LDS-DMA
// loads (four rows of 256 bytes per wave load, so each load reads whole
// cache lines), four chunk buffers, three chunks in flight ahead of the one
// multiplied.  The 16-byte slots of row R are XOR-swizzled by R % 16, so
// that the operand reads (32 rows, one slot each) touch every bank once per
// 16 lanes.  Wave w multiplies slots 2w and 2w + 1 of every chunk (lane l:
// row l % 32, slot 2w + l / 32, the slot's four values over four chained
// MFMAs); the waves' partial tiles are added in wave order at the end.  Rows
// past T or E read the last valid row and are not written.
constexpr long long kRouterStagedWgs = 256;  // one workgroup per CU at least
constexpr int kRawBufferWord3 = 0x00020000;  // descriptor word 3 for raw (untyped) buffer access on CDNA

template <int NE>
constexpr int router_lds_buf()
{
    return 32 * 256 + 32 * NE * 256;  // a chunk's token rows and router rows
}

// Four floats as bf16 (nearest even), packed in 8 bytes (the rounding of
// the input conversion's bf16 rows).
__device__ __forceinline__ uint2 router_bf16x4(float4 v)
{
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v.x, v.y}, bf16x2)),
                      __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){v.z, v.w}, bf16x2)));
}

// (the body is a device function: its LDS-DMA address casts have no host
// form, and the kernel's host-side stub is only emitted for a body without)
// CONV: the workgroup also writes its 32 token rows as bf16 (xb, rows of
// ldb values): each lane reads back the 16 bytes its own DMA put in LDS (row
// 4 w + l / 16, the row's slot (l % 16) ^ (row % 16)), so the 16 lanes of a
// row store one contiguous 128-byte run of it, after the chunk's products.
template <int NE, bool CONV>
__device__ __forceinline__ void router_lds_body(const float *__restrict__ x, int ldx, int T, int kp,
                                                const float *__restrict__ w, int ldw, const double *__restrict__ bias,
                                                int E, double *__restrict__ logits, const float *__restrict__ row_scale,
                                                uint16_t *__restrict__ xb, int ldb, char *s0, char *s1, char *s2,
                                                char *s3)
{
    constexpr int NW = 8;
    constexpr int XB = 32 * 256;            // a chunk's token rows
    constexpr int BUF = router_lds_buf<NE>();
    constexpr int PER_WAVE = 16 * NE * 64;  // floats of a wave's partial tiles
    static_assert(2 * PER_WAVE * 4 <= BUF, "two waves' partial tiles per chunk buffer");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t0 = blockIdx.x * 32, e0 = blockIdx.y * 32 * NE;
    const int nchunks = kp / 64;

    // DMA: wave w loads rows 4w .. 4w + 3 of the token tile and of each
    // expert tile; lane l takes row 4w + l / 16 and writes LDS slot l % 16
    // of it, which holds the row's 16-byte slot (l % 16) ^ (row % 16)
    const __amdgpu_buffer_rsrc_t xsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x), 0, (int)((long long)T * ldx * 4), kRawBufferWord3);
    const __amdgpu_buffer_rsrc_t wsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(w), 0, (int)((long long)E * ldw * 4), kRawBufferWord3);
    const int rl = 4 * wave + (lane >> 4);
    const int sw = ((lane & 15) ^ (rl & 15)) * 16;  // bytes into the chunk
    const uint32_t xvo = (uint32_t)min(t0 + rl, T - 1) * (uint32_t)ldx * 4u + (uint32_t)sw;
    uint32_t wvo[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) wvo[j] = (uint32_t)min(e0 + 32 * j + rl, E - 1) * (uint32_t)ldw * 4u + (uint32_t)sw;
    auto dma = [&](char *buf, int chunk) {
        const int so = min(chunk, nchunks - 1) * 256;  // past the last chunk: the last again, never read
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xsrc, (__attribute__((address_space(3))) void *)(buf + 4 * wave * 256),
                                                 16, xvo, so, 0, 0);
#pragma unroll
        for (int j = 0; j < NE; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wsrc, (__attribute__((address_space(3))) void *)(buf + XB + (32 * j + 4 * wave) * 256), 16, wvo[j], so,
                0, 0);
    };
    // operand reads: row r = l % 32, slot c = 2 wave + l / 32
    const int r = lane & 31, c = 2 * wave + (lane >> 5);
    const int ro = r * 256 + ((c ^ (r & 15)) * 16);
    // rows past T hold row T - 1 (the DMA clamps the row): their lanes store
    // the same bits to row T - 1, so every wave issues every chunk's store
    uint2 *xbo = CONV ? reinterpret_cast<uint2 *>(xb + (size_t)min(t0 + rl, T - 1) * ldb + sw / 4) : nullptr;
    const int own = 4 * wave * 256 + 16 * lane;  // this lane's DMA slot in a chunk buffer
    floatx16 acc[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.f;
    auto compute = [&](const char *buf, int i) {
        const float4 xv = *reinterpret_cast<const float4 *>(buf + ro);
        float4 xo;
        if constexpr (CONV) xo = *reinterpret_cast<const float4 *>(buf + own);
        float4 wv[NE];
#pragma unroll
        for (int j = 0; j < NE; ++j) wv[j] = *reinterpret_cast<const float4 *>(buf + XB + j * 32 * 256 + ro);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < NE; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32((&xv.x)[s], (&wv[j].x)[s], acc[j], 0, 0, 0);
        if constexpr (CONV) xbo[16 * i] = router_bf16x4(xo);  // columns 64 i + sw / 4 .. + 3
    };
    // chunk i's loads are done once at most the two later chunks' are in
    // flight, and (CONV) the stores of up to three earlier chunks: vector
    // memory operations are counted in issue order, a chunk's store after its
    // products, so step i waits for vmcnt(2 kDma + min(i, 3))
    constexpr int kDma = 1 + NE;
    auto step = [&](char *cur, char *ahead, int i, auto stores) {
        constexpr int n = 2 * kDma + (CONV ? decltype(stores)::value : 0);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));  // vmcnt(n) lgkmcnt(0)
        __builtin_amdgcn_s_barrier();  // every wave's part of chunk i is in; chunk i - 1 is read
        __builtin_amdgcn_sched_barrier(0);
        dma(ahead, i + 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(cur, i);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    dma(s0, 0);
    dma(s1, 1);
    dma(s2, 2);
    // nchunks is a multiple of 4 (the launcher checks)
    step(s0, s3, 0, S0{});
    step(s1, s0, 1, S1{});
    step(s2, s1, 2, S2{});
    step(s3, s2, 3, S3{});
    for (int i = 4; i < nchunks; i += 4) {
        step(s0, s3, i, S3{});
        step(s1, s0, i + 1, S3{});
        step(s2, s1, i + 2, S3{});
        step(s3, s2, i + 3, S3{});
    }
    __builtin_amdgcn_s_waitcnt(0);  // the loads past the last chunk have landed too
    __syncthreads();                // and every read of the chunk buffers is done
    // the waves' partial tiles, two per chunk buffer
    auto part = [&](int q) -> float * {
        char *b = q < 2 ? s0 : q < 4 ? s1 : q < 6 ? s2 : s3;
        return reinterpret_cast<float *>(b) + (q & 1) * PER_WAVE;
    };
    {
        float *mine = part(wave);
#pragma unroll
        for (int j = 0; j < NE; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) mine[(16 * j + i) * 64 + lane] = acc[j][i];
    }
    __syncthreads();
    // accumulator register i of tile j in lane l is token row
    // 8*(i/4) + 4*(l/32) + i%4, expert 32 j + l%32; wave q finishes the
    // registers 16 j + i = q, q + NW, ...
    const int h = lane >> 5;
    for (int ji = wave; ji < 16 * NE; ji += NW) {
        const int j = ji >> 4, i = ji & 15;
        const int t = t0 + 8 * (i >> 2) + 4 * h + (i & 3), e = e0 + 32 * j + r;
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < NW; ++q) v += part(q)[ji * 64 + lane];
        if (t < T && e < E) {
            if (row_scale) v = row_scale[t] * v;
            logits[(size_t)t * E + e] = (double)v + bias[e];
        }
    }
}

template <int NE>
__global__ __launch_bounds__(512) void router_lds_kernel(const float *__restrict__ x, int ldx, int T, int kp,
                                                         const float *__restrict__ w, int ldw,
                                                         const double *__restrict__ bias, int E,
                                                         double *__restrict__ logits,
                                                         const float *__restrict__ row_scale,
                                                         uint16_t *__restrict__ xb, int ldb,
                                                         int32_t *__restrict__ zero, int nzero)
{
    clear_counts(zero, nzero);
    // four separate arrays, so that the compiler tracks the loads into each
    __shared__ __attribute__((aligned(16))) char s0[router_lds_buf<NE>()];
    __shared__ __attribute__((aligned(16))) char s1[router_lds_buf<NE>()];
    __shared__ __attribute__((aligned(16))) char s2[router_lds_buf<NE>()];
    __shared__ __attribute__((aligned(16))) char s3[router_lds_buf<NE>()];
    // the first expert tile of each token tile writes the bf16 rows
    if (xb != nullptr && blockIdx.y == 0)
        router_lds_body<NE, true>(x, ldx, T, kp, w, ldw, bias, E, logits, row_scale, xb, ldb, s0, s1, s2, s3);
    else
        router_lds_body<NE, false>(x, ldx, T, kp, w, ldw, bias, E, logits, row_scale, nullptr, 0, s0, s1, s2, s3);
}

hipError_t launch_router(const float *x, int ldx, int T, int d, const float *w, int ldw, const double *bias, int E,
                         double *logits, hipStream_t s, const float *row_scale, uint16_t *xb, int ldb, int32_t *zero,
                         int nzero)
{
    if (T <= 0) return hipSuccess;
    // xb (optional): the bf16 copy of the rows, written by the staged kernel
    // as it reads them, else by the input conversion first
    if (xb != nullptr && (ldx != d || d % 64 != 0 || ldb < d)) return hipErrorInvalidValue;
    auto convert_first = [&]() -> hipError_t {
        return xb ? launch_convert_inputs_f32(x, T, d, nullptr, 0, xb, ldb, s) : hipSuccess;
    };
    if (T <= 256) {
        if (hipError_t e = convert_first()) return e;
        // rows are zero-padded to a multiple of 64 values
        const int kp = (d + 63) / 64 * 64;
        dim3 grid((T * E + 3) / 4);
        hipLaunchKernelGGL(router_small_kernel, grid, dim3(256), 0, s, x, ldx, T, kp, w, ldw, bias, E, logits,
                           row_scale, zero, nzero);
    } else {
        const int kp = (d + 63) / 64 * 64;
        // two expert tiles per workgroup (each token row read half as
        // often) when the grid still holds two waves per SIMD of the 256
        // CUs, with four waves over K if that is enough, else eight; one
        // tile and four waves otherwise
        const long long tiles2 = (long long)((T + 31) / 32) * ((E + 63) / 64);
        const long long tiles1 = (long long)((T + 31) / 32) * ((E + 31) / 32);
        const bool staged = kp % 256 == 0 && (long long)T * ldx * 4 <= 0x7fffffffLL &&
                            (long long)E * ldw * 4 <= 0x7fffffffLL;
        if (staged && E > 32 && tiles2 >= kRouterStagedWgs) {
            dim3 grid((T + 31) / 32, (E + 63) / 64);
            hipLaunchKernelGGL((router_lds_kernel<2>), grid, dim3(512), 0, s, x, ldx, T, kp, w, ldw, bias, E, logits,
                               row_scale, xb, ldb, zero, nzero);
            return hipGetLastError();
        } else if (staged && tiles1 >= kRouterStagedWgs) {
            dim3 grid((T + 31) / 32, (E + 31) / 32);
            hipLaunchKernelGGL((router_lds_kernel<1>), grid, dim3(512), 0, s, x, ldx, T, kp, w, ldw, bias, E, logits,
                               row_scale, xb, ldb, zero, nzero);
            return hipGetLastError();
        }
        if (hipError_t e = convert_first()) return e;
        if (E > 32 && tiles2 * 8 >= kRouterWaves) {
            dim3 grid((T + 31) / 32, (E + 63) / 64);
            if (tiles2 * 4 >= kRouterWaves)
                hipLaunchKernelGGL((router_mfma_kernel<2, 4>), grid, dim3(256), 0, s, x, ldx, T, kp, w, ldw, bias, E,
                                   logits, row_scale, zero, nzero);
            else
                hipLaunchKernelGGL((router_mfma_kernel<2, 8>), grid, dim3(512), 0, s, x, ldx, T, kp, w, ldw, bias, E,
                                   logits, row_scale, zero, nzero);
        } else {
            dim3 grid((T + 31) / 32, (E + 31) / 32);
            hipLaunchKernelGGL((router_mfma_kernel<1, 4>), grid, dim3(256), 0, s, x, ldx, T, kp, w, ldw, bias, E,
                               logits, row_scale, zero, nzero);
        }
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Top-k: one wave per token.  Score = affinity + balance bias; the k best in
// the order (score descending, expert ascending) -- exactly the first k of
// the reference's sort.SliceStable (mixtureofexperts.go:98-112) -- then
// listed in ascending expert order, gates = affinity / sum of the chosen
// affinities summed in that order (:162-169).
// ---------------------------------------------------------------------------
constexpr int kMaxExperts = 256;
constexpr int kMaxK = 8;

__device__ __forceinline__ bool better(double s1, int e1, double s2, int e2)
{
    return s1 > s2 || (s1 == s2 && e1 < e2);
}

// One level of the wave arg-max: this lane's (score, expert) against the one
// of the lane that the DPP pattern CTRL (a permutation within each row of 16
// lanes) names.  Every lane of a row takes part, so no lane reads outside it.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(double &bs, int &be)
{
    const unsigned long long u = (unsigned long long)__double_as_longlong(bs);
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xF, 0xF, false);
    const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
    const int oe = __builtin_amdgcn_update_dpp(0, be, CTRL, 0xF, 0xF, false);
    const double os = __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
    if (better(os, oe, bs, be)) {
        bs = os;
        be = oe;
    }
}

// The best of the four rows' bests (every lane of a row holds its row's),
// read from lanes 0, 16, 32 and 48: the wave's winner, the same in every lane.
__device__ __forceinline__ int argmax_rows(double bs, int be)
{
    const unsigned long long u = (unsigned long long)__double_as_longlong(bs);
    double ws = 0.0;
    int we = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, 16 * r);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), 16 * r);
        const int re = __builtin_amdgcn_readlane(be, 16 * r);
        const double rs = __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
        if (r == 0 || better(rs, re, ws, we)) {
            ws = rs;
            we = re;
        }
    }
    return we;
}

// Sum of a float over the wave, the same in every lane: DPP moves add
// within each row of 16 lanes (pairs, quads, eights, the row), then the four
// rows' sums are read from lanes 0, 16, 32 and 48 and added in a fixed order.
template <int CTRL>
__device__ __forceinline__ float add_dpp(float v)
{
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// A double of lane l (l the same in every lane), read without LDS.
__device__ __forceinline__ double lane_double(double v, int l)
{
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ float wave_sum(float v)
{
    v = add_dpp<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v = add_dpp<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v = add_dpp<0x141>(v);  // row_half_mirror
    v = add_dpp<0x140>(v);  // row_mirror
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// sort.SliceStable(candidates, score descending) of mixtureofexperts.go:106,
// step for step, for a row with NaN scores: Go's stable sort (package sort:
// insertion sort of blocks of 20, then SymMerge of neighbouring runs of 20,
// 40, 80, ... -- Kim & Kutzner, 2004), with less(i, j) = s[c[i]] > s[c[j]].
// With scores that are totally ordered every stable sort gives the order the
// arg-max rounds of topk_token find; NaN compares neither greater nor less
// than anything, and the order the reference leaves then depends on exactly
// which comparisons and swaps its sort makes, so those are repeated here.
// One lane runs it over the candidate list c[0..n) in LDS (the scores s[] in
// LDS too); SymMerge's two recursive calls work on disjoint ranges, so they
// are kept on an explicit stack (stk, 3 ints per entry; the recursion is at
// most ceil(log2 n) <= 8 deep for n <= 256, so 32 entries never fill).
constexpr int kSortStack = 32;

struct GoSort {
    int *c;
    const double *s;
    __device__ bool less(int i, int j) const { return s[c[i]] > s[c[j]]; }
    __device__ void swap(int i, int j) const
    {
        const int t = c[i];
        c[i] = c[j];
        c[j] = t;
    }
    __device__ void insertion(int a, int b) const
    {
        for (int i = a + 1; i < b; ++i)
            for (int j = i; j > a && less(j, j - 1); --j) swap(j, j - 1);
    }
    __device__ void swap_range(int a, int b, int n) const
    {
        for (int i = 0; i < n; ++i) swap(a + i, b + i);
    }
    __device__ void rotate(int a, int m, int b) const
    {
        int i = m - a, j = b - m;
        while (i != j) {
            if (i > j) {
                swap_range(m - i, m, j);
                i -= j;
            } else {
                swap_range(m - i, m + j - i, i);
                j -= i;
            }
        }
        swap_range(m - i, m, i);
    }
    __device__ void sym_merge(int a0, int m0, int b0, int *stk) const
    {
        int sp = 0;
        stk[0] = a0;
        stk[1] = m0;
        stk[2] = b0;
        sp = 1;
        while (sp > 0) {
            --sp;
            const int a = stk[3 * sp], m = stk[3 * sp + 1], b = stk[3 * sp + 2];
            if (m - a == 1) {
                int i = m, j = b;
                while (i < j) {
                    const int h = (int)((unsigned)(i + j) >> 1);
                    if (less(h, a)) i = h + 1;
                    else j = h;
                }
                for (int k = a; k < i - 1; ++k) swap(k, k + 1);
                continue;
            }
            if (b - m == 1) {
                int i = a, j = m;
                while (i < j) {
                    const int h = (int)((unsigned)(i + j) >> 1);
                    if (!less(m, h)) i = h + 1;
                    else j = h;
                }
                for (int k = m; k > i; --k) swap(k, k - 1);
                continue;
            }
            const int mid = (int)((unsigned)(a + b) >> 1);
            const int n = mid + m;
            int start, r;
            if (m > mid) {
                start = n - b;
                r = mid;
            } else {
                start = a;
                r = m;
            }
            const int p = n - 1;
            while (start < r) {
                const int cc = (int)((unsigned)(start + r) >> 1);
                if (!less(p - cc, cc)) start = cc + 1;
                else r = cc;
            }
            const int end = n - start;
            if (start < m && m < end) rotate(start, m, end);
            if (mid < end && end < b && sp < kSortStack) {
                stk[3 * sp] = mid;
                stk[3 * sp + 1] = end;
                stk[3 * sp + 2] = b;
                ++sp;
            }
            if (a < start && start < mid && sp < kSortStack) {
                stk[3 * sp] = a;
                stk[3 * sp + 1] = start;
                stk[3 * sp + 2] = mid;
                ++sp;
            }
        }
    }
    __device__ void stable(int n, int *stk) const
    {
        int block = 20, a = 0, b = block;
        while (b <= n) {
            insertion(a, b);
            a = b;
            b += block;
        }
        insertion(a, n);
        while (block < n) {
            a = 0;
            b = 2 * block;
            while (b <= n) {
                sym_merge(a, a + block, b, stk);
                a = b;
                b += 2 * block;
            }
            if (a + block < n) sym_merge(a, a + block, n, stk);
            block *= 2;
        }
    }
};

// LDS a top-k wave needs for a row with NaN scores: the scores, the
// candidate list and the merge stack.
struct TopkScratch {
    double *score;  // [kMaxExperts]
    int *cand;      // [kMaxExperts]
    int *stk;       // [3 * kSortStack]
};

// The balance biases of experts lane + 64 j (0 past E).
template <int EPL>
__device__ __forceinline__ void load_balance(const double *__restrict__ balance, int E, int lane, double (&bal)[EPL])
{
#pragma unroll
    for (int j = 0; j < EPL; ++j) bal[j] = lane + 64 * j < E ? balance[lane + 64 * j] : 0.0;
}

// Top-k of one token by one wave (EPL experts per lane; bal[j] is the
// balance bias of expert lane + 64 j, loaded ahead by the caller).  Writes
// chosen and gates (float64 and fp32) for token t; scr: LDS of the wave, used
// only when a score is NaN.  Returns, in lane i < k, the expert of slot i.
template <int EPL>
__device__ __forceinline__ int topk_token(const double *__restrict__ logit_row, int t, int E, int k,
                                           const double (&bal)[EPL], int lane, int32_t *__restrict__ chosen,
                                           double *__restrict__ gates, float *__restrict__ gates32,
                                           const TopkScratch &scr)
{
    double a[EPL], sc[EPL];
    bool taken[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        taken[j] = false;
        if (e < E) {
            a[j] = affinity(logit_row[e]);
            sc[j] = a[j] + bal[j];
        } else {
            a[j] = 0.0;
            sc[j] = -INFINITY;
        }
    }
    bool nan = false;
#pragma unroll
    for (int j = 0; j < EPL; ++j) nan = nan || (lane + 64 * j < E && sc[j] != sc[j]);
    if (__ballot(nan) == 0) {
        // totally ordered scores: k rounds of wave arg-max in the order
        // (score descending, expert ascending), the first k of any stable sort
        for (int r = 0; r < k; ++r) {
            double bs = -INFINITY;
            int be = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const int e = lane + 64 * j;
                if (e < E && !taken[j] && better(sc[j], e, bs, be)) {
                    bs = sc[j];
                    be = e;
                }
            }
            // within each row of 16 lanes by DPP moves (pairs, quads, eights,
            // the row), then across the four rows by lane reads: the same
            // total order, so the same winner as any other reduction tree
            argmax_dpp<0xB1>(bs, be);   // quad_perm [1, 0, 3, 2]
            argmax_dpp<0x4E>(bs, be);   // quad_perm [2, 3, 0, 1]
            argmax_dpp<0x141>(bs, be);  // row_half_mirror
            argmax_dpp<0x140>(bs, be);  // row_mirror
            be = argmax_rows(bs, be);
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                if (lane + 64 * j == be) taken[j] = true;
        }
    } else {
        // NaN scores: the reference's sort, repeated by lane 0
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            if (e < E) {
                scr.score[e] = sc[j];
                scr.cand[e] = e;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS stores are done
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) GoSort{scr.cand, scr.score}.stable(E, scr.stk);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int i = 0; i < k; ++i) {
            const int ce = scr.cand[i];
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                if (lane + 64 * j == ce) taken[j] = true;
        }
    }
    // chosen experts in ascending order, with their affinities (read from
    // the owning lane: b is the same in every lane)
    int list_e[kMaxK] = {};
    double list_a[kMaxK] = {};
    int n = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        unsigned long long m = __ballot(taken[j]);
        while (m) {
            const int b = __builtin_ctzll(m);
            m &= m - 1;
            const unsigned long long u = (unsigned long long)__double_as_longlong(a[j]);
            const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, b);
            const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), b);
            const double av = __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
#pragma unroll
            for (int i = 0; i < kMaxK; ++i)
                if (i == n) {
                    list_e[i] = 64 * j + b;
                    list_a[i] = av;
                }
            ++n;
        }
    }
    double total = 0.0;
#pragma unroll
    for (int i = 0; i < kMaxK; ++i)
        if (i < k) total += list_a[i];
    // lane i < k takes slot i; the k divisions run side by side
    int mine = -1;
    double my_a = 0.0;
#pragma unroll
    for (int i = 0; i < kMaxK; ++i)
        if (lane == i) {
            mine = list_e[i];
            my_a = list_a[i];
        }
    if (lane < k) {
        const double g = my_a / total;
        chosen[(size_t)t * k + lane] = mine;
        gates[(size_t)t * k + lane] = g;
        gates32[(size_t)t * k + lane] = (float)g;
    } else {
        mine = -1;
    }
    return mine;
}

// Tokens per chunk of the many-token dispatch, whose counts are per chunk
// and expert.
constexpr int kChunk = 128;

// chunk_cnt (optional, [chunks][E], zero on entry): each (token, slot) adds
// one to its chunk's count of its expert.  The counts do not depend on the
// order of the adds, so the dispatch built from them is the same as from
// dispatch_count_kernel.
template <int EPL>
__global__ __launch_bounds__(256) void topk_kernel(const double *__restrict__ logits, int T, int E, int k,
                                                   const double *__restrict__ balance, int32_t *__restrict__ chosen,
                                                   double *__restrict__ gates, float *__restrict__ gates32,
                                                   int32_t *__restrict__ chunk_cnt)
{
    __shared__ double score[4][kMaxExperts];
    __shared__ int cand[4][kMaxExperts];
    __shared__ int stk[4][3 * kSortStack];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;  // wave-uniform
    double bal[EPL];
    load_balance<EPL>(balance, E, lane, bal);
    const int mine = topk_token<EPL>(logits + (size_t)t * E, t, E, k, bal, lane, chosen, gates, gates32,
                                     TopkScratch{score[wave], cand[wave], stk[wave]});
    if (chunk_cnt != nullptr && lane < k) atomicAdd(chunk_cnt + (size_t)(t / kChunk) * E + mine, 1);
}

hipError_t launch_topk(const double *logits, int T, int E, int k, const double *balance, int32_t *chosen,
                       double *gates, float *gates32, hipStream_t s, int32_t *chunk_cnt)
{
    if (T <= 0) return hipSuccess;
    dim3 grid((T + 3) / 4);
    if (E <= 64)
        hipLaunchKernelGGL(topk_kernel<1>, grid, dim3(256), 0, s, logits, T, E, k, balance, chosen, gates, gates32,
                           chunk_cnt);
    else if (E <= 128)
        hipLaunchKernelGGL(topk_kernel<2>, grid, dim3(256), 0, s, logits, T, E, k, balance, chosen, gates, gates32,
                           chunk_cnt);
    else
        hipLaunchKernelGGL(topk_kernel<4>, grid, dim3(256), 0, s, logits, T, E, k, balance, chosen, gates, gates32,
                           chunk_cnt);
    return hipGetLastError();
}

// hashedExperts (mixtureofexperts.go:88-96): first = (id*2654435761 + 12345)
// mod E in unsigned 64-bit arithmetic, then k consecutive experts; gates 1/k.
// Ids are checked non-negative by the host before launch.
__device__ __forceinline__ void hash_token(const int64_t *__restrict__ ids, int t, int E, int k,
                                           int32_t *__restrict__ chosen, double *__restrict__ gates,
                                           float *__restrict__ gates32)
{
    const unsigned long long first =
        ((unsigned long long)ids[t] * 2654435761ULL + 12345ULL) % (unsigned long long)E;
    const double g = 1 / (double)k;
    for (int i = 0; i < k; ++i) {
        const int32_t e = (int32_t)((first + (unsigned long long)i) % (unsigned long long)E);
        chosen[(size_t)t * k + i] = e;
        gates[(size_t)t * k + i] = g;
        gates32[(size_t)t * k + i] = (float)g;
    }
}

__global__ void hash_route_kernel(const int64_t *__restrict__ ids, int T, int E, int k, int32_t *__restrict__ chosen,
                                  double *__restrict__ gates, float *__restrict__ gates32)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    hash_token(ids, t, E, k, chosen, gates, gates32);
}

hipError_t launch_hash_route(const int64_t *ids, int T, int E, int k, int32_t *chosen, double *gates, float *gates32,
                             hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(hash_route_kernel, dim3((T + 255) / 256), dim3(256), 0, s, ids, T, E, k, chosen, gates,
                       gates32);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dispatch (mixtureofexperts.go:175-190): per-expert load, exclusive offsets,
// and a stable permutation -- experts ascending, tokens ascending inside an
// expert.  The rank of a token inside its expert comes from wave ballots and
// prefix sums, never from an atomic, so the order is the reference's.  Also
// fills the position tables the expert kernels use (goff, tok) and the
// per-group MFMA tile prefix (tile_off).
// ---------------------------------------------------------------------------
constexpr int kScanMax = 1024;  // experts + shared experts handled by the scans

// Exclusive scan of vals[0..n) (n <= 1024) by a 1024-thread workgroup into
// out[0..n); returns the total.  vals and out may alias.
__device__ int block_exclusive_scan(const int *vals, int *out, int n, int *wave_sums, int *total_slot)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int v = tid < n ? vals[tid] : 0;
    int x = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63) wave_sums[wave] = x;
    __syncthreads();
    if (wave == 0) {
        int w = lane < 16 ? wave_sums[lane] : 0;
        int inc = w;
        for (int off = 1; off < 16; off <<= 1) {
            const int y = __shfl_up(inc, off);
            if (lane >= off) inc += y;
        }
        if (lane < 16) wave_sums[lane] = inc - w;
        if (lane == 15) *total_slot = inc;
    }
    __syncthreads();
    if (tid < n) out[tid] = x - v + wave_sums[wave];
    __syncthreads();
    return *total_slot;
}

struct DispatchShared {
    int cnt[kScanMax];
    int base[kScanMax];
    int tiles[kScanMax];
    int wave_cnt[16][kMaxExperts];
    int wave_sums[16];
    int total;
};

// Group tables from per-expert counts (in sh.cnt) and their exclusive
// offsets (in sh.base): load, offsets, goff, tile_off and the shared-expert
// part of tok.
__device__ void write_group_tables(int T, int k, int E, int S, int bm, DispatchShared &sh, int32_t *__restrict__ load,
                                   int32_t *__restrict__ offsets, int32_t *__restrict__ goff,
                                   int32_t *__restrict__ tok, int32_t *__restrict__ tile_off,
                                   int4 *__restrict__ tile_desc)
{
    const int tid = threadIdx.x;
    const int G = S + E;
    for (int e = tid; e < E; e += blockDim.x) {
        load[e] = sh.cnt[e];
        offsets[e] = sh.base[e];
    }
    if (tid == 0) offsets[E] = T * k;
    for (int g = tid; g < G; g += blockDim.x) {
        const int m = g < S ? T : sh.cnt[g - S];
        sh.tiles[g] = (m + bm - 1) / bm;
        goff[g] = g < S ? g * T : S * T + sh.base[g - S];
    }
    if (tid == 0) goff[G] = S * T + T * k;
    __syncthreads();
    const int total_tiles = block_exclusive_scan(sh.tiles, sh.tiles, G, sh.wave_sums, &sh.total);
    for (int g = tid; g < G; g += blockDim.x) {
        tile_off[g] = sh.tiles[g];
        const int end = g + 1 < G ? sh.tiles[g + 1] : total_tiles;
        const int m = g < S ? T : sh.cnt[g - S];
        const int p = g < S ? g * T : S * T + sh.base[g - S];
        for (int t = sh.tiles[g]; t < end; ++t) {
            // tile -> (group, first position, positions)
            const int first = (t - sh.tiles[g]) * bm;
            tile_desc[t] = make_int4(g, p + first, min(bm, m - first), 0);
        }
    }
    if (tid == 0) tile_off[G] = total_tiles;
    for (long long p = tid; p < (long long)S * T; p += blockDim.x) tok[p] = (int32_t)(p % T);
}

// Whole dispatch by one 1024-thread workgroup for T <= 1024; `chosen` may be
// in LDS.  Tokens form token-waves of 64 (lane = token); the (token-wave,
// expert) pairs are spread over the 16 waves.  For each pair a ballot of
// "has this expert" gives the pair's count (pass 1) and every token's rank
// (pass 2); a per-expert prefix over token-waves in between turns counts into
// starting positions.  No atomics, and every wave has a share of the work.
__device__ void dispatch_block(const int32_t *chosen, int T, int k, int E, int S, int bm, int32_t *__restrict__ load,
                               int32_t *__restrict__ offsets, int32_t *__restrict__ rows, int32_t *__restrict__ pos,
                               int32_t *__restrict__ goff, int32_t *__restrict__ tok,
                               int32_t *__restrict__ tile_off, int4 *__restrict__ tile_desc, DispatchShared &sh)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ntw = (T + 63) / 64;  // token-waves, <= 16
    int ntwp = 1;
    while (ntwp < ntw) ntwp <<= 1;
    const int wpt = 16 / ntwp;  // waves per token-wave
    const int tw = wave / wpt, sub = wave % wpt;
    const int t = tw * 64 + lane;
    const bool active = tw < ntw;
    int ce[kMaxK];
#pragma unroll
    for (int i = 0; i < kMaxK; ++i) ce[i] = (active && t < T && i < k) ? chosen[(size_t)t * k + i] : -1;

    // pass 1: counts per (token-wave, expert)
    if (active) {
        for (int e = sub; e < E; e += wpt) {
            bool has = false;
#pragma unroll
            for (int i = 0; i < kMaxK; ++i) has |= ce[i] == e;
            const unsigned long long b = __ballot(has);
            if (lane == 0) sh.wave_cnt[tw][e] = __popcll(b);
        }
    }
    __syncthreads();
    // per-expert totals and the prefix over token-waves
    for (int e = tid; e < E; e += 1024) {
        int acc = 0;
        for (int w = 0; w < ntw; ++w) acc += sh.wave_cnt[w][e];
        sh.cnt[e] = acc;
    }
    __syncthreads();
    block_exclusive_scan(sh.cnt, sh.base, E, sh.wave_sums, &sh.total);
    write_group_tables(T, k, E, S, bm, sh, load, offsets, goff, tok, tile_off, tile_desc);
    for (int e = tid; e < E; e += 1024) {
        int acc = sh.base[e];
        for (int w = 0; w < ntw; ++w) {
            const int c = sh.wave_cnt[w][e];
            sh.wave_cnt[w][e] = acc;
            acc += c;
        }
    }
    __syncthreads();
    // pass 2: positions
    if (active) {
        for (int e = sub; e < E; e += wpt) {
            int match = -1;
#pragma unroll
            for (int i = 0; i < kMaxK; ++i)
                if (ce[i] == e) match = i;
            const unsigned long long b = __ballot(match >= 0);
            if (match >= 0) {
                const int p = sh.wave_cnt[tw][e] + __popcll(b & ((1ULL << lane) - 1ULL));
                rows[p] = t;
                pos[(size_t)t * k + match] = p;
                tok[(size_t)S * T + p] = t;
            }
        }
    }
}

// With pack.n > 0 the same workgroup then gathers pack's parts into
// pack_dst as pack_words_kernel does (the routing state of a host-API
// forward), one launch fewer.
__global__ __launch_bounds__(1024) void dispatch_kernel(const int32_t *__restrict__ chosen, int T, int k, int E, int S,
                                                        int bm, int32_t *__restrict__ load, int32_t *__restrict__ offsets,
                                                        int32_t *__restrict__ rows, int32_t *__restrict__ pos,
                                                        int32_t *__restrict__ goff, int32_t *__restrict__ tok,
                                                        int32_t *__restrict__ tile_off, int4 *__restrict__ tile_desc,
                                                        PackParts pack, uint32_t *__restrict__ pack_dst)
{
    __shared__ DispatchShared sh;
    dispatch_block(chosen, T, k, E, S, bm, load, offsets, rows, pos, goff, tok, tile_off, tile_desc, sh);
    if (pack.n <= 0) return;
    __syncthreads();  // the tables this workgroup wrote are visible to all of it
    uint32_t *out = pack_dst;
    for (int i = 0; i < PackParts::kMax; ++i) {
        if (i >= pack.n) break;
        const uint32_t *src = pack.src[i];
        for (int j = threadIdx.x; j < pack.words[i]; j += 1024) out[j] = src[j];
        out += (pack.words[i] + 15) / 16 * 16;
    }
}

// Many tokens: chunks of kChunk tokens per workgroup.
//   count:   per-chunk, per-expert counts            -> chunk_cnt[c][e]
//   scan:    one workgroup: per-expert totals, offsets, the group tables, and
//            every chunk's starting position per expert -> chunk_cnt[c][e]
//   scatter: per chunk, wave ranks + the chunk's base  -> rows, pos, tok
// kChunk = 128 tokens per chunk: twice the workgroups of 256 for a shorter
// per-workgroup chain (C3 dispatch 16.5 → 15.6 µs); every placement
// workgroup reads all chunks' counts, so the chunks are not made smaller.
// The counts come from the top-k when it runs just before (launch_topk with
// chunk_cnt), else from dispatch_count_kernel.

__global__ __launch_bounds__(kChunk) void dispatch_count_kernel(const int32_t *__restrict__ chosen, int T, int k, int E,
                                                                int32_t *__restrict__ chunk_cnt)
{
    __shared__ int cnt[kMaxExperts];
    for (int e = threadIdx.x; e < E; e += kChunk) cnt[e] = 0;
    __syncthreads();
    const int t = blockIdx.x * kChunk + threadIdx.x;
    if (t < T)
        for (int i = 0; i < k; ++i) atomicAdd(&cnt[chosen[(size_t)t * k + i]], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kChunk) chunk_cnt[(size_t)blockIdx.x * E + e] = cnt[e];
}

// Placement of one chunk of kChunk tokens, 16 waves.  Every workgroup sums
// the per-chunk counts itself (threads split the chunks of each expert), so
// the totals, the experts' offsets and its own chunk's start need no
// separate scan launch; workgroup 0 also writes the group tables.  Ranks
// inside the chunk come from wave ballots, with the (token-wave, expert)
// pairs spread over the 16 waves.  No atomic decides a position: the LDS
// atomics only add up counts.
__global__ __launch_bounds__(1024) void dispatch_place_kernel(const int32_t *__restrict__ chosen, int T, int k, int E,
                                                              int S, int bm, int chunks,
                                                              const int32_t *__restrict__ chunk_cnt,
                                                              int32_t *__restrict__ load, int32_t *__restrict__ offsets,
                                                              int32_t *__restrict__ rows, int32_t *__restrict__ pos,
                                                              int32_t *__restrict__ goff, int32_t *__restrict__ tok,
                                                              int32_t *__restrict__ tile_off,
                                                              int4 *__restrict__ tile_desc)
{
    __shared__ DispatchShared sh;
    __shared__ int before[kMaxExperts];
    __shared__ int rank_lds[kChunk][kMaxK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = blockIdx.x;
    for (int e = tid; e < E; e += 1024) {
        sh.cnt[e] = 0;
        before[e] = 0;
    }
    __syncthreads();
    // totals over all chunks and over the chunks before this one
    const int per = 1024 / E;  // threads per expert (E <= 256)
    if (tid < per * E) {
        const int e = tid % E, j = tid / E;
        int tot = 0, bef = 0;
        int cc = j;
        for (; cc + 3 * per < chunks; cc += 4 * per) {
            const int n0 = chunk_cnt[(size_t)cc * E + e], n1 = chunk_cnt[(size_t)(cc + per) * E + e];
            const int n2 = chunk_cnt[(size_t)(cc + 2 * per) * E + e], n3 = chunk_cnt[(size_t)(cc + 3 * per) * E + e];
            tot += n0 + n1 + n2 + n3;
            bef += (cc < c ? n0 : 0) + (cc + per < c ? n1 : 0) + (cc + 2 * per < c ? n2 : 0) + (cc + 3 * per < c ? n3 : 0);
        }
        for (; cc < chunks; cc += per) {
            const int n = chunk_cnt[(size_t)cc * E + e];
            tot += n;
            bef += cc < c ? n : 0;
        }
        atomicAdd(&sh.cnt[e], tot);
        atomicAdd(&before[e], bef);
    }
    __syncthreads();
    block_exclusive_scan(sh.cnt, sh.base, E, sh.wave_sums, &sh.total);
    if (c == 0) write_group_tables(T, k, E, S, bm, sh, load, offsets, goff, tok, tile_off, tile_desc);

    // ranks inside the chunk: the 16 waves cover the chunk's kChunk / 64
    // token-waves, kSubsets waves per token-wave; wave w covers token-wave
    // w / kSubsets and the experts e = w % kSubsets (mod kSubsets)
    constexpr int kSubsets = 16 / (kChunk / 64);
    const int tw = wave / kSubsets, sub = wave % kSubsets;
    const int tl = tw * 64 + lane;
    const int t = c * kChunk + tl;
    int ce[kMaxK];
#pragma unroll
    for (int i = 0; i < kMaxK; ++i) ce[i] = (t < T && i < k) ? chosen[(size_t)t * k + i] : -1;
    for (int e = sub; e < E; e += kSubsets) {
        int match = -1;
#pragma unroll
        for (int i = 0; i < kMaxK; ++i)
            if (ce[i] == e) match = i;
        const unsigned long long b = __ballot(match >= 0);
        if (lane == 0) sh.wave_cnt[tw][e] = __popcll(b);
        if (match >= 0) rank_lds[tl][match] = __popcll(b & ((1ULL << lane) - 1ULL));
    }
    __syncthreads();
    // first position of each (token-wave, expert)
    for (int e = tid; e < E; e += 1024) {
        int acc = sh.base[e] + before[e];
#pragma unroll
        for (int w = 0; w < kChunk / 64; ++w) {
            const int n = sh.wave_cnt[w][e];
            sh.wave_cnt[w][e] = acc;
            acc += n;
        }
    }
    __syncthreads();
    if (tid < kChunk) {
        const int tt = c * kChunk + tid;
        if (tt < T) {
            for (int i = 0; i < k; ++i) {
                const int e = chosen[(size_t)tt * k + i];
                const int p = sh.wave_cnt[tid >> 6][e] + rank_lds[tid][i];
                rows[p] = tt;
                pos[(size_t)tt * k + i] = p;
                tok[(size_t)S * T + p] = tt;
            }
        }
    }
}

hipError_t launch_dispatch_packed(const int32_t *chosen, int T, int k, int E, int S, int bm, int32_t *load,
                                  int32_t *offsets, int32_t *rows, int32_t *pos, int32_t *goff, int32_t *tok,
                                  int32_t *tile_off, int4 *tile_desc, const PackParts &pack, uint32_t *dst,
                                  hipStream_t s)
{
    if (T > 1024 || pack.n < 1 || pack.n > PackParts::kMax) return hipErrorInvalidValue;
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, chosen, T, k, E, S, bm, load, offsets, rows, pos,
                       goff, tok, tile_off, tile_desc, pack, dst);
    return hipGetLastError();
}

int dispatch_chunks(int T) { return (T + kChunk - 1) / kChunk; }
bool dispatch_chunked(int T) { return T > 1024; }

hipError_t launch_dispatch(const int32_t *chosen, int T, int k, int E, int S, int bm, int32_t *load, int32_t *offsets,
                           int32_t *rows, int32_t *pos, int32_t *goff, int32_t *tok, int32_t *tile_off,
                           int4 *tile_desc, int32_t *chunk_cnt, hipStream_t s, bool counted)
{
    if (!dispatch_chunked(T)) {  // one workgroup: token-waves x experts over its 16 waves
        hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, chosen, T, k, E, S, bm, load, offsets, rows,
                           pos, goff, tok, tile_off, tile_desc, PackParts{}, nullptr);
        return hipGetLastError();
    }
    const int chunks = dispatch_chunks(T);
    if (!counted) hipLaunchKernelGGL(dispatch_count_kernel, dim3(chunks), dim3(kChunk), 0, s, chosen, T, k, E, chunk_cnt);
    hipLaunchKernelGGL(dispatch_place_kernel, dim3(chunks), dim3(1024), 0, s, chosen, T, k, E, S, bm, chunks,
                       chunk_cnt, load, offsets, rows, pos, goff, tok, tile_off, tile_desc);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Routing for few tokens (decode): route_token_kernel (one workgroup per
// token: input preparation, router logits, top-k or hash routing), then
// dispatch_kernel unless the expert kernels find their own tokens.  With RMSNorm in front
// (normalization/rmsnorm.go:33-53) the norm weights are folded into the
// router rows (wn = w * norm) and the inverse RMS comes from a pass over the
// raw row, logit = inv_rms * dot(x, wn) + bias.
// ---------------------------------------------------------------------------
constexpr int kFusedMaxTK = 2048;  // T*k handled by the two-launch routing

__device__ __forceinline__ uint16_t bf16_bits(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <typename InT>
__device__ __forceinline__ float in_at(const InT *row, int i)
{
    return (float)row[i];
}

// four consecutive inputs starting at a 4-aligned index (16 B aligned for
// float rows, 32 B for double rows when d is a multiple of 4)
__device__ __forceinline__ float4 in4(const float *row, int i) { return *reinterpret_cast<const float4 *>(row + i); }
__device__ __forceinline__ float4 in4(const double *row, int i)
{
    const double2 a = *reinterpret_cast<const double2 *>(row + i);
    const double2 b = *reinterpret_cast<const double2 *>(row + i + 2);
    return make_float4((float)a.x, (float)a.y, (float)b.x, (float)b.y);
}

// One 1024-thread workgroup per token.  Every wave keeps the token's row in
// registers (NX float4 runs per lane, d <= 256*NX); the 16 waves share the
// experts, two router rows in flight at a time; logits go to LDS, then wave
// 0 runs top-k (or hash routing).  The token's prepared row (converted or
// normalised, zero-padded) is written from those registers, run j by wave j
// (rows whose width is not a multiple of 4 re-read the input).  The small
// operands (router and balance biases, norm weights) are loaded at the start
// so that their latency overlaps the row's.
//
// With a.parts = P > 1 (few tokens, many experts) each token has P
// workgroups, part p taking experts [p ceil(E/P), (p + 1) ceil(E/P)), so
// that the router's rows are read by P CUs at once: every part prepares the
// row (the pending combine and the norm, in registers), but only part 0
// writes the combined residual row (to a.x_out, never in place: the other
// parts still read the old row), the prepared row and the zeroed output
// row.  Wave 0 of each part publishes its logits to a.logits and counts the
// part in a.part_cnt[t]; the part that arrives last runs the top-k over all
// of them and resets the count.  No part waits for another.  The logits
// travel as agent-scope atomic stores and loads, which the hardware performs
// at the device's point of coherence (write-through, past the XCD's L2), and
// the count is incremented only once those stores are acknowledged
// (s_waitcnt vmcnt(0)).  A release/acquire pair would give the same ordering
// through a whole-L2 write-back per workgroup and an L2 invalidation per
// token; measured, that cost more than the split saved.
//
// The grid's workgroups past the T * P routing ones (router routing only)
// warm the L2 of their XCD with the router rows its routing workgroups will
// read, while those are still loading and combining the token rows: a
// stack's layer reads its router once per step, and the expert weights
// streamed in between leave none of it in any L2.  The dispatcher deals a
// 1-D grid's workgroups to the 8 XCDs in turn, so workgroup b runs on XCD
// b % 8, and with P dividing 8 the routing workgroups there are all of part
// (b % 8) % P; otherwise every XCD warms all E rows.  Warming workgroup
// 8 j + x of the nw = 8 Q takes slice j of Q of its XCD's rows, one 16-byte
// load per lane per 16 KiB, and keeps nothing.
__device__ __forceinline__ void warm_router(const FusedArgs &a)
{
    const int P = a.parts;
    const int nroute = a.T * P;
    const int i = blockIdx.x - nroute, nq = a.warm_blocks / 8;
    const int xcd = blockIdx.x & 7;
    int r0 = 0, r1 = a.E;
    if (8 % P == 0) {
        const int epp = (a.E + P - 1) / P;
        r0 = min(a.E, (xcd % P) * epp);
        r1 = min(a.E, r0 + epp);
    }
    const size_t n16 = (size_t)(r1 - r0) * a.kp / 4;  // 16-byte units of those rows
    const uint4 *base = reinterpret_cast<const uint4 *>(a.w + (size_t)r0 * a.kp);
    const int j = i / 8;
    const size_t b0 = n16 * j / nq, b1 = n16 * (j + 1) / nq;
    uint32_t acc = 0;
    for (size_t u0 = b0; u0 < b1; u0 += 4096) {
        uint4 v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const size_t u = u0 + threadIdx.x + 1024 * r;
            v[r] = u < b1 ? base[u] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc ^= v[r].x ^ v[r].y ^ v[r].z ^ v[r].w;
    }
    asm volatile("" ::"v"(acc));  // the loads are kept, and waited for before the wave ends
}

// Read-ahead workgroup i of n: slice i of n of each region, one 16-byte
// load per lane per 16 KiB (four in flight), nothing kept.
__device__ __forceinline__ void read_ahead(const FusedArgs &a, int i, int n)
{
    uint32_t acc = 0;
#pragma unroll 1
    for (int r = 0; r < 4; ++r) {
        const size_t n16 = a.ra_bytes[r] / 16;
        const uint4 *base = reinterpret_cast<const uint4 *>(a.ra[r]);
        const size_t b0 = n16 * i / n, b1 = n16 * (i + 1) / n;
        for (size_t u0 = b0; u0 < b1; u0 += 4096) {
            uint4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const size_t u = u0 + threadIdx.x + 1024 * q;
                v[q] = u < b1 ? base[u] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) acc ^= v[q].x ^ v[q].y ^ v[q].z ^ v[q].w;
        }
    }
    asm volatile("" ::"v"(acc));  // the loads are kept, and waited for before the wave ends
}

// Warming workgroups for a router routing launch whose routing workgroups
// fit the GPU at once (a later round would find the rows warm anyway): 8 per
// 16 KiB of the rows one XCD reads, at most 16 per XCD.
static int route_warm_blocks(int T, int E, int kp, int parts, bool hash)
{
    if (hash || T * parts > 256) return 0;
    const int rows = 8 % parts == 0 ? (E + parts - 1) / parts : E;
    const long long n16 = (long long)rows * kp / 4;
    return 8 * (int)std::min<long long>(16, std::max<long long>(1, (n16 + 1023) / 1024));
}

template <typename InT, bool NORM, bool HASH, int EPL, int NX>
__global__ __launch_bounds__(1024) void route_token_kernel(FusedArgs a)
{
    if (!HASH && (int)blockIdx.x >= a.T * a.parts) {
        const int j = blockIdx.x - a.T * a.parts - a.warm_blocks;
        if (j < 0) warm_router(a);
        else read_ahead(a, j, a.ra_blocks);
        return;
    }
    __shared__ double lg[kMaxExperts];
    __shared__ int cand[kMaxExperts];  // the top-k's candidate list and merge stack (NaN rows)
    __shared__ int stk[3 * kSortStack];
    __shared__ __attribute__((aligned(16))) float comb[NX * 256];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int P = a.parts;
    const int t = blockIdx.x / P, part = blockIdx.x - t * P;
    const int epp = (a.E + P - 1) / P;
    const int eb = part * epp, ee = min(a.E, eb + epp);  // this part's experts
    const InT *xr = reinterpret_cast<const InT *>(a.x) + (size_t)t * a.d;
    const bool vec = (a.d & 3) == 0;

    // Each phase below issues all of its loads before it uses any of them, so
    // that a wave waits for one round trip per phase: addresses are clamped
    // into the row (never a branch around a load) and what lies past the row
    // is masked after the load.
    // the small operands (router and balance biases, norm weights), requested
    // first: the combine or the row's loads cover their latency
    double bias_l = 0.0;  // router bias of expert wave + 16 j in lane j
    double bal[EPL];      // balance biases (wave 0)
    if (!HASH) {
        if (eb + wave + 16 * lane < ee) bias_l = a.bias[eb + wave + 16 * lane];
        if (wave == 0) load_balance<EPL>(a.balance, a.E, lane, bal);
    }
    float4 nv = make_float4(1.f, 1.f, 1.f, 1.f);
    if (NORM && vec && wave < NX && 4 * lane + 256 * wave < a.d)
        nv = *reinterpret_cast<const float4 *>(a.norm + 4 * lane + 256 * wave);

    bool from_comb = false;  // the token's row is in comb (LDS)
    if constexpr (sizeof(InT) == 4) {
        if (a.pend_slot) {  // the previous layer's combine (combine_kernel's arithmetic)
            const float *xin_row = reinterpret_cast<const float *>(xr);
            float *x = a.x_out ? a.x_out + (size_t)t * a.d : const_cast<float *>(xin_row);
            // the routed rows and gates of this token (at most 8; slots past
            // pend_k re-read slot 0 and are not added), all requested before
            // the adds, which keep the reference's order.  Without a pos
            // table the rows' addresses need no load, and the gates are
            // requested after the rows.
            const float *row[8];
            if (a.pend_pos) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int q = a.pend_pos[(size_t)t * a.pend_k + (i < a.pend_k ? i : 0)];
                    row[i] = a.pend_slot + (size_t)(a.pend_S * a.T + q) * a.d;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    row[i] = a.pend_slot + (size_t)(a.pend_S * a.T + t * a.pend_k + (i < a.pend_k ? i : 0)) * a.d;
            }
            float g[8];
            auto load_gates = [&]() {
#pragma unroll
                for (int i = 0; i < 8; ++i) g[i] = a.pend_gates[(size_t)t * a.pend_k + (i < a.pend_k ? i : 0)];
            };
            // the first four shared experts' rows (past pend_S: shared row 0,
            // or with no shared experts a routed row, not added)
            const float *srow[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) srow[s] = a.pend_slot + ((size_t)(s < a.pend_S ? s : 0) * a.T + t) * a.d;
            if (vec) {  // four values per lane (d <= 4096)
                const int c = 4 * (int)threadIdx.x;
                if (c < a.d) {
                    float4 v8[8], sh[4];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v8[i] = *reinterpret_cast<const float4 *>(row[i] + c);
#pragma unroll
                    for (int s = 0; s < 4; ++s) sh[s] = *reinterpret_cast<const float4 *>(srow[s] + c);
                    const float4 xc = *reinterpret_cast<const float4 *>(xin_row + c);
                    load_gates();
                    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        if (s < a.pend_S) {
                            acc.x += sh[s].x;
                            acc.y += sh[s].y;
                            acc.z += sh[s].z;
                            acc.w += sh[s].w;
                        }
                    for (int s = 4; s < a.pend_S; ++s) {
                        const float4 u = *reinterpret_cast<const float4 *>(a.pend_slot + ((size_t)s * a.T + t) * a.d + c);
                        acc.x += u.x;
                        acc.y += u.y;
                        acc.z += u.z;
                        acc.w += u.w;
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (i < a.pend_k) {
                            acc.x = fmaf(g[i], v8[i].x, acc.x);
                            acc.y = fmaf(g[i], v8[i].y, acc.y);
                            acc.z = fmaf(g[i], v8[i].z, acc.z);
                            acc.w = fmaf(g[i], v8[i].w, acc.w);
                        }
                    const float4 v = make_float4(xc.x + acc.x, xc.y + acc.y, xc.z + acc.z, xc.w + acc.w);
                    if (part == 0) *reinterpret_cast<float4 *>(x + c) = v;
                    *reinterpret_cast<float4 *>(comb + c) = v;
                }
            } else {
                load_gates();
                for (int c = threadIdx.x; c < a.d; c += 1024) {
                    float v8[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v8[i] = row[i][c];
                    const float xc = xin_row[c];
                    float acc = 0.f;
                    for (int s = 0; s < a.pend_S; ++s) acc += a.pend_slot[((size_t)s * a.T + t) * a.d + c];
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (i < a.pend_k) acc = fmaf(g[i], v8[i], acc);
                    const float v = xc + acc;
                    if (part == 0) x[c] = v;
                    comb[c] = v;
                }
            }
            __syncthreads();
            from_comb = true;
        }
    }

    // the row, zero past d
    float4 xv[NX];
    if (from_comb) {
#pragma unroll
        for (int j = 0; j < NX; ++j) xv[j] = *reinterpret_cast<const float4 *>(comb + 4 * lane + 256 * j);
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const int i = 4 * lane + 256 * j;
            if (i >= a.d) xv[j].x = 0.f;
            if (i + 1 >= a.d) xv[j].y = 0.f;
            if (i + 2 >= a.d) xv[j].z = 0.f;
            if (i + 3 >= a.d) xv[j].w = 0.f;
        }
    } else if (vec) {
#pragma unroll
        for (int j = 0; j < NX; ++j) xv[j] = in4(xr, min(4 * lane + 256 * j, a.d - 4));
#pragma unroll
        for (int j = 0; j < NX; ++j)
            if (4 * lane + 256 * j >= a.d) xv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            const int i = 4 * lane + 256 * j;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < a.d) v.x = in_at(xr, i);
            if (i + 1 < a.d) v.y = in_at(xr, i + 1);
            if (i + 2 < a.d) v.z = in_at(xr, i + 2);
            if (i + 3 < a.d) v.w = in_at(xr, i + 3);
            xv[j] = v;
        }
    }
    float ss = 0.f;
    if (NORM) {
#pragma unroll
        for (int j = 0; j < NX; ++j) {
            ss = fmaf(xv[j].x, xv[j].x, ss);
            ss = fmaf(xv[j].y, xv[j].y, ss);
            ss = fmaf(xv[j].z, xv[j].z, ss);
            ss = fmaf(xv[j].w, xv[j].w, ss);
        }
    }
    float inv = 1.0f;
    if (NORM) {
        ss = wave_sum(ss);
        inv = 1.0f / sqrtf(ss / (float)a.d + 1e-6f);
    }

    // prepared row (part 0); up to d = 2048 it is written before the
    // products, so that the norm weights need no register across them
    auto write_prepared = [&]() {
        if (part != 0) {
        } else if (vec) {
#pragma unroll
            for (int j = 0; j < NX; ++j) {
                const int i = 4 * lane + 256 * j;
                if (j == wave && i < a.kp) {  // i < d, or padding (xv holds zeros there)
                    float4 v = xv[j];
                    if (NORM) {
                        v.x = v.x * inv * nv.x;
                        v.y = v.y * inv * nv.y;
                        v.z = v.z * inv * nv.z;
                        v.w = v.w * inv * nv.w;
                        if (i >= a.d) v = make_float4(0.f, 0.f, 0.f, 0.f);
                    }
                    if (a.xf) *reinterpret_cast<float4 *>(a.xf + (size_t)t * a.kp + i) = v;
                    if (a.xb) {
                        const uint2 b = make_uint2((uint32_t)bf16_bits(v.x) | ((uint32_t)bf16_bits(v.y) << 16),
                                                   (uint32_t)bf16_bits(v.z) | ((uint32_t)bf16_bits(v.w) << 16));
                        *reinterpret_cast<uint2 *>(a.xb + (size_t)t * a.kp + i) = b;
                    }
                }
            }
        } else {
            for (int i = threadIdx.x; i < a.kp; i += 1024) {
                float v = 0.f;
                if (i < a.d) {
                    v = from_comb ? comb[i] : in_at(xr, i);
                    if (NORM) v = v * inv * a.norm[i];
                }
                if (a.xf) a.xf[(size_t)t * a.kp + i] = v;
                if (a.xb) a.xb[(size_t)t * a.kp + i] = bf16_bits(v);
            }
        }
        if (a.zero_out && part == 0)
            for (int i = threadIdx.x; i < a.d; i += 1024) a.zero_out[(size_t)t * a.d + i] = 0.f;
    };
    if constexpr (NX <= 8) write_prepared();
    if (!HASH) {
        for (int e0 = eb + wave; e0 < ee; e0 += 32) {
            const int e1 = e0 + 16;
            const bool two = e1 < ee;
            const float *w0 = a.w + (size_t)e0 * a.kp;
            const float *w1 = a.w + (size_t)(two ? e1 : e0) * a.kp;
            float d0 = 0.f, d1 = 0.f;
            // a group of runs of both rows in flight (64 registers up to d = 2048,
            // 16 above, where the row itself holds 64), then their products
            constexpr int G = NX <= 8 ? NX : 2;
#pragma unroll
            for (int jb = 0; jb < NX; jb += G) {
                float4 p[G], q[G];
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    const int ic = min(4 * lane + 256 * (jb + j), a.kp - 4);
                    p[j] = *reinterpret_cast<const float4 *>(w0 + ic);
                    q[j] = *reinterpret_cast<const float4 *>(w1 + ic);
                }
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    if (4 * lane + 256 * (jb + j) < a.kp) {
                        const float4 x4 = xv[jb + j];
                        d0 = fmaf(x4.x, p[j].x, d0);
                        d0 = fmaf(x4.y, p[j].y, d0);
                        d0 = fmaf(x4.z, p[j].z, d0);
                        d0 = fmaf(x4.w, p[j].w, d0);
                        d1 = fmaf(x4.x, q[j].x, d1);
                        d1 = fmaf(x4.y, q[j].y, d1);
                        d1 = fmaf(x4.z, q[j].z, d1);
                        d1 = fmaf(x4.w, q[j].w, d1);
                    }
                }
                if constexpr (G < NX) __builtin_amdgcn_sched_barrier(0);  // one group in flight at a time
            }
            d0 = wave_sum(d0);
            d1 = wave_sum(d1);
            // e0 = eb + wave + 16 (2 it), e1 = e0 + 16: lanes 2 it and 2 it + 1
            const int j0 = (e0 - eb - wave) / 16;
            const double b0 = lane_double(bias_l, j0), b1 = lane_double(bias_l, j0 + 1);
            if (lane == 0) {
                lg[e0] = (double)(d0 * inv) + b0;
                if (two) lg[e1] = (double)(d1 * inv) + b1;
            }
        }
    }
    if constexpr (NX > 8) write_prepared();
    __syncthreads();
    if (wave != 0) return;
    if (HASH) {
        if (lane == 0) hash_token(a.ids, t, a.E, a.k, a.chosen, a.gates, a.gates32);
        return;
    }
    if (P > 1) {
        // The hand-off rests on the hardware, not on the memory model's
        // release/acquire (which costs a write-back and an invalidation of
        // the whole L2 of the XCD): agent-scope stores and loads are
        // performed at the device's point of coherence, past the L2 of any
        // one XCD (write-through), so a store that vmcnt(0) has seen
        // acknowledged is visible to every later agent-scope load on the
        // device.  The two asm statements keep the compiler's side in order:
        // each clobbers memory, so no store moves below the wait, and no load
        // of the logits moves above the count that tells this part it is the
        // last.
        double *row = a.logits + (size_t)t * a.E;
        for (int e = eb + lane; e < ee; e += 64)
            __hip_atomic_store(row + e, lg[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stores are acknowledged
        int prior = 0;
        if (lane == 0) prior = __hip_atomic_fetch_add(a.part_cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__shfl(prior, 0) != P - 1) return;  // not the last part
        asm volatile("" ::: "memory");
        for (int e = lane; e < a.E; e += 64) lg[e] = __hip_atomic_load(row + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) __hip_atomic_store(a.part_cnt + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the logits in lg are read before a NaN row's scores overwrite them
    topk_token<EPL>(lg, t, a.E, a.k, bal, lane, a.chosen, a.gates, a.gates32, TopkScratch{lg, cand, stk});
}

bool fused_route_fits(int T, int k, int kp) { return T >= 1 && T * k <= kFusedMaxTK && T <= 1024 && kp <= 4096; }

// Parts per token: up to 128 workgroups in all, at least 32 experts per
// part, at most 8 parts; one for hash routing.  Every part repeats the
// token's combine and norm, so fewer, larger parts won: at C5 decode (T=64,
// E=64) 2 parts took 421 us of routing per step, 4 parts 438, 8 parts 592.
int route_fused_parts(int T, int E, bool hash)
{
    if (hash || T <= 0 || T > kMaxSplitRouteTokens) return 1;
    return std::max(1, std::min({(128 + T - 1) / T, E / 32, 8}));
}

template <typename InT, bool NORM, int NX>
static hipError_t launch_token_nx(const FusedArgs &fa, bool hash, hipStream_t s)
{
    FusedArgs a = fa;
    a.warm_blocks = route_warm_blocks(a.T, a.E, a.kp, a.parts, hash);
    if (hash) a.ra_blocks = 0;
    dim3 grid(a.T * a.parts + a.warm_blocks + a.ra_blocks);
    if (hash) hipLaunchKernelGGL((route_token_kernel<InT, NORM, true, 1, NX>), grid, dim3(1024), 0, s, a);
    else if (a.E <= 64) hipLaunchKernelGGL((route_token_kernel<InT, NORM, false, 1, NX>), grid, dim3(1024), 0, s, a);
    else if (a.E <= 128) hipLaunchKernelGGL((route_token_kernel<InT, NORM, false, 2, NX>), grid, dim3(1024), 0, s, a);
    else hipLaunchKernelGGL((route_token_kernel<InT, NORM, false, 4, NX>), grid, dim3(1024), 0, s, a);
    return hipGetLastError();
}

template <typename InT, bool NORM>
static hipError_t launch_token_typed(const FusedArgs &a, bool hash, hipStream_t s)
{
    if (a.kp <= 256) return launch_token_nx<InT, NORM, 1>(a, hash, s);
    if (a.kp <= 1024) return launch_token_nx<InT, NORM, 4>(a, hash, s);
    if (a.kp <= 2048) return launch_token_nx<InT, NORM, 8>(a, hash, s);
    if (a.kp <= 4096) return launch_token_nx<InT, NORM, 16>(a, hash, s);
    return hipErrorInvalidValue;
}

hipError_t launch_route_fused(const FusedArgs &a, bool input_f64, bool hash, bool dispatch, hipStream_t s)
{
    if (!fused_route_fits(a.T, a.k, a.kp)) return hipErrorInvalidValue;
    // more than one part needs the arrival counts, and a pending combine
    // then must not be written in place
    if (a.parts < 1 || (a.parts > 1 && (hash || !a.part_cnt || (a.pend_slot && (!a.x_out || a.x_out == a.x)))))
        return hipErrorInvalidValue;
    hipError_t e;
    if (input_f64) e = a.norm ? launch_token_typed<double, true>(a, hash, s) : launch_token_typed<double, false>(a, hash, s);
    else e = a.norm ? launch_token_typed<float, true>(a, hash, s) : launch_token_typed<float, false>(a, hash, s);
    if (e != hipSuccess || !dispatch) return e;
    hipLaunchKernelGGL(dispatch_kernel, dim3(1), dim3(1024), 0, s, a.chosen, a.T, a.k, a.E, a.S, a.bm, a.load,
                       a.offsets, a.rows, a.pos, a.goff, a.tok, a.tile_off, a.tile_desc, PackParts{}, nullptr);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Router backward (mixtureofexperts.go:262-282): per token, the gradient of
// each chosen gate is the output gradient dotted with that slot's expert
// output; through the gate normalisation and the affinity, the router logit
// of chosen expert e gets (gg_i - sum_j gg_j g_j) / sum_j a_j * sigmoid(l) /
// (2 a).  One wave per token; the sums over slots run in slot order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void router_backward_kernel(const double *__restrict__ og, int d,
                                                             const float *__restrict__ expert_out, int ld_out,
                                                             const int32_t *__restrict__ chosen,
                                                             const double *__restrict__ gates,
                                                             const double *__restrict__ logits,
                                                             const int32_t *__restrict__ pos, int S, int T, int E,
                                                             int k, double *__restrict__ lg, float *__restrict__ lgf)
{
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    for (int e = lane; e < E; e += 64) {
        lg[(size_t)t * E + e] = 0.0;
        lgf[(size_t)t * E + e] = 0.f;
    }
    double gg[kMaxK];
    for (int i = 0; i < k && i < kMaxK; ++i) {
        const float *row = expert_out + (size_t)(S * T + pos[(size_t)t * k + i]) * ld_out;
        double s = 0.0;
        for (int m = lane; m < d; m += 64) s += og[(size_t)t * d + m] * (double)row[m];
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
        gg[i] = s;
    }
    __syncthreads();  // the zero fill above precedes lane 0's writes
    if (lane != 0) return;
    double wsum = 0.0, atot = 0.0;
    for (int i = 0; i < k && i < kMaxK; ++i) {
        wsum += gg[i] * gates[(size_t)t * k + i];
        atot += affinity(logits[(size_t)t * E + chosen[(size_t)t * k + i]]);
    }
    for (int i = 0; i < k && i < kMaxK; ++i) {
        const int e = chosen[(size_t)t * k + i];
        const double l = logits[(size_t)t * E + e];
        const double a = affinity(l);
        const double sig = 1.0 / (1.0 + go_exp(-l));
        const double v = (gg[i] - wsum) / atot * (sig / (2.0 * a));
        lg[(size_t)t * E + e] = v;
        lgf[(size_t)t * E + e] = (float)v;
    }
}

hipError_t launch_router_backward(const double *og, int d, const float *expert_out, int ld_out,
                                  const int32_t *chosen, const double *gates, const double *logits,
                                  const int32_t *pos, int S, int T, int E, int k, double *lg, float *lgf,
                                  hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    if (k > kMaxK) return hipErrorInvalidValue;
    hipLaunchKernelGGL(router_backward_kernel, dim3(T), dim3(64), 0, s, og, d, expert_out, ld_out, chosen, gates,
                       logits, pos, S, T, E, k, lg, lgf);
    return hipGetLastError();
}

}  // namespace gtmoe
