// Input preparation, RMSNorm, the weighted combine, and small fills.
#include <algorithm>

#include "kernels.h"

namespace gtmoe {

namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Four floats as bf16 (nearest even), packed in 8 bytes.
__device__ __forceinline__ uint2 to_bf16x4(float a, float b, float c, float d)
{
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2)),
                      __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){c, d}, bf16x2)));
}

// Four consecutive values of a row (zeros past d); rows with d % 4 == 0
// are read with vector loads.
__device__ __forceinline__ void load_row4(const float *row, int j, int d, bool vec, float (&v)[4])
{
    if (vec && j < d) {
        const float4 q = *reinterpret_cast<const float4 *>(row + j);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = j + i < d ? row[j + i] : 0.f;
    }
}
__device__ __forceinline__ void load_row4(const double *row, int j, int d, bool vec, float (&v)[4])
{
    if (vec && j < d) {
        const double2 a = *reinterpret_cast<const double2 *>(row + j);
        const double2 b = *reinterpret_cast<const double2 *>(row + j + 2);
        v[0] = (float)a.x;
        v[1] = (float)a.y;
        v[2] = (float)b.x;
        v[3] = (float)b.y;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = j + i < d ? (float)row[j + i] : 0.f;
    }
}

__device__ __forceinline__ void store_row4(float *xf, uint16_t *xb, size_t of, size_t ob, const float (&v)[4])
{
    if (xf) *reinterpret_cast<float4 *>(xf + of) = make_float4(v[0], v[1], v[2], v[3]);
    if (xb) *reinterpret_cast<uint2 *>(xb + ob) = to_bf16x4(v[0], v[1], v[2], v[3]);
}

}  // namespace

// One row per workgroup: padded fp32 copy (ldf columns, zeros past d) and/or
// padded bf16 copy.  Either output may be null; ldf and ldb are multiples of
// 64.  Each thread handles four consecutive columns per step.
template <typename InT>
__global__ __launch_bounds__(256) void convert_inputs_kernel(const InT *__restrict__ x, int d, float *__restrict__ xf,
                                                             int ldf, uint16_t *__restrict__ xb, int ldb)
{
    const int t = blockIdx.x;
    const int ld = xf ? ldf : ldb;
    const InT *row = x + (size_t)t * d;
    const bool vec = (d & 3) == 0;
    for (int j = threadIdx.x * 4; j < ld; j += 1024) {
        float v[4];
        load_row4(row, j, d, vec, v);
        store_row4(xf, xb, (size_t)t * ldf + j, (size_t)t * ldb + j, v);
    }
}

hipError_t launch_convert_inputs_f64(const double *x, int T, int d, float *xf, int ldf, uint16_t *xb, int ldb,
                                     hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(convert_inputs_kernel<double>, dim3(T), dim3(256), 0, s, x, d, xf, ldf, xb, ldb);
    return hipGetLastError();
}

hipError_t launch_convert_inputs_f32(const float *x, int T, int d, float *xf, int ldf, uint16_t *xb, int ldb,
                                     hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(convert_inputs_kernel<float>, dim3(T), dim3(256), 0, s, x, d, xf, ldf, xb, ldb);
    return hipGetLastError();
}

// RMSNorm (normalization/rmsnorm.go:33-53): y = x / sqrt(mean(x^2) + 1e-6) * w,
// one row per workgroup, written padded as fp32 and/or bf16.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, int d, const float *__restrict__ w,
                                                      float *__restrict__ xf, int ldf, uint16_t *__restrict__ xb,
                                                      int ldb)
{
    __shared__ float partial[4];
    const int t = blockIdx.x;
    const float *row = x + (size_t)t * d;
    const bool vec = (d & 3) == 0;
    float ss = 0.f;
    for (int j = threadIdx.x * 4; j < d; j += 1024) {
        float v[4];
        load_row4(row, j, d, vec, v);
#pragma unroll
        for (int i = 0; i < 4; ++i) ss = fmaf(v[i], v[i], ss);
    }
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = partial[0] + partial[1] + partial[2] + partial[3];
    const float inv = 1.0f / sqrtf(total / (float)d + 1e-6f);
    const int ld = xf ? ldf : ldb;
    for (int j = threadIdx.x * 4; j < ld; j += 1024) {
        float v[4], g[4];
        load_row4(row, j, d, vec, v);
        load_row4(w, j, d, vec, g);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = v[i] * inv * g[i];
        store_row4(xf, xb, (size_t)t * ldf + j, (size_t)t * ldb + j, v);
    }
}

hipError_t launch_rmsnorm(const float *x, int T, int d, const float *w, float *xf, int ldf, uint16_t *xb, int ldb,
                          hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, s, x, d, w, xf, ldf, xb, ldb);
    return hipGetLastError();
}

// Slot rows are fp32 (fp32 path) or bf16 (MFMA path); C consecutive values
// of a row as floats (C = 4: one 16-byte load of fp32, C = 8: one of bf16).
template <int C>
__device__ __forceinline__ void loadC(const float *p, float (&v)[C])
{
#pragma unroll
    for (int q = 0; q < C; q += 4) {
        const float4 f = *reinterpret_cast<const float4 *>(p + q);
        v[q] = f.x;
        v[q + 1] = f.y;
        v[q + 2] = f.z;
        v[q + 3] = f.w;
    }
}
template <int C>
__device__ __forceinline__ void loadC(const uint16_t *p, float (&v)[C])
{
#pragma unroll
    for (int q = 0; q < C; q += 8) {
        const uint4 u = *reinterpret_cast<const uint4 *>(p + q);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[q + 2 * i] = __uint_as_float(w[i] << 16);
            v[q + 2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}
__device__ __forceinline__ float load1(const float *p) { return *p; }
__device__ __forceinline__ float load1(const uint16_t *p) { return __uint_as_float((uint32_t)*p << 16); }

// Weighted combine (mixtureofexperts.go:182-205) in the reference's order:
// out = 0, + each shared expert's row, then + gate_i * routed row for the
// slots in chosen order.  Routed slot rows are found through the dispatch's
// pos table, or, with pos == nullptr, at S*T + t*k + i (rows indexed by
// (token, slot), as the self-dispatching decode kernels write them).  With a residual: out = residual + that sum
// (transformer/block.go:77).  Writes fp32 and/or float64 output.  Grid
// (T, ceil(d / 1024)); each thread owns four consecutive columns.
// Each thread owns C consecutive columns (C = 4 for fp32 slot rows, 8 for
// bf16: 16-byte loads); the routed rows (KB >= k of them, rows past k re-read
// row 0 and are not added) are requested before the adds, which keep the
// reference's order.  vec_io: residual and outputs are 16-byte aligned.
//
// With norm.w set (a stack whose next layer takes bf16 rows; the row fits
// one workgroup, d <= 256 C, and its stride is d): the next layer's RMSNorm
// (normalization/rmsnorm.go:33-53) is done here on the new row, which the
// workgroup holds whole -- its bf16 normalised row and its inverse RMS are
// written, so the next layer needs no pass of its own over the residual.
template <typename SlotT, int KB>
__global__ __launch_bounds__(256) void combine_kernel(int T, int d, int S, int k, const SlotT *__restrict__ slot_out,
                                                      const int32_t *__restrict__ pos,
                                                      const float *__restrict__ gates32,
                                                      const float *__restrict__ residual, float *__restrict__ out32,
                                                      double *__restrict__ out64, bool vec_io, CombineNorm norm)
{
    constexpr int C = sizeof(SlotT) == 2 ? 8 : 4;
    __shared__ float partial[4];
    const int t = blockIdx.x;
    if (norm.w) {
        // one row per workgroup: every thread takes part in the reduction
        const int j0 = threadIdx.x * C;
        const bool mine = j0 < d;
        float acc[C];
#pragma unroll
        for (int q = 0; q < C; ++q) acc[q] = 0.f;
        if (mine) {
            int p[KB];
            float g[KB];
#pragma unroll
            for (int i = 0; i < KB; ++i) {
                const int ii = i < k ? i : 0;
                p[i] = S * T + (pos ? pos[(size_t)t * k + ii] : t * k + ii);
                g[i] = gates32[(size_t)t * k + ii];
            }
            float v[KB][C];
#pragma unroll
            for (int i = 0; i < KB; ++i) loadC<C>(slot_out + (size_t)p[i] * d + j0, v[i]);
            for (int s = 0; s < S; ++s) {
                float u[C];
                loadC<C>(slot_out + ((size_t)s * T + t) * d + j0, u);
#pragma unroll
                for (int q = 0; q < C; ++q) acc[q] += u[q];
            }
#pragma unroll
            for (int i = 0; i < KB; ++i)
                if (i < k)
#pragma unroll
                    for (int q = 0; q < C; ++q) acc[q] = fmaf(g[i], v[i][q], acc[q]);
            const size_t o = (size_t)t * d + j0;
            float r[C];
            loadC<C>(residual + o, r);
#pragma unroll
            for (int q = 0; q < C; ++q) acc[q] = r[q] + acc[q];
#pragma unroll
            for (int q = 0; q < C; q += 4)
                *reinterpret_cast<float4 *>(out32 + o + q) = make_float4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3]);
        }
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < C; ++q) ss = fmaf(acc[q], acc[q], ss);
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float total = partial[0] + partial[1] + partial[2] + partial[3];
        const float inv = 1.0f / sqrtf(total / (float)d + 1e-6f);
        if (threadIdx.x == 0) norm.inv[t] = inv;
        if (mine) {
            float w[C];
            loadC<C>(norm.w + j0, w);
#pragma unroll
            for (int q = 0; q < C; q += 4)
                *reinterpret_cast<uint2 *>(norm.xb + (size_t)t * norm.ldb + j0 + q) =
                    to_bf16x4(acc[q] * inv * w[q], acc[q + 1] * inv * w[q + 1], acc[q + 2] * inv * w[q + 2],
                              acc[q + 3] * inv * w[q + 3]);
        }
        return;
    }
    const int j0 = (blockIdx.y * 256 + threadIdx.x) * C;
    if (j0 >= d) return;
    int p[KB];
    float g[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        const int ii = i < k ? i : 0;
        p[i] = S * T + (pos ? pos[(size_t)t * k + ii] : t * k + ii);
        g[i] = gates32[(size_t)t * k + ii];
    }
    const int n = min(C, d - j0);
    float acc[C];
#pragma unroll
    for (int q = 0; q < C; ++q) acc[q] = 0.f;
    if (n == C && d % C == 0 && vec_io) {
        float v[KB][C];
#pragma unroll
        for (int i = 0; i < KB; ++i) loadC<C>(slot_out + (size_t)p[i] * d + j0, v[i]);
        for (int s = 0; s < S; ++s) {
            float u[C];
            loadC<C>(slot_out + ((size_t)s * T + t) * d + j0, u);
#pragma unroll
            for (int q = 0; q < C; ++q) acc[q] += u[q];
        }
#pragma unroll
        for (int i = 0; i < KB; ++i)
            if (i < k)
#pragma unroll
                for (int q = 0; q < C; ++q) acc[q] = fmaf(g[i], v[i][q], acc[q]);
        const size_t o = (size_t)t * d + j0;
        if (residual) {
            float r[C];
            loadC<C>(residual + o, r);
#pragma unroll
            for (int q = 0; q < C; ++q) acc[q] = r[q] + acc[q];
        }
        if (out32)
#pragma unroll
            for (int q = 0; q < C; q += 4)
                *reinterpret_cast<float4 *>(out32 + o + q) = make_float4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3]);
        if (out64)
#pragma unroll
            for (int q = 0; q < C; q += 2)
                *reinterpret_cast<double2 *>(out64 + o + q) = make_double2((double)acc[q], (double)acc[q + 1]);
        return;
    }
    for (int q = 0; q < n; ++q) {
        for (int s = 0; s < S; ++s) acc[q] += load1(slot_out + ((size_t)s * T + t) * d + j0 + q);
#pragma unroll
        for (int i = 0; i < KB; ++i)
            if (i < k) acc[q] = fmaf(g[i], load1(slot_out + (size_t)p[i] * d + j0 + q), acc[q]);
    }
    for (int q = 0; q < n; ++q) {
        const size_t o = (size_t)t * d + j0 + q;
        float v = acc[q];
        if (residual) v = residual[o] + v;
        if (out32) out32[o] = v;
        if (out64) out64[o] = (double)v;
    }
}

bool combine_norm_fits(int d, bool slot_bf16) { return slot_bf16 && d % 8 == 0 && d <= 2048; }

hipError_t launch_combine(int T, int d, int S, int k, const void *slot_out, bool slot_bf16, const int32_t *pos,
                          const float *gates32, const float *residual, float *out32, double *out64, hipStream_t s,
                          const CombineNorm &norm)
{
    if (T <= 0) return hipSuccess;
    if (k < 1 || k > 8) return hipErrorInvalidValue;
    auto aligned = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool vec_io = aligned(residual) && aligned(out32) && aligned(out64);  // null counts as aligned
    if (norm.w && (!combine_norm_fits(d, slot_bf16) || !residual || !out32 || out64 || !vec_io || !norm.xb ||
                   !norm.inv || norm.ldb < d || norm.ldb % 8 != 0 || !aligned(norm.xb) || !aligned(norm.w)))
        return hipErrorInvalidValue;
    auto go = [&](auto kb_tag) {
        constexpr int KB = decltype(kb_tag)::value;
        if (slot_bf16)
            hipLaunchKernelGGL((combine_kernel<uint16_t, KB>), dim3(T, (d + 2047) / 2048), dim3(256), 0, s, T, d, S,
                               k, static_cast<const uint16_t *>(slot_out), pos, gates32, residual, out32, out64,
                               vec_io, norm);
        else
            hipLaunchKernelGGL((combine_kernel<float, KB>), dim3(T, (d + 1023) / 1024), dim3(256), 0, s, T, d, S, k,
                               static_cast<const float *>(slot_out), pos, gates32, residual, out32, out64, vec_io,
                               norm);
    };
    if (k <= 2) go(std::integral_constant<int, 2>{});
    else if (k <= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
    return hipGetLastError();
}

__global__ void f32_to_f64_kernel(const float *__restrict__ x, double *__restrict__ y, long long n)
{
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (double)x[i];
}

hipError_t launch_f32_to_f64(const float *x, double *y, long long n, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(f32_to_f64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

__global__ void fill_i32_kernel(int32_t *p, int n, int32_t v)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

hipError_t launch_fill_i32(int32_t *p, int n, int32_t v, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((n + 255) / 256), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

// The routing state a host-API forward hands back, gathered into one block
// (of pinned host memory, written across the bus by this kernel): the 4-byte
// words of each part one after the other, every part starting at a multiple
// of 16 words.
__global__ __launch_bounds__(256) void pack_words_kernel(PackParts p, uint32_t *__restrict__ dst)
{
    uint32_t *out = dst;
    for (int i = 0; i < PackParts::kMax; ++i) {
        if (i >= p.n) break;
        const uint32_t *src = p.src[i];
        for (int j = blockIdx.x * 256 + threadIdx.x; j < p.words[i]; j += gridDim.x * 256) out[j] = src[j];
        out += (p.words[i] + 15) / 16 * 16;
    }
}

hipError_t launch_pack_words(const PackParts &p, uint32_t *dst, hipStream_t s)
{
    if (p.n < 0 || p.n > PackParts::kMax) return hipErrorInvalidValue;
    long long most = 0;
    for (int i = 0; i < p.n; ++i) most = std::max<long long>(most, p.words[i]);
    const int blocks = (int)std::min<long long>(64, std::max<long long>(1, (most + 255) / 256));
    hipLaunchKernelGGL(pack_words_kernel, dim3(blocks), dim3(256), 0, s, p, dst);
    return hipGetLastError();
}

}  // namespace gtmoe
