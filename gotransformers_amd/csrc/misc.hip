// Input preparation, RMSNorm, the weighted combine, and small fills.
#include "common.h"

namespace gtmoe {

namespace {

// float -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

}  // namespace

// One row per workgroup: padded fp32 copy (ldf columns, zeros past d) and/or
// padded bf16 copy.  Either output may be null.
template <typename InT>
__global__ __launch_bounds__(256) void convert_inputs_kernel(const InT *__restrict__ x, int d, float *__restrict__ xf,
                                                             int ldf, uint16_t *__restrict__ xb, int ldb)
{
    const int t = blockIdx.x;
    const int ld = xf ? ldf : ldb;
    for (int j = threadIdx.x; j < ld; j += blockDim.x) {
        const float v = j < d ? (float)x[(size_t)t * d + j] : 0.f;
        if (xf) xf[(size_t)t * ldf + j] = v;
        if (xb) xb[(size_t)t * ldb + j] = to_bf16(v);
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
    float ss = 0.f;
    for (int j = threadIdx.x; j < d; j += 256) ss = fmaf(row[j], row[j], ss);
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = partial[0] + partial[1] + partial[2] + partial[3];
    const float inv = 1.0f / sqrtf(total / (float)d + 1e-6f);
    const int ld = xf ? ldf : ldb;
    for (int j = threadIdx.x; j < ld; j += 256) {
        const float v = j < d ? row[j] * inv * w[j] : 0.f;
        if (xf) xf[(size_t)t * ldf + j] = v;
        if (xb) xb[(size_t)t * ldb + j] = to_bf16(v);
    }
}

hipError_t launch_rmsnorm(const float *x, int T, int d, const float *w, float *xf, int ldf, uint16_t *xb, int ldb,
                          hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, s, x, d, w, xf, ldf, xb, ldb);
    return hipGetLastError();
}

// Weighted combine (mixtureofexperts.go:182-205) in the reference's order:
// out = 0, + each shared expert's row, then + gate_i * routed row for the
// slots in chosen order.  With a residual: out = residual + that sum
// (transformer/block.go:77).  Writes fp32 and/or float64 output.  Grid
// (T, ceil(d / 1024)); each thread owns four consecutive columns.
__global__ __launch_bounds__(256) void combine_kernel(int T, int d, int S, int k, const float *__restrict__ slot_out,
                                                      const int32_t *__restrict__ pos,
                                                      const float *__restrict__ gates32,
                                                      const float *__restrict__ residual, float *__restrict__ out32,
                                                      double *__restrict__ out64)
{
    const int t = blockIdx.x;
    const int j0 = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (j0 >= d) return;
    int p[8];
    float g[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        p[i] = i < k ? S * T + pos[(size_t)t * k + i] : 0;
        g[i] = i < k ? gates32[(size_t)t * k + i] : 0.f;
    }
    const int n = min(4, d - j0);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (n == 4 && (d & 3) == 0) {
        for (int s = 0; s < S; ++s) {
            const float4 v = *reinterpret_cast<const float4 *>(slot_out + ((size_t)s * T + t) * d + j0);
            acc[0] += v.x;
            acc[1] += v.y;
            acc[2] += v.z;
            acc[3] += v.w;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i < k) {
                const float4 v = *reinterpret_cast<const float4 *>(slot_out + (size_t)p[i] * d + j0);
                acc[0] = fmaf(g[i], v.x, acc[0]);
                acc[1] = fmaf(g[i], v.y, acc[1]);
                acc[2] = fmaf(g[i], v.z, acc[2]);
                acc[3] = fmaf(g[i], v.w, acc[3]);
            }
    } else {
        for (int q = 0; q < n; ++q) {
            for (int s = 0; s < S; ++s) acc[q] += slot_out[((size_t)s * T + t) * d + j0 + q];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (i < k) acc[q] = fmaf(g[i], slot_out[(size_t)p[i] * d + j0 + q], acc[q]);
        }
    }
    for (int q = 0; q < n; ++q) {
        const size_t o = (size_t)t * d + j0 + q;
        float v = acc[q];
        if (residual) v = residual[o] + v;
        if (out32) out32[o] = v;
        if (out64) out64[o] = (double)v;
    }
}

hipError_t launch_combine(int T, int d, int S, int k, const float *slot_out, const int32_t *pos, const float *gates32,
                          const float *residual, float *out32, double *out64, hipStream_t s)
{
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(combine_kernel, dim3(T, (d + 1023) / 1024), dim3(256), 0, s, T, d, S, k, slot_out, pos, gates32,
                       residual, out32, out64);
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

}  // namespace gtmoe
