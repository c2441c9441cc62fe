// The elementwise work around the decode linears (reference: src/model/qwen.ts:401-405,
// :447-478; src/gpu/kernels/norm/rmsnorm.wgsl, activation/silu_mul.wgsl, misc/vec_add.wgsl),
// fused where the reference runs two launches with a pass break between them:
//
//   add_rmsnorm_kernel  s = x + d (the residual add after o / down), optionally stored as the new
//                       residual stream, then y = s * rstd * w with rstd = 1 / sqrt(mean(s^2) + eps)
//                       (the RMSNorm in front of q/k/v, gate/up or lm_head); without d it is the
//                       plain RMSNorm. One workgroup per row; the row's sum of squares is added
//                       per thread, then per wave (butterfly), then over the 4 waves in order.
//                       Rows up to 4096 values stay in registers (one read of x, d and w); longer
//                       rows read the stored sum (or x and d) a second time for the output. The
//                       sum may be stored in place over x or d (the residual stream updated in
//                       place): every thread reads back only what it wrote.
//   silu_mul_kernel     y = (g / (1 + exp(-g))) * u, four values per thread.
//
// Both are HBM-bound streams (bytes per row: x, d, s and y once; per element of silu_mul: g, u, y).
#include <cmath>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kKeep = 4;     // 16-byte pieces of a row kept per thread: rows up to 4096 values

__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const ElemArgs a)
{
    __shared__ float red[4];
    const int row = blockIdx.x, C = a.C;
    const float* x = a.x + (size_t)row * C;
    const float* d = a.d ? a.d + (size_t)row * C : nullptr;
    float* s_out = a.s ? a.s + (size_t)row * C : nullptr;
    float* y = a.y + (size_t)row * C;
    float ss = 0.f;
    if (a.vec && C <= 4 * 256 * kKeep) {
        // one pass over HBM: the row (and the weight) stay in registers across the reduction
        f32x4 v[kKeep], g[kKeep];
#pragma unroll
        for (int k = 0; k < kKeep; k++) {
            const int i = threadIdx.x + 256 * k;
            if (i < C / 4) {
                v[k] = ld_global(reinterpret_cast<const f32x4*>(x) + i);
                g[k] = ld_global(reinterpret_cast<const f32x4*>(a.w) + i);
                if (d) {
                    const f32x4 e = ld_global(reinterpret_cast<const f32x4*>(d) + i);
                    v[k] = f32x4{v[k].x + e.x, v[k].y + e.y, v[k].z + e.z, v[k].w + e.w};
                    if (s_out) st_global(reinterpret_cast<f32x4*>(s_out) + i, v[k]);
                }
                ss = fmaf(v[k].x, v[k].x, ss);
                ss = fmaf(v[k].y, v[k].y, ss);
                ss = fmaf(v[k].z, v[k].z, ss);
                ss = fmaf(v[k].w, v[k].w, ss);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float rstd = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)C + a.eps);
#pragma unroll
        for (int k = 0; k < kKeep; k++) {
            const int i = threadIdx.x + 256 * k;
            if (i < C / 4)
                st_global(reinterpret_cast<f32x4*>(y) + i, f32x4{v[k].x * rstd * g[k].x, v[k].y * rstd * g[k].y,
                                                                 v[k].z * rstd * g[k].z, v[k].w * rstd * g[k].w});
        }
        return;
    }
    if (a.vec) {
        for (int i = threadIdx.x; i < C / 4; i += 256) {
            f32x4 v = ld_global(reinterpret_cast<const f32x4*>(x) + i);
            if (d) {
                const f32x4 w = ld_global(reinterpret_cast<const f32x4*>(d) + i);
                v = f32x4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
                if (s_out) st_global(reinterpret_cast<f32x4*>(s_out) + i, v);
            }
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
    } else {
        for (int i = threadIdx.x; i < C; i += 256) {
            float v = x[i];
            if (d) {
                v = v + d[i];
                if (s_out) s_out[i] = v;
            }
            ss = fmaf(v, v, ss);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    const float rstd = 1.0f / sqrtf(total / (float)C + a.eps);
    // second pass: the stored sum (each thread reads back exactly the elements it wrote, so an
    // in-place sum over x or d is read correctly), else x and d again (L2-resident: this
    // workgroup just read them)
    if (a.vec) {
        for (int i = threadIdx.x; i < C / 4; i += 256) {
            f32x4 v;
            if (s_out) {
                v = ld_global(reinterpret_cast<const f32x4*>(s_out) + i);
            } else {
                v = ld_global(reinterpret_cast<const f32x4*>(x) + i);
                if (d) {
                    const f32x4 w = ld_global(reinterpret_cast<const f32x4*>(d) + i);
                    v = f32x4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
                }
            }
            const f32x4 g = ld_global(reinterpret_cast<const f32x4*>(a.w) + i);
            st_global(reinterpret_cast<f32x4*>(y) + i,
                      f32x4{v.x * rstd * g.x, v.y * rstd * g.y, v.z * rstd * g.z, v.w * rstd * g.w});
        }
    } else {
        for (int i = threadIdx.x; i < C; i += 256) {
            float v;
            if (s_out) {
                v = s_out[i];
            } else {
                v = x[i];
                if (d) v = v + d[i];
            }
            y[i] = v * rstd * a.w[i];
        }
    }
}

__device__ __forceinline__ float silu_mul1(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

__global__ __launch_bounds__(256) void silu_mul_kernel(const float* gate, const float* up, float* y, long long n)
{
    const long long i4 = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long n4 = n / 4;
    if (i4 < n4) {
        const f32x4 g = ld_global(reinterpret_cast<const f32x4*>(gate) + i4);
        const f32x4 u = ld_global(reinterpret_cast<const f32x4*>(up) + i4);
        st_global(reinterpret_cast<f32x4*>(y) + i4,
                  f32x4{silu_mul1(g.x, u.x), silu_mul1(g.y, u.y), silu_mul1(g.z, u.z), silu_mul1(g.w, u.w)});
    } else if (i4 - n4 < n - 4 * n4) {
        const long long i = 4 * n4 + (i4 - n4);              // the tail (n % 4 values)
        y[i] = silu_mul1(gate[i], up[i]);
    }
}

}  // namespace

hipError_t launch_add_rmsnorm(const ElemArgs& a, hipStream_t stream)
{
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(a.M), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* gate, const float* up, float* y, long long n, hipStream_t stream)
{
    const long long threads = n / 4 + (n % 4);
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, gate, up, y, n);
    return hipGetLastError();
}

}  // namespace ql
