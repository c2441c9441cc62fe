// Decode GEMV for GPTQ int4 linears, M = 1..16 rows: y[M,N] = x[M,K] * W^T (+ bias), fp32 out.
//
// Replaces the reference's gemm_gemv_f16 / gemm_gemv_split_f16 + gemm_gemv_split_reduce pair
// (src/gpu/kernels/gemm/*.wgsl, dispatched by src/model/qwen.ts:568-610), which streams fp16
// weights that the CPU dequantized at load time. Here the weights stay packed (4 bits/weight)
// and are dequantized in registers.
//
// Arithmetic (chosen so the result tracks the reference CPU path — fp32 weights, double
// accumulation — to well under 1e-4 relative):
//   y[m,n] = sum_g s[g,n] * sum_{k in g} (q[k,n] - z[g,n]) * x[m,k]
//   * (q - z) is an exact small integer in fp16 (magic-number unpack, ql_device.h);
//   * x is split into x_hi = f16(x) and x_lo = f16(x - x_hi) (x = x_hi + x_lo to ~2^-22 rel), so
//     each row m becomes two MFMA rows and products are exact in the fp32 MFMA accumulator;
//   * the per-group scale is applied in fp32 to the group's partial sums.
// The multiply-adds run on v_mfma_f32_16x16x32_f16: one MFMA consumes 4 packed rows (32 k) of
// 16 columns; each lane feeds one packed word per column, which is exactly the B-operand
// fragment (8 consecutive k of one column), so no LDS or shuffles are needed for weights.
//
// Work split: a workgroup (4 waves) owns 64 output columns and one K segment (a range of whole
// quantization groups); its waves take the segment's groups round-robin and are reduced through
// LDS in wave order. With split > 1 segments, partial sums go to scratch and the last workgroup
// of a column strip to finish (atomic arrival counter) adds them in ascending segment order —
// deterministic, like the reference's two-pass reduce (gemm_gemv_split_reduce.wgsl:32-38),
// without a second launch. The counter is reset by that workgroup, so no memset is needed.
#include "ql_device.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kTargetWaves = 4096;
constexpr int kGemvFusedMaxM = 4;          // M <= 4: activations split in the kernel prologue
constexpr int kGemvLdsXsBytes = 32768;     // LDS budget for that split (per workgroup)

// x [M,K] (f32 or f16) -> split activations in the MFMA A-operand order:
//   xs[(c * R + 2m + h)] = 8 fp16 values of row m, chunk c (k = 8c..8c+7) in perm_k order,
//   h = 0: x_hi, h = 1: x_lo;  R = 2M.
__global__ __launch_bounds__(256) void xsplit_kernel(const GemvBatch b)
{
    const GemvLinear& L = b.L[blockIdx.y];
    if (!L.xs_owner) return;
    const int M = b.M;
    const int chunks = L.K >> 3;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= chunks * M) return;
    const int c = t / M;
    const int m = t - c * M;
    float v[8];
    if (b.x_dtype == 0) {
        const float4* src = reinterpret_cast<const float4*>(
            static_cast<const float*>(L.x) + (size_t)m * L.K + (size_t)c * 8);
        const float4 a0 = src[0], a1 = src[1];
        v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
        v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    } else {
        const f16x8 h = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(
            static_cast<const uint16_t*>(L.x) + (size_t)m * L.K + (size_t)c * 8));
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)h[e];
    }
    f16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float xv = v[perm_k(e)];
        const _Float16 h = (_Float16)xv;
        hi[e] = h;
        lo[e] = (_Float16)(xv - (float)h);
    }
    uint4* dst = const_cast<uint4*>(L.xs) + (size_t)c * (2 * M) + 2 * m;
    dst[0] = __builtin_bit_cast(uint4, hi);
    dst[1] = __builtin_bit_cast(uint4, lo);
}

template <int T, int KB, bool FUSED>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(const GemvBatch b)
{
    extern __shared__ uint4 xs_lds[];     // FUSED: split activations of this K segment
    __shared__ float red[kGemvWaves][kGemvMaxM][kGemvCols];
    __shared__ uint32_t is_last;

    int wg = blockIdx.x;
    int li = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatch; i++)
        if (i < b.count && wg >= b.L[i].wg_begin) li = i;
    const GemvLinear& L = b.L[li];
    wg -= L.wg_begin;
    const int strip = wg % L.strips;
    const int seg = wg / L.strips;

    const int M = b.M;
    const int R = 2 * M;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int N = L.N;
    const int NC = (N + 7) >> 3;
    const int n = strip * kGemvCols + 4 * j;
    const bool col_ok = n < N;
    const int G = L.K / (KB * 32);
    const int g0 = (int)((int64_t)G * seg / L.split);
    const int g1 = (int)((int64_t)G * (seg + 1) / L.split);
    const int p0 = g0 * KB * 4;           // first packed row (8-k chunk) of the segment

    // software pipeline: the next group's packed words, zeros and scales are in flight while
    // the current group is converted and multiplied
    uint4 wn[KB];
    uint32_t zn = 0x77777777u;
    uint2 sn = uint2{0u, 0u};
    auto fetch = [&](int g) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
            wn[kb] = *reinterpret_cast<const uint4*>(L.qweight +
                                                     (size_t)((g * KB + kb) * 4 + kq) * N + n);
        if (L.qzeros) zn = L.qzeros[(size_t)g * NC + (n >> 3)];
        sn = *reinterpret_cast<const uint2*>(L.scales + (size_t)g * N + n);
    };
#pragma unroll
    for (int kb = 0; kb < KB; kb++) wn[kb] = uint4{0u, 0u, 0u, 0u};
    int g = g0 + wave;
    if (g < g1 && col_ok) fetch(g);

    if (FUSED) {
        // x [M,K] -> x_hi/x_lo fp16 in MFMA A-operand order, for this segment only
        const int chunks = (g1 - g0) * KB * 4;
        for (int idx = threadIdx.x; idx < chunks * M; idx += 256) {
            const int c = idx / M;
            const int m = idx - c * M;
            float v[8];
            const size_t base = (size_t)m * L.K + (size_t)(p0 + c) * 8;
            if (b.x_dtype == 0) {
                const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(L.x) + base);
                const float4 a0 = src[0], a1 = src[1];
                v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
                v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
            } else {
                const f16x8 h = __builtin_bit_cast(
                    f16x8, *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(L.x) + base));
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = (float)h[e];
            }
            f16x8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float xv = v[perm_k(e)];
                const _Float16 h = (_Float16)xv;
                hi[e] = h;
                lo[e] = (_Float16)(xv - (float)h);
            }
            xs_lds[c * R + 2 * m] = __builtin_bit_cast(uint4, hi);
            xs_lds[c * R + 2 * m + 1] = __builtin_bit_cast(uint4, lo);
        }
        __syncthreads();
    }

    f32x4 acc[4][T];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int t = 0; t < T; t++) acc[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (; g < g1; g += kGemvWaves) {
        uint4 w[KB];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) w[kb] = wn[kb];
        const uint32_t zw = L.qzeros ? (zn >> (4 * (n & 7))) : 0x7777u;
        const uint2 sv = sn;
        if (g + kGemvWaves < g1 && col_ok) fetch(g + kGemvWaves);

        uint32_t zz[4];
        float s[4];
        const uint32_t sw[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
#pragma unroll
        for (int u = 0; u < 4; u++) {
            zz[u] = zero_pair(((zw >> (4 * u)) & 15u) + 1u);
            s[u] = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
        }
        f32x4 c[4][T];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int t = 0; t < T; t++) c[u][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int p = (g * KB + kb) * 4 + kq;
            f16x8 a[T];
#pragma unroll
            for (int t = 0; t < T; t++) {
                const int row = 16 * t + j;
                if (row < R)
                    a[t] = __builtin_bit_cast(f16x8, FUSED ? xs_lds[(p - p0) * R + row]
                                                           : L.xs[(size_t)p * R + row]);
                else
                    a[t] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
            }
            const uint32_t words[4] = {w[kb].x, w[kb].y, w[kb].z, w[kb].w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const f16x8 bq = centered_nibbles(words[u], zz[u]);
#pragma unroll
                for (int t = 0; t < T; t++) c[u][t] = mfma_16x16x32_f16(a[t], bq, c[u][t]);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int t = 0; t < T; t++) acc[u][t] += s[u] * c[u][t];
    }

    // MFMA D layout: lane (j, kq) holds rows 4kq..4kq+3 of column j; rows are (m, hi/lo) pairs.
#pragma unroll
    for (int u = 0; u < 4; u++) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int m0 = 8 * t + 2 * kq;
            if (m0 < M) red[wave][m0][4 * j + u] = acc[u][t][0] + acc[u][t][1];
            if (m0 + 1 < M) red[wave][m0 + 1][4 * j + u] = acc[u][t][2] + acc[u][t][3];
        }
    }
    __syncthreads();

    const bool split = L.split > 1;
    for (int idx = threadIdx.x; idx < M * kGemvCols; idx += 256) {
        const int m = idx >> 6;
        const int col = idx & 63;
        const int nn = strip * kGemvCols + col;
        if (nn >= N) continue;
        const float sum = ((red[0][m][col] + red[1][m][col]) + red[2][m][col]) + red[3][m][col];
        if (!split) {
            L.y[(size_t)m * N + nn] = L.bias ? sum + L.bias[nn] : sum;
        } else {
            L.partial[((size_t)seg * M + m) * N + nn] = sum;
        }
    }
    if (!split) return;

    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&L.counters[strip], 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t last = prev == (uint32_t)(L.split - 1);
        if (last) __hip_atomic_store(&L.counters[strip], 0u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        is_last = last;
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    for (int idx = threadIdx.x; idx < M * kGemvCols; idx += 256) {
        const int m = idx >> 6;
        const int col = idx & 63;
        const int nn = strip * kGemvCols + col;
        if (nn >= N) continue;
        float sum = L.partial[(size_t)m * N + nn];
        for (int s2 = 1; s2 < L.split; s2++) sum += L.partial[((size_t)s2 * M + m) * N + nn];
        L.y[(size_t)m * N + nn] = L.bias ? sum + L.bias[nn] : sum;
    }
}

// Any shape, any M: one lane per output column, fp32 weights (exact), fp32 accumulation.
// round_f16 = 1 gives the GEMM semantics instead: x and W rounded to fp16 (RNE) first.
__global__ __launch_bounds__(256) void linear_simple_kernel(GemvLinear L, int M, int x_dtype,
                                                            int round_f16)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int m0 = blockIdx.y * 8;
    if (n >= L.N) return;
    const int K = L.K;
    const int NC = (L.N + 7) >> 3;
    const int mc = min(8, M - m0);
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.f;
    const int P = (K + 7) >> 3;
    for (int p = 0; p < P; p++) {
        const int g = (p * 8) / L.group;
        const uint32_t word = L.qweight[(size_t)p * L.N + n];
        const int z = (int)zero_of(L.qzeros, g, NC, n);
        const float s = (float)__builtin_bit_cast(_Float16, L.scales[(size_t)g * L.N + n]);
        for (int kk = 0; kk < 8; kk++) {
            const int i = p * 8 + kk;
            if (i >= K) break;
            float w = (float)((int)((word >> (4 * kk)) & 15u) - z) * s;
            if (round_f16) w = (float)(_Float16)w;
#pragma unroll
            for (int mm = 0; mm < 8; mm++) {
                if (mm < mc) {
                    const size_t xi = (size_t)(m0 + mm) * K + i;
                    float xv = x_dtype == 0 ? static_cast<const float*>(L.x)[xi]
                                            : (float)__builtin_bit_cast(
                                                  _Float16, static_cast<const uint16_t*>(L.x)[xi]);
                    if (round_f16) xv = (float)(_Float16)xv;
                    acc[mm] += xv * w;
                }
            }
        }
    }
    for (int mm = 0; mm < mc; mm++) {
        const float v = acc[mm];
        L.y[(size_t)(m0 + mm) * L.N + n] = L.bias ? v + L.bias[n] : v;
    }
}

template <int T, bool FUSED>
hipError_t launch_tiles(const GemvBatch& b, int kb, size_t lds, hipStream_t stream)
{
    dim3 grid(b.wg_total), block(256);
    switch (kb) {
    case 1: hipLaunchKernelGGL((gemv_mfma_kernel<T, 1, FUSED>), grid, block, lds, stream, b); break;
    case 2: hipLaunchKernelGGL((gemv_mfma_kernel<T, 2, FUSED>), grid, block, lds, stream, b); break;
    case 4: hipLaunchKernelGGL((gemv_mfma_kernel<T, 4, FUSED>), grid, block, lds, stream, b); break;
    case 8: hipLaunchKernelGGL((gemv_mfma_kernel<T, 8, FUSED>), grid, block, lds, stream, b); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool gemv_fast_ok(int M, int N, int K, int group)
{
    return M >= 1 && M <= kGemvMaxM && N > 0 && K > 0 && N % 4 == 0 &&
           (group == 32 || group == 64 || group == 128 || group == 256) && K % group == 0;
}

bool gemv_fused(int M) { return M <= kGemvFusedMaxM; }

GemvShape gemv_shape(int M, int N, int K, int group)
{
    GemvShape s;
    s.strips = (N + kGemvCols - 1) / kGemvCols;
    s.groups = K / group;
    int slices = (kTargetWaves + s.strips - 1) / s.strips;   // K slices wanted per strip
    if (slices > s.groups) slices = s.groups;
    if (slices < 1) slices = 1;
    s.waves = kGemvWaves;
    s.split = (slices + kGemvWaves - 1) / kGemvWaves;
    if (gemv_fused(M)) {
        // the segment's split activations must fit the LDS budget: 2M rows x group/8 chunks x 16 B
        int max_groups = kGemvLdsXsBytes / (4 * M * group);
        if (max_groups < 1) max_groups = 1;
        const int need = (s.groups + max_groups - 1) / max_groups;
        if (s.split < need) s.split = need;
    }
    if (s.split > s.groups) s.split = s.groups;
    if (s.split < 1) s.split = 1;
    return s;
}

uint64_t gemv_xs_bytes(int M, int K)
{
    if (gemv_fused(M)) return 0;
    return ((uint64_t)4 * M * K + 255) & ~(uint64_t)255;
}

uint64_t gemv_partial_bytes(int M, int N, int split)
{
    if (split <= 1) return 0;
    return ((uint64_t)split * M * N * 4 + 255) & ~(uint64_t)255;
}

hipError_t launch_gemv_batch(const GemvBatch& b, hipStream_t stream)
{
    const int group = b.L[0].group;
    for (int i = 1; i < b.count; i++)
        if (b.L[i].group != group) return hipErrorInvalidValue;
    const int kb = group / 32;
    if (gemv_fused(b.M)) {
        size_t lds = 0;
        for (int i = 0; i < b.count; i++) {
            const int G = b.L[i].K / group;
            const int gmax = (G + b.L[i].split - 1) / b.L[i].split;
            lds = max(lds, (size_t)gmax * kb * 4 * (2 * b.M) * 16);
        }
        return launch_tiles<1, true>(b, kb, lds, stream);
    }
    int max_chunks = 0;
    for (int i = 0; i < b.count; i++)
        if (b.L[i].xs_owner) max_chunks = max(max_chunks, (b.L[i].K >> 3) * b.M);
    dim3 xgrid((max_chunks + 255) / 256, b.count);
    hipLaunchKernelGGL(xsplit_kernel, xgrid, dim3(256), 0, stream, b);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return b.M <= 8 ? launch_tiles<1, false>(b, kb, 0, stream)
                    : launch_tiles<2, false>(b, kb, 0, stream);
}

hipError_t launch_gemv_simple(const GemvLinear& L, int M, int x_dtype, hipStream_t stream)
{
    dim3 grid((L.N + 255) / 256, (M + 7) / 8);
    hipLaunchKernelGGL(linear_simple_kernel, grid, dim3(256), 0, stream, L, M, x_dtype, 0);
    return hipGetLastError();
}

hipError_t launch_gemm_simple(const GemmArgs& a, hipStream_t stream)
{
    GemvLinear L{};
    L.qweight = a.qweight; L.qzeros = a.qzeros; L.scales = a.scales; L.bias = a.bias;
    L.x = a.x; L.y = a.y; L.N = a.N; L.K = a.K; L.group = a.group;
    dim3 grid((a.N + 255) / 256, (a.M + 7) / 8);
    hipLaunchKernelGGL(linear_simple_kernel, grid, dim3(256), 0, stream, L, a.M, a.x_dtype, 1);
    return hipGetLastError();
}

}  // namespace ql
