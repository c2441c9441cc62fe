// Decode GEMV for GPTQ int4 linears, M = 1..16 rows: y[M,N] = x[M,K] * W^T (+ bias), fp32 out.
//
// Replaces the reference's gemm_gemv_f16 / gemm_gemv_split_f16 + gemm_gemv_split_reduce pair
// (src/gpu/kernels/gemm/*.wgsl, dispatched by src/model/qwen.ts:568-610), which streams fp16
// weights that the CPU dequantized at load time. Here the weights stay packed (4 bits/weight)
// and are unpacked in registers; the multiply-adds run on MFMA.
//
// Arithmetic (tracks the reference CPU path — fp32 weights, double accumulation — to ~1e-6):
//   y[m,n] = sum_g s[g,n] * ( sum_{k in g} q[k,n] * x[m,k]  -  z[g,n] * Sx[g,m] ),
//   Sx[g,m] = sum_{k in g} x[m,k]   (fp32, fixed order).
// * q is taken straight from the packed word by shifting and masking: a nibble at bits 4-7 of a
//   16-bit half is an exact fp16 subnormal q * 2^-20 (7 integer ops per packed word of 8
//   weights, no conversions). Bits 4-7 and not 0-3: MFMA products with operands at the bottom of
//   the subnormal range (q * 2^-24) were measured to lose ~1e-6 relative accuracy, bits 4-7 none.
// * x is scaled per (row, group) by a power of two 2^E (range normalisation:
//   max_{k in g} |x| * 2^E * 16 < 2^15), times the factor 16 matching the nibble position; the
//   scaled value a is split into a_hi = f16(a), a_lo = f16(a - a_hi), so each row m becomes two
//   MFMA rows and every product is exact in the fp32 accumulator. The group's products carry
//   2^(E-16), removed with the group scale in the group epilogue. 16 lanes own one group of one
//   row: max, exponent, split and group sum are one pass with 16-lane butterflies.
// One v_mfma_f32_16x16x32_f16 consumes 4 packed rows (32 k) of 16 columns: each lane feeds one
// packed word of one column, which is exactly the B-operand fragment (8 k of one column).
//
// Work split: a workgroup (4 waves) owns 64 output columns and one K segment (a range of whole
// quantization groups); its waves take the segment's groups round-robin and are reduced through
// LDS in wave order. With split > 1 segments, each workgroup stores its partial sums with
// agent-scope (cross-XCD coherent) stores and bumps a per-strip arrival counter; the last one
// adds the partials in ascending segment order — deterministic, like the reference's two-pass
// reduce (gemm_gemv_split_reduce.wgsl:32-38), in one launch — and resets the counter.
// Agent-scope *fences* are avoided on purpose: on this part they write back and invalidate the
// whole L2, which was measured to cost more than the GEMV itself.
#include "ql_device.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kTargetWaves = 4096;
constexpr int kGemvFusedMaxM = 4;          // M <= 4: activations prepared in the kernel prologue
constexpr int kGemvLdsXsBytes = 32768;     // LDS budget for them (per workgroup)

// Factor folded into the activations: every nibble arrives as q * 2^-20.
constexpr float kActScale = 16.f;

// Exponent E with max|x| * 2^E * 16 < 2^15 (E = 0 when all values are zero).
__device__ __forceinline__ int row_exponent(float amax)
{
    if (!(amax > 0.f)) return 0;
    int ex;
    (void)frexpf(amax, &ex);                 // amax < 2^ex
    int E = 11 - ex;
    return E < -100 ? -100 : (E > 100 ? 100 : E);
}

__device__ __forceinline__ void load8(const void* x, int x_dtype, size_t base, float v[8])
{
    if (x_dtype == 0) {
        const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base);
        const float4 a0 = src[0], a1 = src[1];
        v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
        v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    } else {
        const f16x8 h = __builtin_bit_cast(
            f16x8, *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base));
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)h[e];
    }
}

// 8 activations (natural k order) -> scaled hi/lo fp16 fragments in perm_k slot order.
__device__ __forceinline__ void split8(const float v[8], float scale, uint4* hi_out, uint4* lo_out)
{
    f16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float a = v[perm_k(e)] * (scale * kActScale);
        const _Float16 h = (_Float16)a;
        hi[e] = h;
        lo[e] = (_Float16)(a - (float)h);
    }
    *hi_out = __builtin_bit_cast(uint4, hi);
    *lo_out = __builtin_bit_cast(uint4, lo);
}

// 8 nibbles of a packed word as exact fp16 subnormals q * 2^-20, in perm_k slot order.
__device__ __forceinline__ f16x8 nibbles_subnormal(uint32_t w)
{
    const uint32_t p0 = (w << 4) & 0x00F000F0u;   // k0, k4
    const uint32_t p1 = w & 0x00F000F0u;          // k1, k5
    const uint32_t p2 = (w >> 4) & 0x00F000F0u;   // k2, k6
    const uint32_t p3 = (w >> 8) & 0x00F000F0u;   // k3, k7
    const f16x2 a = as_f16x2(p0), b = as_f16x2(p1), c = as_f16x2(p2), d = as_f16x2(p3);
    return f16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// One 8-k chunk of activations, owned by one of CPG lanes (CPG = group / 8, consecutive lanes)
// that together hold one quantization group of one row: returns the group's {2^(16-E), Sx} to
// every lane and writes the lane's scaled hi/lo fragments. Butterfly reductions give every lane
// the same bits (IEEE addition is commutative), so the result does not depend on the lane.
template <int CPG>
__device__ __forceinline__ float2 prep_group_chunk(const float v[8], uint4* hi_out, uint4* lo_out)
{
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
#pragma unroll
    for (int off = 1; off < CPG; off <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off));
        sum += __shfl_xor(sum, off);
    }
    const int E = row_exponent(amax);
    split8(v, ldexpf(1.f, E), hi_out, lo_out);
    return float2{ldexpf(1.f, 16 - E), sum};
}

// Activations of a linear with M > 4, prepared once per call:
//   xs[c * 2M + 2m + h] (h: hi/lo) for every 8-k chunk c; gs[g * M + m] = {2^(16-E), Sx[g,m]}.
// group/8 lanes per (group, row); grid.x covers G * M * group/8 lanes, grid.y the batch.
template <int CPG>
__global__ __launch_bounds__(256) void xsplit_kernel(const GemvBatch b)
{
    const GemvLinear& L = b.L[blockIdx.y];
    if (!L.xs_owner) return;
    const int M = b.M;
    const int G = L.K / L.group;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int item = idx / CPG;                        // (group, row) pair, uniform per CPG lanes
    if (item >= G * M) return;
    const int c = idx - item * CPG;
    const int cpg = CPG;
    const int g = item / M;
    const int m = item - g * M;
    const int chunk = g * cpg + c;
    float v[8];
    load8(L.x, b.x_dtype, (size_t)m * L.K + (size_t)chunk * 8, v);
    uint4* xs = const_cast<uint4*>(L.xs);
    const float2 gs = prep_group_chunk<CPG>(v, &xs[(size_t)chunk * 2 * M + 2 * m],
                                       &xs[(size_t)chunk * 2 * M + 2 * m + 1]);
    if (c == 0) const_cast<float2*>(L.gs)[(size_t)g * M + m] = gs;
}

template <int T, int KB, bool FUSED>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(const GemvBatch b)
{
    extern __shared__ uint4 dyn_lds[];        // FUSED: split activations + Sx of this segment
    __shared__ float red[kGemvWaves][kGemvMaxM][kGemvCols];
    __shared__ uint32_t is_last;

    int wg = blockIdx.x;
    int li = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatch; i++)
        if (i < b.count && wg >= b.L[i].wg_begin) li = i;
    const GemvLinear& L = b.L[li];
    const uint32_t* __restrict__ qweight = L.qweight;
    const uint32_t* __restrict__ qzeros = L.qzeros;
    const uint16_t* __restrict__ scales = L.scales;
    const int N = L.N;
    const int K = L.K;
    const int split = L.split;
    wg -= L.wg_begin;
    const int strip = wg % L.strips;
    const int seg = wg / L.strips;

    const int M = b.M;
    const int R = 2 * M;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int NC = (N + 7) >> 3;
    const int n = strip * kGemvCols + 4 * j;
    const bool col_ok = n < N;
    const int G = K / (KB * 32);
    const int g0 = (int)((int64_t)G * seg / split);
    const int g1 = (int)((int64_t)G * (seg + 1) / split);
    const int p0 = g0 * KB * 4;               // first packed row (8-k chunk) of the segment
    const int chunks = (g1 - g0) * KB * 4;

    // software pipeline: the next group's packed words, zeros and scales are in flight while
    // the current group is unpacked and multiplied
    uint4 wn[KB];
    uint32_t zn = 0x77777777u;
    uint2 sn = uint2{0u, 0u};
    auto fetch = [&](int g) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
            wn[kb] = *reinterpret_cast<const uint4*>(qweight + (size_t)((g * KB + kb) * 4 + kq) * N + n);
        if (qzeros) zn = qzeros[(size_t)g * NC + (n >> 3)];
        sn = *reinterpret_cast<const uint2*>(scales + (size_t)g * N + n);
    };
#pragma unroll
    for (int kb = 0; kb < KB; kb++) wn[kb] = uint4{0u, 0u, 0u, 0u};
    int g = g0 + wave;
    if (g < g1 && col_ok) fetch(g);

    uint4* xs_lds = dyn_lds;
    float2* gs_lds = reinterpret_cast<float2*>(dyn_lds + (FUSED ? chunks * R : 0));
    if (FUSED) {
        // the segment's activations: KB*4 lanes per (group, row), one chunk of 8 k per lane
        constexpr int CPG = KB * 4;
        const int items = (g1 - g0) * M;
        for (int base = 0; base < items * CPG; base += 256) {
            const int idx = base + threadIdx.x;
            const int item = idx / CPG;                 // uniform per CPG lanes
            if (item < items) {
                const int cl = idx - item * CPG;
                const int gg = item / M;
                const int m = item - gg * M;
                const int c = gg * CPG + cl;            // chunk within the segment
                float v[8];
                load8(L.x, b.x_dtype, (size_t)m * K + (size_t)(p0 + c) * 8, v);
                const float2 gsv = prep_group_chunk<CPG>(v, &xs_lds[c * R + 2 * m], &xs_lds[c * R + 2 * m + 1]);
                if (cl == 0) gs_lds[gg * M + m] = gsv;
            }
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
        const uint32_t zw = qzeros ? (zn >> (4 * (n & 7))) : 0x7777u;
        const uint2 sv = sn;
        if (g + kGemvWaves < g1 && col_ok) fetch(g + kGemvWaves);

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
                const f16x8 bq = nibbles_subnormal(words[u]);
#pragma unroll
                for (int t = 0; t < T; t++) c[u][t] = mfma_16x16x32_f16(a[t], bq, c[u][t]);
            }
        }
        // group epilogue: acc += s * 2^(16-E) * C (all rows), acc -= s * z * Sx (hi rows only)
        const uint32_t sw[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
        float2 gsr[T][2];
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int m = 8 * t + 2 * kq + h;
                gsr[t][h] = m < M ? (FUSED ? gs_lds[(g - g0) * M + m] : L.gs[(size_t)g * M + m])
                                  : float2{0.f, 0.f};
            }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
            const float sz = s * (float)(((zw >> (4 * u)) & 15u) + 1u);
#pragma unroll
            for (int t = 0; t < T; t++) {
                const float sb0 = s * gsr[t][0].x, sb1 = s * gsr[t][1].x;
                acc[u][t][0] += sb0 * c[u][t][0] - sz * gsr[t][0].y;
                acc[u][t][1] += sb0 * c[u][t][1];
                acc[u][t][2] += sb1 * c[u][t][2] - sz * gsr[t][1].y;
                acc[u][t][3] += sb1 * c[u][t][3];
            }
        }
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

    for (int idx = threadIdx.x; idx < M * kGemvCols; idx += 256) {
        const int m = idx >> 6;
        const int col = idx & 63;
        const int nn = strip * kGemvCols + col;
        if (nn >= N) continue;
        const float sum = ((red[0][m][col] + red[1][m][col]) + red[2][m][col]) + red[3][m][col];
        if (split == 1) {
            L.y[(size_t)m * N + nn] = L.bias ? sum + L.bias[nn] : sum;
        } else {
            __hip_atomic_store(&L.partial[((size_t)seg * M + m) * N + nn], sum, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (split == 1) return;

    // this wave's partial stores are complete (written through to the coherence point) before
    // the workgroup signals arrival
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&L.counters[strip], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t last = prev == (uint32_t)(split - 1);
        if (last) __hip_atomic_store(&L.counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = last;
    }
    __syncthreads();
    if (!is_last) return;
    for (int idx = threadIdx.x; idx < M * kGemvCols; idx += 256) {
        const int m = idx >> 6;
        const int col = idx & 63;
        const int nn = strip * kGemvCols + col;
        if (nn >= N) continue;
        float sum = 0.f;
        for (int s2 = 0; s2 < split; s2++)
            sum += __hip_atomic_load(&L.partial[((size_t)s2 * M + m) * N + nn], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
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
        // the segment's split activations (2M rows x group/8 chunks x 16 B) plus its per-group
        // {scale, sum} pairs (M float2 per group) must fit the LDS budget
        int max_groups = kGemvLdsXsBytes / (4 * M * group + 8 * M);
        if (max_groups < 1) max_groups = 1;
        const int need = (s.groups + max_groups - 1) / max_groups;
        if (s.split < need) s.split = need;
    }
    if (s.split > s.groups) s.split = s.groups;
    if (s.split < 1) s.split = 1;
    return s;
}

// scratch layout for M > 4: xs [K/8][2M] uint4, then gs [K/group][M] float2
uint64_t gemv_xs_bytes(int M, int K)
{
    if (gemv_fused(M)) return 0;
    const uint64_t xs = (uint64_t)4 * M * K;
    const uint64_t gs = (uint64_t)8 * M * (K / 32);
    return (xs + gs + 255) & ~(uint64_t)255;
}

uint64_t gemv_partial_bytes(int M, int N, int split)
{
    if (split <= 1) return 0;
    return ((uint64_t)split * M * N * 4 + 255) & ~(uint64_t)255;
}

void gemv_xs_layout(GemvLinear& L, char* base, int M)
{
    L.xs = reinterpret_cast<const uint4*>(base);
    L.gs = reinterpret_cast<const float2*>(base + (size_t)4 * M * L.K);
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
            lds = max(lds, (size_t)gmax * kb * 4 * (2 * b.M) * 16 + (size_t)gmax * b.M * 8);
        }
        return launch_tiles<1, true>(b, kb, lds, stream);
    }
    int lanes = 0;
    for (int i = 0; i < b.count; i++) lanes = max(lanes, (b.L[i].K >> 3) * b.M);
    const dim3 xg((lanes + 255) / 256, b.count);
    switch (kb) {
    case 1: hipLaunchKernelGGL(xsplit_kernel<4>, xg, dim3(256), 0, stream, b); break;
    case 2: hipLaunchKernelGGL(xsplit_kernel<8>, xg, dim3(256), 0, stream, b); break;
    case 4: hipLaunchKernelGGL(xsplit_kernel<16>, xg, dim3(256), 0, stream, b); break;
    case 8: hipLaunchKernelGGL(xsplit_kernel<32>, xg, dim3(256), 0, stream, b); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return b.M <= 8 ? launch_tiles<1, false>(b, kb, 0, stream) : launch_tiles<2, false>(b, kb, 0, stream);
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
