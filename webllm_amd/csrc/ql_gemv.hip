// Decode GEMV for GPTQ int4 linears, M = 1..16 rows: y[M,N] = x[M,K] * W^T (+ bias), fp32 out.
//
// Replaces the reference's gemm_gemv_f16 / gemm_gemv_split_f16 + gemm_gemv_split_reduce pair
// (src/gpu/kernels/gemm/*.wgsl, dispatched by src/model/qwen.ts:568-610), which streams fp16
// weights that the CPU dequantized at load time. Here the weights stay packed (4 bits/weight)
// and the products run on the int8 matrix cores with exact integer accumulation.
//
// Arithmetic (tracks the reference CPU path — fp32 weights, double accumulation — to ~1e-7):
//   y[m,n] = sum_g s[g,n] * ( 2^-E[g,m] * sum_{k in g} q[k,n] * X[m,k] * 2^-24  -  z[g,n] * Sx[g,m] )
//   X[m,k] = round(x[m,k] * 2^(E+24)),  E[g,m] chosen so max_{k in g} |x| * 2^E < 64,
//   Sx[g,m] = sum_{k in g} x[m,k]  (fp32, fixed order).
// * q: a packed word w holds 8 nibbles; w & 0x0F0F0F0F and (w >> 4) & 0x0F0F0F0F are 8 int8
//   values (3 integer ops per word, no conversions).
// * X is split into 4 signed base-256 digits: with V = (X + 0x808080) ^ 0x808080 the four bytes
//   of V are exactly the two's-complement digits b0..b3, X = sum_i b_i 256^i. Each digit is one
//   MFMA row (row 4m + i), so v_mfma_i32_16x16x64_i8 gives exact int32 dot products sum q*b_i;
//   the group epilogue combines them in fp32 (x precision ~2^-30 of the group maximum).
// * Per 64-k block a lane feeds packed rows 2kq, 2kq+1 of one column (16 nibbles); the
//   activation digits are staged in the same byte order, so the dot product is unchanged.
//
// Work split: a workgroup (4 waves) owns 256 output columns (64 per wave) and one K segment of
// whole quantization groups; the segment's activation digits are built once in LDS and shared by
// the 4 waves. Each wave streams its columns' groups with kPrefetch groups of packed words in
// flight. With split > 1 segments, each workgroup stores its partial sums with agent-scope
// (cross-XCD coherent) stores and bumps a per-strip arrival counter; the last one adds the
// partials in ascending segment order — deterministic, like the reference's two-pass reduce
// (gemm_gemv_split_reduce.wgsl:32-38), in one launch — and resets the counter. Agent-scope
// *fences* are avoided on purpose: on this part they write back and invalidate the whole L2.
#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

// Tunables (compile-time; the defaults are the measured best on MI355X):
//   QL_GEMV_TARGET_WAVES  waves a launch aims for (K segments per column strip follow from it)
//   QL_GEMV_PREFETCH      groups each wave keeps in flight ahead of the one it multiplies
//   QL_GEMV_MIN_GROUPS    fewest quantization groups per K segment (caps the split)
#ifndef QL_GEMV_TARGET_WAVES
#define QL_GEMV_TARGET_WAVES 1024
#endif
#ifndef QL_GEMV_MIN_GROUPS
#define QL_GEMV_MIN_GROUPS 2
#endif
#ifndef QL_GEMV_PREFETCH
#define QL_GEMV_PREFETCH 2
#endif
constexpr int kTargetWaves = QL_GEMV_TARGET_WAVES;
constexpr int kPrefetch = QL_GEMV_PREFETCH;
constexpr int kMinGroupsPerWave = QL_GEMV_MIN_GROUPS;   // split-K stops where segments get shorter
constexpr int kLdsBudget = 49152;          // activation digits + group stats per workgroup

template <int T, int NB>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(const GemvBatch b)
{
    // dynamic LDS: activation digits [segment block][kq][row] (16 B), then {2^-E, Sx}[group][m]
    extern __shared__ uint4 dyn_lds[];
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
    const int R = 4 * M;                      // MFMA rows: 4 digits per activation row
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int NC = (N + 7) >> 3;
    const int n = strip * kGemvStripCols + wave * 64 + 4 * j;
    const bool col_ok = n < N;
    const int G = K / (NB * 64);
    const int g0 = (int)((int64_t)G * seg / split);
    const int g1 = (int)((int64_t)G * (seg + 1) / split);
    const int gseg = g1 - g0;

    uint4* xd = dyn_lds;                                                   // digits
    float2* gst = reinterpret_cast<float2*>(dyn_lds + gseg * NB * 4 * R);  // group stats

    // software pipeline: each wave keeps the packed words, zeros and scales of its next
    // kPrefetch groups in flight (static register slots; the group loop is unrolled by
    // kPrefetch). Every load is unconditional — past-the-end groups and columns are clamped to
    // valid addresses and contribute with scale 0 — so the loop is straight-line and the
    // compiler waits for exactly the slot it consumes.
    const int n_ld = col_ok ? n : N - 4;
    uint4 wb[kPrefetch][2 * NB];
    uint32_t zb[kPrefetch];
    uint2 sb[kPrefetch];
    auto fetch = [&](int d, int g) {
        g = min(g, g1 - 1);
#pragma unroll
        for (int r = 0; r < 2 * NB; r++) {
            const int prow = (g * NB + (r >> 1)) * 8 + 2 * kq + (r & 1);
            wb[d][r] = *reinterpret_cast<const uint4*>(qweight + (size_t)prow * N + n_ld);
        }
        zb[d] = qzeros ? qzeros[(size_t)g * NC + (n_ld >> 3)] : 0x77777777u;
        sb[d] = *reinterpret_cast<const uint2*>(scales + (size_t)g * N + n_ld);
    };
#pragma unroll
    for (int d = 0; d < kPrefetch; d++) fetch(d, g0 + d);

    {
        // the segment's activation digits: 8*NB lanes per (group, row), one 8-k chunk per lane
        constexpr int CPG = NB * 8;
        const int items = gseg * M;
        for (int base = 0; base < items * CPG; base += 256) {
            const int idx = base + threadIdx.x;
            const int item = idx / CPG;                 // uniform per CPG lanes
            if (item < items) {
                const int c = idx - item * CPG;         // chunk within the group
                const int gg = item / M;
                const int m = item - gg * M;
                float v[8];
                load8(L.x, b.x_dtype, (size_t)m * K + (size_t)(g0 + gg) * (NB * 64) + (size_t)c * 8, v);
                const int blk = gg * NB + (c >> 3);     // 64-k block within the segment
                const int ckq = (c & 7) >> 1;
                uint2* rows = reinterpret_cast<uint2*>(&xd[(blk * 4 + ckq) * R + 4 * m]) + (c & 1);
                const float2 st = prep_chunk<CPG>(v, rows, 2);
                if (c == 0) gst[gg * M + m] = st;
            }
        }
        __syncthreads();
    }

    float acc[4][T];
#pragma unroll
    for (int u = 0; u < 4; u++)
#pragma unroll
        for (int t = 0; t < T; t++) acc[u][t] = 0.f;

    auto consume = [&](int gg, const uint4* w, uint32_t zn, uint2 sv) {
        i32x4 c[4][T];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int t = 0; t < T; t++) c[u][t] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int bb = 0; bb < NB; bb++) {
            i32x4 a[T];
#pragma unroll
            for (int t = 0; t < T; t++) {
                const int row = 16 * t + j;
                a[t] = row < R ? __builtin_bit_cast(i32x4, xd[((gg * NB + bb) * 4 + kq) * R + row])
                               : i32x4{0, 0, 0, 0};
            }
            const uint4 w0 = w[2 * bb], w1 = w[2 * bb + 1];
            const uint32_t lo[4] = {w0.x, w0.y, w0.z, w0.w};
            const uint32_t hi[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const i32x4 bq = i32x4{(int)(lo[u] & 0x0F0F0F0Fu), (int)((lo[u] >> 4) & 0x0F0F0F0Fu),
                                       (int)(hi[u] & 0x0F0F0F0Fu), (int)((hi[u] >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
                for (int t = 0; t < T; t++) c[u][t] = mfma_i8(a[t], bq, c[u][t]);
            }
        }
        // group epilogue: lane (j, kq) holds, per tile t, digits 0..3 of row m = 4t + kq
        const uint32_t zw = zn >> (4 * (n & 7));
        const uint32_t sw[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
        float2 st[T];
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int m = 4 * t + kq;
            st[t] = m < M ? gst[gg * M + m] : float2{0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
            const float sz = s * (float)(((zw >> (4 * u)) & 15u) + 1u);
#pragma unroll
            for (int t = 0; t < T; t++) {
                float v = fmaf((float)c[u][t][0], 0x1p-8f, (float)c[u][t][1]);
                v = fmaf(v, 0x1p-8f, (float)c[u][t][2]);
                v = fmaf(v, 0x1p-8f, (float)c[u][t][3]);            // sum q * X * 2^-24
                acc[u][t] = fmaf(s * st[t].x, v, acc[u][t]);
                acc[u][t] = fmaf(-sz, st[t].y, acc[u][t]);
            }
        }
    };

    for (int ib = 0; ib < gseg; ib += kPrefetch) {
#pragma unroll
        for (int d = 0; d < kPrefetch; d++) {
            const int i = ib + d;
            uint4 w[2 * NB];
#pragma unroll
            for (int r = 0; r < 2 * NB; r++) w[r] = wb[d][r];
            const uint32_t zn = zb[d];
            const uint2 sv = col_ok ? sb[d] : uint2{0u, 0u};
            fetch(d, g0 + i + kPrefetch);
            if (i < gseg) consume(i, w, zn, sv);
        }
    }

    // results: lane holds y[4t + kq][n + u] in acc[u][t]
    if (split == 1) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int m = 4 * t + kq;
            if (m < M && col_ok) {
                float4 o = float4{acc[0][t], acc[1][t], acc[2][t], acc[3][t]};
                if (L.bias) {
                    const float4 bv = *reinterpret_cast<const float4*>(L.bias + n);
                    o.x += bv.x; o.y += bv.y; o.z += bv.z; o.w += bv.w;
                }
                *reinterpret_cast<float4*>(L.y + (size_t)m * N + n) = o;
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int m = 4 * t + kq;
        if (m < M && col_ok) {
            float* p = L.partial + ((size_t)seg * M + m) * N + n;
#pragma unroll
            for (int u = 0; u < 4; u++)
                __hip_atomic_store(p + u, acc[u][t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
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
    for (int idx = threadIdx.x; idx < M * kGemvStripCols; idx += 256) {
        const int m = idx / kGemvStripCols;
        const int nn = strip * kGemvStripCols + (idx - m * kGemvStripCols);
        if (nn >= N) continue;
        // coherent loads in batches of 8 (issued together, one wait per batch), summed in
        // ascending segment order
        const float* pp = L.partial + (size_t)m * N + nn;
        const size_t stride = (size_t)M * N;
        float sum = 0.f;
        for (int s0 = 0; s0 < split; s0 += 8) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; e++)
                v[e] = s0 + e < split ? __hip_atomic_load(pp + (size_t)(s0 + e) * stride, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                      : 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (s0 + e < split) sum += v[e];
        }
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

template <int T>
hipError_t launch_tiles(const GemvBatch& b, int nb, size_t lds, hipStream_t stream)
{
    dim3 grid(b.wg_total), block(256);
    switch (nb) {
    case 1: hipLaunchKernelGGL((gemv_mfma_kernel<T, 1>), grid, block, lds, stream, b); break;
    case 2: hipLaunchKernelGGL((gemv_mfma_kernel<T, 2>), grid, block, lds, stream, b); break;
    case 4: hipLaunchKernelGGL((gemv_mfma_kernel<T, 4>), grid, block, lds, stream, b); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t lds_per_group(int M, int group) { return (size_t)(group / 64) * 4 * (4 * M) * 16 + 8 * (size_t)M; }

}  // namespace

bool gemv_fast_ok(int M, int N, int K, int group)
{
    return M >= 1 && M <= kGemvMaxM && N > 0 && K > 0 && N % 4 == 0 &&
           (group == 64 || group == 128 || group == 256) && K % group == 0;
}

GemvShape gemv_shape(int M, int N, int K, int group)
{
    GemvShape s;
    s.strips = (N + kGemvStripCols - 1) / kGemvStripCols;
    s.groups = K / group;
    s.waves = 4;
    s.split = (kTargetWaves + 4 * s.strips - 1) / (4 * s.strips);
    const int max_split = s.groups / kMinGroupsPerWave;
    if (s.split > max_split) s.split = max_split;
    // the segment's activation digits and group stats must fit the LDS budget
    const int max_groups = (int)(kLdsBudget / lds_per_group(M, group));
    const int need = (s.groups + max_groups - 1) / (max_groups > 0 ? max_groups : 1);
    if (s.split < need) s.split = need;
    if (s.split > s.groups) s.split = s.groups;
    if (s.split < 1) s.split = 1;
    return s;
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
    size_t lds = 0;
    for (int i = 0; i < b.count; i++) {
        const int G = b.L[i].K / group;
        const int gmax = (G + b.L[i].split - 1) / b.L[i].split;
        lds = max(lds, (size_t)gmax * lds_per_group(b.M, group));
    }
    const int nb = group / 64;
    if (b.M <= 4) return launch_tiles<1>(b, nb, lds, stream);
    if (b.M <= 8) return launch_tiles<2>(b, nb, lds, stream);
    return launch_tiles<4>(b, nb, lds, stream);
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
