// Decode attention over the KV cache and the cache store, the non-linear GPU work of a decode
// step beside the quantized linears (reference: src/model/qwen.ts:424-442,
// src/gpu/kernels/attention/attention_gqa_cache.wgsl, src/gpu/kernels/misc/kv_store.wgsl).
//
// Cache layout (as the reference's): per layer one fp32 K and one fp32 V buffer, [max_t, KV * D]
// row-major, row t holding every kv head's vector for position t. Query row m of a call sits at
// absolute position past + m and sees keys 0 .. past + m (causal). Query head h reads kv head
// h / G, G = H / KV (grouped-query attention).
//
// attn_kernel<GM, NJ>: one workgroup (4 waves) per (query row m, run of up to GM heads of one kv
// group, key split). K and V rows are read once for all the heads of the run.
//   scores   16 lanes per key, each holding NJ 16-byte pieces of the row (4 floats per 64 of D:
//            coalesced reads), 4 keys per wave per step, dot products with the GM query vectors
//            kept in registers, butterfly over the 16 lanes; scores in LDS
//   softmax  per head: max, e = exp(score - max), sum over the split's keys
//   output   thread (chunk c of 4 values of D, part q) sums p_s * V[s] over keys s = q mod parts;
//            the parts are added in ascending order (deterministic)
// Without a key split (one split) p = e / sum, normalized before weighting V as the reference's
// CPU attention does, and the workgroup writes the output. With splits (enough workgroups for
// the chip when rows x heads are few, as in decode) each split writes its max, sum and the
// unnormalized e-weighted V sums to the context's workspace and attn_combine_kernel merges the
// splits in ascending order: out = sum_i acc_i exp(max_i - max) / sum_i sum_i exp(max_i - max).
// Bytes per call: the visible K and V rows once (plus q and out); HBM-bound at long contexts.
#include <algorithm>
#include <cmath>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnLdsFloats = 16384;    // 64 KiB of LDS per workgroup: scores, reductions, parts
constexpr int kAttnWantBlocks = 512;     // workgroups to aim for (two per CU)
constexpr int kAttnMinKeys = 64;         // keys per split, at least
constexpr int kAttnSplitMinT = 512;      // shorter contexts: no key split (the merge launch costs more)
constexpr int kAttnMinBlocks = 256;      // fewer workgroups: give up sharing K/V rows over heads
constexpr int kU = 4;                    // K row loads in flight per lane before use
constexpr int kUV = 8;                   // V row loads in flight per lane before use

// per-head max or sum over the workgroup; red holds 4 * GM floats; all threads call it
template <int GM, bool MAX>
__device__ __forceinline__ void block_reduce(float (&v)[GM], float* red)
{
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int g = 0; g < GM; g++) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float w = __shfl_xor(v[g], o);
            v[g] = MAX ? fmaxf(v[g], w) : v[g] + w;
        }
        if ((threadIdx.x & 63) == 0) red[g * 4 + wave] = v[g];
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GM; g++) {
        const float* r = red + g * 4;
        v[g] = MAX ? fmaxf(fmaxf(r[0], r[1]), fmaxf(r[2], r[3])) : (r[0] + r[1]) + (r[2] + r[3]);
    }
    __syncthreads();
}

template <int GM, int NJ>
__global__ __launch_bounds__(kAttnThreads) void attn_kernel(const AttnArgs a)
{
    extern __shared__ float lds[];
    const int run = blockIdx.x, split = blockIdx.y, m = blockIdx.z;
    const int D = a.D, H = a.H, G = a.G;
    const int kvh = run / a.runs_per_group;
    const int h0 = kvh * G + (run % a.runs_per_group) * a.heads_per_run;
    const int ng = min(a.heads_per_run, kvh * G + G - h0);          // heads of this run (<= GM)
    const int row_len = a.KV * D;
    const int T = a.past + m + 1;                                   // visible keys
    const int chunk = (T + a.nsplit - 1) / a.nsplit;
    const int s_lo = min(T, split * chunk), n = min(T, s_lo + chunk) - s_lo;
    const int cap = a.chunk_cap;
    float* scores = lds;                                            // [GM][cap]
    float* red = lds + GM * cap;                                    // [GM][4]
    float* parts = red + 4 * GM;                                    // [P][GM][D]

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l16 = lane & 15, kq = lane >> 4;
    f32x4 qv[GM][NJ];
#pragma unroll
    for (int g = 0; g < GM; g++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int d = 64 * j + 4 * l16;
            qv[g][j] = (g < ng && d < D) ? *reinterpret_cast<const f32x4*>(a.q + ((size_t)m * H + h0 + g) * D + d)
                                         : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    const float* kbase = a.k + (size_t)s_lo * row_len + (size_t)kvh * D;
    // kU steps of 16 keys: every row load of the round is issued before the first dot product
    for (int i0 = 0; i0 < n; i0 += 16 * kU) {
        f32x4 kv[kU][NJ];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int i = i0 + 16 * u + wave * 4 + kq;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int d = 64 * j + 4 * l16;
                kv[u][j] = (i < n && d < D) ? *reinterpret_cast<const f32x4*>(kbase + (size_t)i * row_len + d)
                                            : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const int i = i0 + 16 * u + wave * 4 + kq;
#pragma unroll
            for (int g = 0; g < GM; g++) {
                float dot = 0.f;
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    dot = fmaf(qv[g][j].x, kv[u][j].x, dot);
                    dot = fmaf(qv[g][j].y, kv[u][j].y, dot);
                    dot = fmaf(qv[g][j].z, kv[u][j].z, dot);
                    dot = fmaf(qv[g][j].w, kv[u][j].w, dot);
                }
                dot += __shfl_xor(dot, 8);
                dot += __shfl_xor(dot, 4);
                dot += __shfl_xor(dot, 2);
                dot += __shfl_xor(dot, 1);
                if (i < n && l16 == 0) scores[g * cap + i] = dot * a.scale;
            }
        }
    }
    __syncthreads();

    float mx[GM], sum[GM];
#pragma unroll
    for (int g = 0; g < GM; g++) {
        mx[g] = -INFINITY;
        for (int i = threadIdx.x; i < n; i += kAttnThreads) mx[g] = fmaxf(mx[g], scores[g * cap + i]);
    }
    block_reduce<GM, true>(mx, red);
#pragma unroll
    for (int g = 0; g < GM; g++) {
        sum[g] = 0.f;
        for (int i = threadIdx.x; i < n; i += kAttnThreads) {
            const float e = expf(scores[g * cap + i] - mx[g]);
            scores[g * cap + i] = e;
            sum[g] += e;
        }
    }
    block_reduce<GM, false>(sum, red);        // its barriers also order the e stores
    const bool whole = a.nsplit == 1;
    if (whole) {
#pragma unroll
        for (int g = 0; g < GM; g++)
            for (int i = threadIdx.x; i < n; i += kAttnThreads) scores[g * cap + i] = scores[g * cap + i] / sum[g];
        __syncthreads();
    }

    const int nc = D / 4;                     // 4-value chunks of D
    const int P = kAttnThreads / nc;          // parts over the keys
    const int c = threadIdx.x % nc, part = threadIdx.x / nc;
    if (part < P) {
        f32x4 acc[GM];
#pragma unroll
        for (int g = 0; g < GM; g++) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float* vbase = a.v + (size_t)s_lo * row_len + (size_t)kvh * D + 4 * c;
        for (int i0 = part; i0 < n; i0 += P * kUV) {
            f32x4 vv[kUV];
#pragma unroll
            for (int u = 0; u < kUV; u++) {
                const int i = i0 + P * u;
                vv[u] = i < n ? *reinterpret_cast<const f32x4*>(vbase + (size_t)i * row_len) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < kUV; u++) {
                const int i = i0 + P * u;
                if (i < n) {
#pragma unroll
                    for (int g = 0; g < GM; g++) {
                        const float p = scores[g * cap + i];
                        acc[g].x = fmaf(p, vv[u].x, acc[g].x);
                        acc[g].y = fmaf(p, vv[u].y, acc[g].y);
                        acc[g].z = fmaf(p, vv[u].z, acc[g].z);
                        acc[g].w = fmaf(p, vv[u].w, acc[g].w);
                    }
                }
            }
        }
#pragma unroll
        for (int g = 0; g < GM; g++) *reinterpret_cast<f32x4*>(parts + (part * GM + g) * D + 4 * c) = acc[g];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < ng * nc; t += kAttnThreads) {
        const int g = t / nc, cc = t - g * nc;
        f32x4 o = *reinterpret_cast<const f32x4*>(parts + g * D + 4 * cc);
        for (int q2 = 1; q2 < P; q2++) {
            const f32x4 w = *reinterpret_cast<const f32x4*>(parts + (q2 * GM + g) * D + 4 * cc);
            o.x += w.x;
            o.y += w.y;
            o.z += w.z;
            o.w += w.w;
        }
        const size_t row = (size_t)m * H + h0 + g;                  // (m, h)
        if (whole) {
            st_global(reinterpret_cast<f32x4*>(a.out + row * D + 4 * cc), o);
        } else {
            const size_t slot = row * a.nsplit + split;
            st_global(reinterpret_cast<f32x4*>(a.ws + slot * D + 4 * cc), o);
            if (cc == 0) {
                float* st = a.ws + (size_t)a.M * H * a.nsplit * D + 2 * slot;
                st_global(st, mx[g]);
                st_global(st + 1, sum[g]);
            }
        }
    }
}

// one wave per (h, m): lane i < S reads split i's max and sum (S <= 64), the wave forms the
// weights exp(max_i - max) / sum_j sum_j exp(max_j - max) in LDS, then lanes take 4-value chunks
// of D and add the splits in ascending order
__global__ __launch_bounds__(64) void attn_combine_kernel(const AttnArgs a)
{
    __shared__ float wgt[64];
    const int h = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
    const size_t row = (size_t)m * a.H + h;
    const int S = a.nsplit, D = a.D;
    const float* st = a.ws + (size_t)a.M * a.H * S * D + 2 * row * S;
    const float mi = lane < S ? ld_global(st + 2 * lane) : -INFINITY;
    const float li = lane < S ? ld_global(st + 2 * lane + 1) : 0.f;
    float mx = mi;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const float e = lane < S ? expf(mi - mx) : 0.f;
    float l = li * e;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
    wgt[lane] = e / l;
    __syncthreads();
    for (int cc = lane; cc < D / 4; cc += 64) {
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
        const f32x4* src = reinterpret_cast<const f32x4*>(a.ws + row * S * D) + cc;
#pragma unroll 8
        for (int i = 0; i < S; i++) {
            const float w = wgt[i];
            const f32x4 v = ld_global(src + (size_t)i * (D / 4));
            o.x = fmaf(w, v.x, o.x);
            o.y = fmaf(w, v.y, o.y);
            o.z = fmaf(w, v.z, o.z);
            o.w = fmaf(w, v.w, o.w);
        }
        st_global(reinterpret_cast<f32x4*>(a.out + row * D) + cc, o);
    }
}

// dst[(pos0 + r) * row_len + c] = src[r * row_len + c], four floats per thread
__global__ __launch_bounds__(256) void kv_store_kernel(const float* src, float* dst, int n4, int row4, int pos0)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const int r = i / row4, c = i - r * row4;
    const f32x4 v = ld_global(reinterpret_cast<const f32x4*>(src) + i);
    st_global(reinterpret_cast<f32x4*>(dst) + (size_t)(pos0 + r) * row4 + c, v);
}

typedef void (*AttnFn)(AttnArgs);

template <int NJ>
AttnFn attn_fn_nj(int gm)
{
    switch (gm) {
    case 1: return attn_kernel<1, NJ>;
    case 2: return attn_kernel<2, NJ>;
    case 4: return attn_kernel<4, NJ>;
    default: return NJ <= 2 ? attn_kernel<8, NJ <= 2 ? NJ : 2> : nullptr;
    }
}

AttnFn attn_fn(int gm, int nj)
{
    if (nj == 1) return attn_fn_nj<1>(gm);
    if (nj == 2) return attn_fn_nj<2>(gm);
    return attn_fn_nj<4>(gm);
}

size_t attn_lds_bytes(int gm, int cap, int D)
{
    const int P = kAttnThreads / (D / 4);
    return ((size_t)gm * cap + 4 * gm + (size_t)P * gm * D) * sizeof(float);
}

}  // namespace

// Heads per run (GM: 1, 2, 4 or 8, at most 16 f32x4 of query registers), key splits (enough
// workgroups, scores within LDS, workspace within its capacity) and the LDS size. Runs of several
// heads read each K/V row once for all of them; while the grid would still be short of
// kAttnMinBlocks workgroups, fewer heads per run buy parallelism (the rows then come from L2).
int plan_attention(AttnArgs* a)
{
    const int nj = a->D <= 64 ? 1 : a->D <= 128 ? 2 : 4;
    int gm = 1;
    while (gm < 8 && gm < a->G && 2 * gm * nj <= 16) gm *= 2;
    const int tcap = a->past + a->M;
    for (;; gm /= 2) {
        const int hpr = std::min(gm, a->G);
        const int runs = a->KV * ((a->G + hpr - 1) / hpr);
        // scores of gm heads x the split's keys in what the reductions and V parts leave of LDS
        // (less 4 * gm: the split's key count is rounded up to a multiple of 4, which keeps the
        // parts after the scores 16-byte aligned)
        const int budget = kAttnLdsFloats - 8 * gm - (kAttnThreads / (a->D / 4)) * gm * a->D;
        const int min_split = (int)(((long long)gm * tcap + budget - 1) / budget);
        const long long blocks = (long long)runs * a->M;
        int want = (int)std::min<long long>(64, (kAttnWantBlocks + blocks - 1) / blocks);
        want = tcap < kAttnSplitMinT ? 1 : std::min(want, (tcap + kAttnMinKeys - 1) / kAttnMinKeys);
        int ns = std::max(min_split, std::max(want, 1));
        const size_t ws = (size_t)a->M * a->H * ns * (a->D + 2) * sizeof(float);
        if (ns > 1 && ws > kAttnWsBytes) ns = min_split;
        const size_t ws2 = (size_t)a->M * a->H * ns * (a->D + 2) * sizeof(float);
        const bool few = (long long)runs * a->M * ns < kAttnMinBlocks && gm > 1;
        if (!few && (ns == 1 || ws2 <= kAttnWsBytes)) {
            a->heads_per_run = hpr;
            a->gm = gm;
            a->runs_per_group = (a->G + hpr - 1) / hpr;
            a->nsplit = ns;
            a->chunk_cap = ((tcap + ns - 1) / ns + 3) & ~3;
            a->nj = nj;
            return 0;
        }
        if (gm == 1) return -1;
    }
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t stream)
{
    const AttnFn fn = attn_fn(a.gm, a.nj);
    if (!fn) return hipErrorInvalidValue;
    const size_t lds = attn_lds_bytes(a.gm, a.chunk_cap, a.D);
    hipLaunchKernelGGL(fn, dim3(a.KV * a.runs_per_group, a.nsplit, a.M), dim3(kAttnThreads), lds, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.H, a.M), dim3(64), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kv_store(const float* src, float* dst, int rows, int row_len, int pos0, hipStream_t stream)
{
    const int n4 = rows * row_len / 4;
    hipLaunchKernelGGL(kv_store_kernel, dim3((n4 + 255) / 256), dim3(256), 0, stream, src, dst, n4, row_len / 4, pos0);
    return hipGetLastError();
}

}  // namespace ql
