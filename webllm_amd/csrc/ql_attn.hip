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
// group, key split). K and V rows are read once for all the heads of the run, in one pass:
//   16 lanes per key, each holding NJ 16-byte pieces of the K and V rows (4 floats per 64 of D:
//   coalesced reads); a wave takes 4 keys per step, every lane two steps' rows in flight. A lane
//   keeps, per head, the running max, the sum of exp(score - max) and the e-weighted V sums of
//   its own keys (online softmax: a new max rescales the sums), so no phase waits for another.
//   The four key lanes of a wave then merge their states (xor 16, xor 32), the four waves merge
//   through LDS in wave order: state (m, l, acc) and (m', l', acc') give m* = max(m, m'),
//   l* = l e^(m - m*) + l' e^(m' - m*), acc* likewise.
// Without a key split the workgroup writes acc / l. With splits (enough workgroups for the chip
// when rows x heads are few, as in decode) each split writes its max, sum and acc to the
// context's workspace and attn_combine_kernel merges the splits in ascending order:
// out = sum_i acc_i exp(max_i - max) / sum_i sum_i exp(max_i - max).
// Bytes per call: the visible K and V rows once (plus q and out); HBM-bound at long contexts.
#include <algorithm>
#include <cmath>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWantBlocks = 512;     // workgroups to aim for (two per CU)
constexpr int kAttnMinKeys = 64;         // keys per split, at least (32 measured slower at 7B, 4096 positions)
constexpr int kAttnSplitMinT = 512;      // shorter contexts: no key split (the merge launch costs more)
constexpr int kAttnMinBlocks = 256;      // fewer workgroups: give up sharing K/V rows over heads
constexpr int kAttnMaxSplit = 128;      // key splits at most (the merge takes up to 256)
constexpr int kKB = 4;                   // wave steps (4 keys each) whose K and V rows a lane holds

// Scores are kept in base-2 units (the host folds log2(e) into the 1/sqrt(D) scale), so every
// exponential is the hardware exp2 (v_exp_f32, about 1 ulp) instead of a library expf.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum over the 16 lanes of a DPP row: row_ror:8, row_ror:4, quad_perm [2,3,0,1], [1,0,3,2]. Each
// step adds a pair that commutes, so every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_f<0x128>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0xB1>(v);
}

// online-softmax state (m, l, acc) merged with another: the larger max wins, both sides rescaled;
// a side without keys (m = -inf) contributes nothing
template <int NJ>
__device__ __forceinline__ void merge_state(float& m, float& l, f32x4 (&acc)[NJ], float mo, float lo,
                                            const f32x4 (&ao)[NJ])
{
    const float mn = fmaxf(m, mo);
    const float sa = m == -INFINITY ? 0.f : ex2(m - mn);
    const float sb = mo == -INFINITY ? 0.f : ex2(mo - mn);
    l = l * sa + lo * sb;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        acc[j].x = acc[j].x * sa + ao[j].x * sb;
        acc[j].y = acc[j].y * sa + ao[j].y * sb;
        acc[j].z = acc[j].z * sa + ao[j].z * sb;
        acc[j].w = acc[j].w * sa + ao[j].w * sb;
    }
    m = mn;
}

template <int GM, int NJ>
__global__ __launch_bounds__(kAttnThreads) void attn_kernel(const AttnArgs a)
{
    extern __shared__ float lds[];                                  // [4 waves][GM][D + 4]
    const int run = blockIdx.x, split = blockIdx.y, m = blockIdx.z;
    const int D = a.D, H = a.H, G = a.G;
    const int kvh = run / a.runs_per_group;
    const int h0 = kvh * G + (run % a.runs_per_group) * a.heads_per_run;
    const int ng = min(a.heads_per_run, kvh * G + G - h0);          // heads of this run (<= GM)
    const int row_len = a.KV * D;
    const int T = a.past + m + 1;                                   // visible keys
    const int chunk = (T + a.nsplit - 1) / a.nsplit;
    const int s_lo = min(T, split * chunk), n = min(T, s_lo + chunk) - s_lo;

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
    float mr[GM], lr[GM];
    f32x4 acc[GM][NJ];
#pragma unroll
    for (int g = 0; g < GM; g++) {
        mr[g] = -INFINITY;
        lr[g] = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[g][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float* kbase = a.k + (size_t)s_lo * row_len + (size_t)kvh * D;
    const float* vbase = a.v + (size_t)s_lo * row_len + (size_t)kvh * D;
    // kKB steps of 16 keys: every K and V row load of the round is issued before the first use
    for (int i0 = 0; i0 < n; i0 += 16 * kKB) {
        f32x4 kr[kKB][NJ], vr[kKB][NJ];
#pragma unroll
        for (int u = 0; u < kKB; u++) {
            const int i = i0 + 16 * u + wave * 4 + kq;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int d = 64 * j + 4 * l16;
                const bool ok = i < n && d < D;
                kr[u][j] = ok ? *reinterpret_cast<const f32x4*>(kbase + (size_t)i * row_len + d) : f32x4{0.f, 0.f, 0.f, 0.f};
                vr[u][j] = ok ? *reinterpret_cast<const f32x4*>(vbase + (size_t)i * row_len + d) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int g = 0; g < GM; g++) {
            float sc[kKB];
#pragma unroll
            for (int u = 0; u < kKB; u++) {
                float dot = 0.f;
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    dot = fmaf(qv[g][j].x, kr[u][j].x, dot);
                    dot = fmaf(qv[g][j].y, kr[u][j].y, dot);
                    dot = fmaf(qv[g][j].z, kr[u][j].z, dot);
                    dot = fmaf(qv[g][j].w, kr[u][j].w, dot);
                }
                dot = row16_sum(dot);
                sc[u] = i0 + 16 * u + wave * 4 + kq < n ? dot * a.scale : -INFINITY;
            }
            float bm = sc[0];
#pragma unroll
            for (int u = 1; u < kKB; u++) bm = fmaxf(bm, sc[u]);
            const float mn = fmaxf(mr[g], bm);
            if (mn == -INFINITY) continue;                          // no key of this lane yet
            const float r = ex2(mr[g] - mn);                        // 0 while the state is empty
            lr[g] *= r;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                acc[g][j].x *= r;
                acc[g][j].y *= r;
                acc[g][j].z *= r;
                acc[g][j].w *= r;
            }
#pragma unroll
            for (int u = 0; u < kKB; u++) {
                const float p = ex2(sc[u] - mn);                    // 0 past the split's keys
                lr[g] += p;
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    acc[g][j].x = fmaf(p, vr[u][j].x, acc[g][j].x);
                    acc[g][j].y = fmaf(p, vr[u][j].y, acc[g][j].y);
                    acc[g][j].z = fmaf(p, vr[u][j].z, acc[g][j].z);
                    acc[g][j].w = fmaf(p, vr[u][j].w, acc[g][j].w);
                }
            }
            mr[g] = mn;
        }
    }
    // the four key lanes of the wave (kq): merged pairwise; both partners compute the same sums
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1)
#pragma unroll
        for (int g = 0; g < GM; g++) {
            const float mo = __shfl_xor(mr[g], o), lo = __shfl_xor(lr[g], o);
            f32x4 ao[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                ao[j].x = __shfl_xor(acc[g][j].x, o);
                ao[j].y = __shfl_xor(acc[g][j].y, o);
                ao[j].z = __shfl_xor(acc[g][j].z, o);
                ao[j].w = __shfl_xor(acc[g][j].w, o);
            }
            merge_state<NJ>(mr[g], lr[g], acc[g], mo, lo, ao);
        }
    // the waves' states through LDS, merged in wave order
    const int stride = D + 4;
    if (kq == 0)
#pragma unroll
        for (int g = 0; g < GM; g++) {
            float* st = lds + (size_t)(wave * GM + g) * stride;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int d = 64 * j + 4 * l16;
                if (d < D) *reinterpret_cast<f32x4*>(st + d) = acc[g][j];
            }
            if (l16 == 0) {
                st[D] = mr[g];
                st[D + 1] = lr[g];
            }
        }
    __syncthreads();
    const int nc = D / 4;
    const bool whole = a.nsplit == 1;
    for (int t = threadIdx.x; t < ng * nc; t += kAttnThreads) {
        const int g = t / nc, c = t - g * nc;
        const float* st0 = lds + (size_t)g * stride;
        float mw = st0[D], lw = st0[D + 1];
        f32x4 o[1] = {*reinterpret_cast<const f32x4*>(st0 + 4 * c)};
        for (int w = 1; w < 4; w++) {
            const float* st = lds + (size_t)(w * GM + g) * stride;
            const f32x4 ow[1] = {*reinterpret_cast<const f32x4*>(st + 4 * c)};
            merge_state<1>(mw, lw, o, st[D], st[D + 1], ow);
        }
        const size_t row = (size_t)m * H + h0 + g;                  // (m, h)
        if (whole) {
            const float inv = 1.f / lw;
            st_global(reinterpret_cast<f32x4*>(a.out + row * D + 4 * c),
                      f32x4{o[0].x * inv, o[0].y * inv, o[0].z * inv, o[0].w * inv});
        } else {
            const size_t slot = row * a.nsplit + split;
            st_global(reinterpret_cast<f32x4*>(a.ws + slot * D + 4 * c), o[0]);
            if (c == 0) {
                float* stt = a.ws + (size_t)a.M * H * a.nsplit * D + 2 * slot;
                st_global(stt, mw);
                st_global(stt + 1, lw);
            }
        }
    }
}

// one workgroup per (h, m): wave 0 reads the splits' max and sum (lane i: splits i, i + 64, ...;
// S <= 256) and forms the weights exp(max_i - max) / sum_j sum_j exp(max_j - max) in LDS (sums
// in a fixed order); thread (part p, 4-value chunk c) then adds splits p, p + P, ... in ascending
// order, and the P parts are added in order
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a)
{
    __shared__ float wgt[256];
    __shared__ f32x4 part[256];
    const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const size_t row = (size_t)m * a.H + h;
    const int S = a.nsplit, D = a.D;
    if (t < 64) {
        const float* st = a.ws + (size_t)a.M * a.H * S * D + 2 * row * S;
        float mi[4], li[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = t + 64 * r;
            mi[r] = i < S ? ld_global(st + 2 * i) : -INFINITY;
            li[r] = i < S ? ld_global(st + 2 * i + 1) : 0.f;
        }
        float mx = fmaxf(fmaxf(mi[0], mi[1]), fmaxf(mi[2], mi[3]));
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float e[4], l = 0.f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            e[r] = mi[r] != -INFINITY ? ex2(mi[r] - mx) : 0.f;
            l += li[r] * e[r];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
#pragma unroll
        for (int r = 0; r < 4; r++) wgt[t + 64 * r] = e[r] / l;
    }
    __syncthreads();
    const int nc = D / 4;
    const int P = 256 / nc;
    const int c = t % nc, p = t / nc;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    if (p < P) {
        const f32x4* src = reinterpret_cast<const f32x4*>(a.ws + row * S * D) + c;
#pragma unroll 4
        for (int i = p; i < S; i += P) {
            const float w = wgt[i];
            const f32x4 v = ld_global(src + (size_t)i * nc);
            o.x = fmaf(w, v.x, o.x);
            o.y = fmaf(w, v.y, o.y);
            o.z = fmaf(w, v.z, o.z);
            o.w = fmaf(w, v.w, o.w);
        }
    }
    part[t] = o;
    __syncthreads();
    if (t < nc) {
        f32x4 r = part[t];
        for (int q = 1; q < P; q++) {
            const f32x4 w = part[q * nc + t];
            r.x += w.x;
            r.y += w.y;
            r.z += w.z;
            r.w += w.w;
        }
        st_global(reinterpret_cast<f32x4*>(a.out + row * D) + t, r);
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
    case 7: return NJ <= 2 ? attn_kernel<7, NJ <= 2 ? NJ : 2> : nullptr;
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
    (void)cap;
    return (size_t)4 * gm * (D + 4) * sizeof(float);
}

}  // namespace

// Heads per run (GM: 1, 2, 4, 7 or 8, at most 16 f32x4 of query registers), key splits (enough
// workgroups, workspace within its capacity) and the LDS size. Runs of several
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
        // one pass keeps no per-key state in LDS, so any split length fits
        const int min_split = 1;
        const long long blocks = (long long)runs * a->M;
        int want = (int)std::min<long long>(kAttnMaxSplit, (kAttnWantBlocks + blocks - 1) / blocks);
        want = tcap < kAttnSplitMinT ? 1 : std::min(want, (tcap + kAttnMinKeys - 1) / kAttnMinKeys);
        int ns = std::max(min_split, std::max(want, 1));
        // as many splits as the workspace holds
        const int fit = (int)std::min<size_t>(kAttnMaxSplit, kAttnWsBytes / ((size_t)a->M * a->H * (a->D + 2) * sizeof(float)));
        if (ns > fit) ns = std::max(1, fit);
        const size_t ws2 = (size_t)a->M * a->H * ns * (a->D + 2) * sizeof(float);
        const bool few = (long long)runs * a->M * ns < kAttnMinBlocks && gm > 1;
        if (!few && (ns == 1 || ws2 <= kAttnWsBytes)) {
            a->heads_per_run = hpr;
            // seven heads per kv head (Qwen2.5-7B, 28 / 4): an instance without a padding head
            a->gm = gm == 8 && hpr == 7 ? 7 : gm;
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
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.H, a.M), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_kv_store(const float* src, float* dst, int rows, int row_len, int pos0, hipStream_t stream)
{
    const int n4 = rows * row_len / 4;
    hipLaunchKernelGGL(kv_store_kernel, dim3((n4 + 255) / 256), dim3(256), 0, stream, src, dst, n4, row_len / 4, pos0);
    return hipGetLastError();
}

}  // namespace ql
