// Decode GEMV over fp16 weights: y[M, N] = x[M, K] . W[N, K]^T (+ bias), x and y fp32, fp32
// accumulation. This is the tied lm_head / embedding product of the reference
// (src/model/qwen.ts:488-489, src/gpu/kernels/gemm/gemm_gemv_f16.wgsl): W is the fp16 `embed`
// buffer, [N, K] row-major, and at Qwen2.5-0.5B size (151936 x 896, 272 MB) the largest single
// read of a decode step. HBM-bound: every weight byte is read once per launch. Two kernels: an
// fp32-FMA one for a single row (below) and a matrix-core one for 2..16 rows per launch.
//
// FMA kernel. A wave walks 16-row tiles of W. Within a tile, lane (r16, rg) covers rows
// 4 rg .. 4 rg + 3 and the 8-k chunks r16, r16 + 16, ... of K (16 lanes span 128 k, 256
// contiguous bytes of a row), so one 8-value read of x from LDS feeds four rows' 16-byte weight
// loads. A wave's jobs (tile, 128-k step) stream through a register ring P jobs deep that runs
// across tiles; at a tile's end the 16 lanes of each row add their sums (xor butterfly) and one
// lane stores. Workgroups stay resident and take tiles gw, gw + waves, ... so x is staged in LDS
// once per workgroup.
#include <algorithm>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kRowsPerTile = 16;
constexpr int kStepK = 128;          // k per job (16 lanes x 8)
constexpr int kP = 4;                // jobs in flight per wave

template <int MT>
__global__ __launch_bounds__(256) void gemv_f16w_kernel(const F16wArgs a)
{
    extern __shared__ float xs[];    // x [M][K]
    const int M = a.M, K = a.K, N = a.N;
    for (int i = threadIdx.x * 4; i < M * K; i += 256 * 4)
        *reinterpret_cast<f32x4*>(xs + i) = ld_global(reinterpret_cast<const f32x4*>(a.x + i));
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, rg = lane >> 4;
    const int S = K / kStepK;                                  // jobs per tile
    const int tiles = (N + kRowsPerTile - 1) / kRowsPerTile;
    const int gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
    const int ntw = gw < tiles ? (tiles - 1 - gw) / nw + 1 : 0;   // this wave's tiles
    const int njobs = ntw * S;
    const char* wb = reinterpret_cast<const char*>(a.w);
    const uint32_t rowb = (uint32_t)K * 2u;

    // fetch cursor: (tile, step) of the next job to load; past the end it stays on the last job
    int ft = gw, fs = 0, fq = 0;
    u32x4 ring[kP][4];
    float rbias[kP];                 // bias of row 4 rg + (r16 & 3) of the job's tile
    // without a bias, any valid float (never added)
    const float* bp = a.bias ? a.bias : reinterpret_cast<const float*>(a.x);
    auto fetch = [&](int d) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = min(ft * kRowsPerTile + 4 * rg + i, N - 1);
            const uint64_t off = (uint64_t)n * rowb + (uint64_t)(fs * kStepK + 8 * r16) * 2u;
            ring[d][i] = ld_global(reinterpret_cast<const u32x4*>(wb + off));
        }
        rbias[d] = ld_global(bp + (a.bias ? min(ft * kRowsPerTile + 4 * rg + (r16 & 3), N - 1) : 0));
        if (fq + 1 < njobs) {
            fq++;
            if (++fs == S) {
                fs = 0;
                ft += nw;
            }
        }
    };
    float acc[4][MT];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[i][m] = 0.f;

    if (njobs == 0) return;
#pragma unroll
    for (int d = 0; d < kP; d++) fetch(d);
    int ct = gw, cs = 0;                                       // consume cursor
    const int njobs_p = (njobs + kP - 1) / kP * kP;
    for (int q = 0; q < njobs_p; q += kP) {
#pragma unroll
        for (int d = 0; d < kP; d++) {
            if (q + d < njobs) {
                const int k0 = cs * kStepK + 8 * r16;
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    if (m >= M) continue;
                    const f32x4 x0 = *reinterpret_cast<const f32x4*>(xs + m * K + k0);
                    const f32x4 x1 = *reinterpret_cast<const f32x4*>(xs + m * K + k0 + 4);
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const f16x8 w = __builtin_bit_cast(f16x8, ring[d][i]);
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[i][m] = fmaf(xv[e], (float)w[e], acc[i][m]);
                    }
                }
                if (++cs == S) {
                    // the tile's rows: the 16 lanes of each row add their sums
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int m = 0; m < MT; m++) {
                            if (m >= M) continue;
                            float v = acc[i][m];
                            v += __shfl_xor(v, 8);
                            v += __shfl_xor(v, 4);
                            v += __shfl_xor(v, 2);
                            v += __shfl_xor(v, 1);
                            // every lane holds the row's sum; lane r16 = i stores row 4 rg + i with
                            // the bias its ring slot carries (no load on this path)
                            const int n = ct * kRowsPerTile + 4 * rg + i;
                            if (r16 == i && n < N) st_global(a.y + (size_t)m * N + n, a.bias ? v + rbias[d] : v);
                            acc[i][m] = 0.f;
                        }
                    cs = 0;
                    ct += nw;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    asm volatile("" ::"v"(ring[d][i].x), "v"(ring[d][i].y), "v"(ring[d][i].z), "v"(ring[d][i].w));
                asm volatile("" ::"v"(rbias[d]));
            }
            fetch(d);
        }
    }
}

// The matrix-core form, 2..16 rows of x per pass. Each wave walks 16-column tiles of y (16 rows of
// W) over all of K in steps of 32: for step t, lane (i, g) = (lane % 16, lane / 16) loads the 16
// bytes W[n0 + i][32 t + 8 g .. + 7], which is as it stands the v_mfma_f32_16x16x32_f16 A fragment
// of W (no conversion). x enters as the B fragments of two fp16 parts per 8 values, scaled per row
// and step: with s such that max|x[m][32 t .. 32 t + 31]| 2^s lies in [2^14, 2^15),
// hi = f16(x 2^s) and lo = f16(x 2^s - hi), which keep about 22 bits of every value (absolute
// error below 2^-22 of the step's max|x|). A step's two MFMAs (lo, then hi onto it) start from
// zero and its 4 results per lane are added into fp32 accumulators as fma(d, 2^-s, acc) by the
// VALU, so the matrix unit never carries the long sum. At a tile's end lane (i, g) holds
// y[i][n0 + 4 g .. + 3] (+ bias), one 16-byte store where N allows. LDS holds x's fragments as
// [t][g][row] 16-byte units, hi then lo (zeros past K), then a zero unit for the lanes of rows
// past M, then the scales 2^-s as [t][row], all written in one pass per workgroup. The first weight
// loads are issued before x is staged, and each step reads the next step's fragments before its own
// MFMAs. Workgroups stay resident and take tiles gw, gw + waves, ...
constexpr int kMfRows = 16;           // rows of x per pass (the MFMA tile height)
constexpr int kMfP = 16;              // weight fragments in flight per wave
constexpr size_t kMfLdsMax = 64u << 10;

// quad broadcast: every lane of a group of 4 takes lane r's value
template <int R>
__device__ __forceinline__ float quad_bcast(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), R * 0x55, 0xF, 0xF, false));
}

// LDS bytes of the matrix-core form for M rows: per 32-k step and row 8 fragment units and a
// scale, and the zero unit
size_t gemv_f16w_mfma_lds(int M, int K) { return (size_t)((K + 31) / 32) * M * (8 * 16 + 4) + 16; }

// KFULL: K % 32 == 0 (every fragment lies inside its row); BIAS: a bias vector is given.
template <bool KFULL, bool BIAS>
__global__ __launch_bounds__(256, 2) void gemv_f16w_mfma_kernel(const F16wArgs a)
{
    extern __shared__ u32x4 xu[];     // hi units [S * 4][M], lo units, zero unit, scales [S][M]
    const int M = a.M, K = a.K, N = a.N;
    const int S = (K + 31) / 32;               // steps per tile
    const int U = S * 4 * M;
    float* scl = reinterpret_cast<float*>(xu + 2 * U + 1);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    const int tiles = (N + 15) / 16;
    const int gw = blockIdx.x * 4 + wave, nw = gridDim.x * 4;
    const int ntw = gw < tiles ? (tiles - 1 - gw) / nw + 1 : 0;
    const int njobs = ntw * S;
    const char* wb = reinterpret_cast<const char*>(a.w);
    const uint64_t rowb = (uint64_t)K * 2u;

    int ft = gw, fs = 0, fq = 0;      // fetch cursor (stays on the last step past the end)
    u32x4 ring[kMfP];
    float rbias[kMfP];                // bias of column n0 + 4 g + (i16 & 3) of the step's tile
    auto fetch = [&](int d) {
        const int n = min(ft * 16 + i16, N - 1);
        // past K: a valid address; the fragment is zeroed where it is consumed
        const int k = KFULL ? fs * 32 + 8 * g : min(fs * 32 + 8 * g, K - 8);
        ring[d] = ld_global(reinterpret_cast<const u32x4*>(wb + (uint64_t)n * rowb + (uint64_t)k * 2u));
        if (BIAS) rbias[d] = ld_global(a.bias + min(ft * 16 + 4 * g + (i16 & 3), N - 1));
        if (fq + 1 < njobs) {
            fq++;
            if (++fs == S) {
                fs = 0;
                ft += nw;
            }
        }
    };
    // the first weight fragments are in flight while x is staged
#pragma unroll
    for (int d = 0; d < kMfP; d++) fetch(d);

    // staging: one (row, step) per thread: 32 values, their scale, 4 hi and 4 lo units
    for (int w = tid; w < S * M; w += 256) {
        const int m = w % M, t = w / M;
        const float* src = a.x + (size_t)m * K + 32 * t;
        f32x4 v[8];
        float mx = 0.f;
#pragma unroll
        for (int h = 0; h < 8; h++) {
            v[h] = (KFULL || 32 * t + 4 * h < K) ? ld_global(reinterpret_cast<const f32x4*>(src + 4 * h))
                                                 : f32x4{0.f, 0.f, 0.f, 0.f};
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[h].x), fabsf(v[h].y)), fmaxf(fabsf(v[h].z), fabsf(v[h].w))));
        }
        // s = 14 - floor(log2 max|x|); 0 for an all-zero or non-finite step
        const int sh = (mx > 0.f && mx <= 3.4028235e38f) ? 14 - ilogbf(mx) : 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const f32x4& vv = v[2 * q + (e >> 1)];
                const f32x2 xs = (e & 1) ? f32x2{ldexpf(vv.z, sh), ldexpf(vv.w, sh)}
                                         : f32x2{ldexpf(vv.x, sh), ldexpf(vv.y, sh)};
                const f16x2 hh = __builtin_convertvector(xs, f16x2);
                const f32x2 r = xs - __builtin_convertvector(hh, f32x2);
                hw[e] = __builtin_bit_cast(uint32_t, hh);
                lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, f16x2));
            }
            const int u = (t * 4 + q) * M + m;
            xu[u] = u32x4{hw[0], hw[1], hw[2], hw[3]};
            xu[U + u] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        }
        scl[t * M + m] = ldexpf(1.f, -sh);
    }
    if (tid == 0) xu[2 * U] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();

    if (njobs == 0) return;
    const bool live = i16 < M;                 // lane's x row (the B column) exists
    // byte addresses for step t: hi unit lbase + t lstep (lo: + loff), scale sbase + t sstep; lanes
    // of rows past M read the zero unit for all three
    const char* xb = reinterpret_cast<const char*>(xu);
    const uint32_t zero_b = (uint32_t)(2 * U) * 16u;
    const uint32_t lbase = live ? (uint32_t)(g * M + i16) * 16u : zero_b;
    const uint32_t lstep = live ? (uint32_t)(4 * M) * 16u : 0u;
    const uint32_t loff = live ? (uint32_t)U * 16u : 0u;
    const uint32_t sbase = live ? zero_b + 16u + (uint32_t)i16 * 4u : zero_b;
    const uint32_t sstep = live ? (uint32_t)M * 4u : 0u;
    f16x8 xh, xl;                              // fragments and scale of the next step to consume
    float xs;
    auto xread = [&](int t) {
        const uint32_t ah = lbase + (uint32_t)t * lstep;
        xh = *reinterpret_cast<const f16x8*>(xb + ah);
        xl = *reinterpret_cast<const f16x8*>(xb + ah + loff);
        xs = *reinterpret_cast<const float*>(xb + sbase + (uint32_t)t * sstep);
    };
    xread(0);

    const bool vec_store = N % 4 == 0;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    int ct = gw, cs = 0;
    const int njobs_p = (njobs + kMfP - 1) / kMfP * kMfP;
    for (int q = 0; q < njobs_p; q += kMfP) {
#pragma unroll
        for (int d = 0; d < kMfP; d++) {
            if (q + d < njobs) {
                const f16x8 ch = xh, cl = xl;
                const float sc = xs;
                xread(cs + 1 == S ? 0 : cs + 1);
                f16x8 wf = __builtin_bit_cast(f16x8, ring[d]);
                if (!KFULL && cs * 32 + 8 * g >= K) wf = f16x8{};
                f32x4 dd = mfma_16x16x32_f16(wf, cl, f32x4{0.f, 0.f, 0.f, 0.f});
                dd = mfma_16x16x32_f16(wf, ch, dd);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[r] = fmaf(dd[r], sc, acc[r]);
                if (++cs == S) {
                    // acc[r] = y[m = i16][n0 + 4 g + r]
                    const int n = ct * 16 + 4 * g;
                    f32x4 v = acc;
                    if (BIAS) {
                        v[0] += quad_bcast<0>(rbias[d]);
                        v[1] += quad_bcast<1>(rbias[d]);
                        v[2] += quad_bcast<2>(rbias[d]);
                        v[3] += quad_bcast<3>(rbias[d]);
                    }
                    float* yr = a.y + (size_t)i16 * N;
                    if (live) {
                        if (vec_store && n + 3 < N) {
                            st_global(reinterpret_cast<f32x4*>(yr + n), v);
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; r++)
                                if (n + r < N) st_global(yr + n + r, v[r]);
                        }
                    }
                    acc = f32x4{0.f, 0.f, 0.f, 0.f};
                    cs = 0;
                    ct += nw;
                }
            } else {
                asm volatile("" ::"v"(ring[d].x), "v"(ring[d].y), "v"(ring[d].z), "v"(ring[d].w));
                if (BIAS) asm volatile("" ::"v"(rbias[d]));
            }
            fetch(d);
        }
    }
}

// Any K (and any alignment): one lane per output, k ascending.
__global__ __launch_bounds__(256) void gemv_f16w_simple_kernel(const F16wArgs a)
{
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int m = blockIdx.y;
    if (n >= a.N) return;
    const uint16_t* row = a.w + (size_t)n * a.K;
    const float* x = a.x + (size_t)m * a.K;
    float acc = 0.f;
    for (int k = 0; k < a.K; k++) acc = fmaf(x[k], (float)__builtin_bit_cast(_Float16, row[k]), acc);
    if (a.bias) acc += a.bias[n];
    a.y[(size_t)m * a.N + n] = acc;
}

}  // namespace

size_t gemv_f16w_lds(int M, int K) { return (size_t)M * K * sizeof(float); }

bool gemv_f16w_fast_ok(int M, int N, int K)
{
    return M >= 1 && N > 0 && K > 0 && K % kStepK == 0 && gemv_f16w_lds(4, K) <= (96u << 10);
}

// The embedding lookup (embedding_f16.wgsl): out[r, :] = f32(W[tokens[r], :]). A workgroup covers
// 2048 values of one row, 8 per lane (one 16-byte load, two 16-byte stores) where the row length
// and offsets allow, else one value per load. A token id >= vocab writes zeros.
__global__ __launch_bounds__(256) void embed_rows_kernel(const EmbedArgs a)
{
    const int r = blockIdx.y;
    const uint32_t tok = __builtin_amdgcn_readfirstlane(a.tokens[r]);
    const bool ok = tok < (uint32_t)a.vocab;
    const uint16_t* src = a.w + (size_t)(ok ? tok : 0u) * a.D;
    float* dst = a.out + (size_t)r * a.D;
    if (a.vec) {
        const int i = (blockIdx.x * 256 + threadIdx.x) * 8;
        if (i < a.D) {
            f32x4 lo = f32x4{0.f, 0.f, 0.f, 0.f}, hi = lo;
            if (ok) {
                const f16x8 h = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(src + i));
                lo = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
                hi = f32x4{(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
            }
            *reinterpret_cast<f32x4*>(dst + i) = lo;
            *reinterpret_cast<f32x4*>(dst + i + 4) = hi;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int i = blockIdx.x * 2048 + e * 256 + threadIdx.x;
            if (i < a.D) dst[i] = ok ? (float)__builtin_bit_cast(_Float16, src[i]) : 0.f;
        }
    }
}

hipError_t launch_embed_rows(const EmbedArgs& a, hipStream_t stream)
{
    hipLaunchKernelGGL(embed_rows_kernel, dim3((a.D + 2047) / 2048, a.rows), dim3(256), 0, stream, a);
    return hipGetLastError();
}

// rows of x per pass of the matrix-core form that fit its LDS budget (0: K too long for one row)
static int gemv_f16w_mfma_rows(int K)
{
    const size_t per_row = gemv_f16w_mfma_lds(1, K) - 16;
    return (int)std::min<size_t>(kMfRows, (kMfLdsMax - 16) / per_row);
}

hipError_t launch_gemv_f16w(const F16wArgs& a, bool fast, int cu_count, hipStream_t stream)
{
    // one row (the decode lm_head) keeps the fp32-FMA kernel, measured faster there; two or more
    // rows take the matrix-core form, which reads the weights once per 16 rows
    const int R = gemv_f16w_mfma_rows(a.K);
    if (R >= 1 && a.K % 8 == 0 && !(fast && a.M == 1)) {
        const int tiles = (a.N + 15) / 16;
        // resident workgroups (4 waves each, two per CU), each walking many tiles with x staged once
        const int grid = std::max(1, std::min((tiles + 3) / 4, 2 * cu_count));
        for (int m0 = 0; m0 < a.M; m0 += R) {
            F16wArgs p = a;
            p.M = std::min(R, a.M - m0);
            p.x = a.x + (size_t)m0 * a.K;
            p.y = a.y + (size_t)m0 * a.N;
            const size_t lds = gemv_f16w_mfma_lds(p.M, a.K);
            const bool kfull = a.K % 32 == 0;
            if (kfull && a.bias) hipLaunchKernelGGL((gemv_f16w_mfma_kernel<true, true>), dim3(grid), dim3(256), lds, stream, p);
            else if (kfull) hipLaunchKernelGGL((gemv_f16w_mfma_kernel<true, false>), dim3(grid), dim3(256), lds, stream, p);
            else if (a.bias) hipLaunchKernelGGL((gemv_f16w_mfma_kernel<false, true>), dim3(grid), dim3(256), lds, stream, p);
            else hipLaunchKernelGGL((gemv_f16w_mfma_kernel<false, false>), dim3(grid), dim3(256), lds, stream, p);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (!fast) {
        dim3 grid((a.N + 255) / 256, a.M);
        hipLaunchKernelGGL(gemv_f16w_simple_kernel, grid, dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    const int tiles = (a.N + kRowsPerTile - 1) / kRowsPerTile;
    // resident workgroups (4 waves each, two per CU), each walking many tiles with x staged once
    const int grid = std::max(1, std::min((tiles + 3) / 4, 2 * cu_count));
    for (int m = 0; m < a.M; m++) {
        F16wArgs p = a;
        p.M = 1;
        p.x = a.x + (size_t)m * a.K;
        p.y = a.y + (size_t)m * a.N;
        hipLaunchKernelGGL(gemv_f16w_kernel<1>, dim3(grid), dim3(256), gemv_f16w_lds(1, a.K), stream, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ql
