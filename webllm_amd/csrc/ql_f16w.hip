// Decode GEMV over fp16 weights: y[M, N] = x[M, K] . W[N, K]^T (+ bias), x and y fp32, fp32
// accumulation. This is the tied lm_head / embedding product of the reference
// (src/model/qwen.ts:488-489, src/gpu/kernels/gemm/gemm_gemv_f16.wgsl): W is the fp16 `embed`
// buffer, [N, K] row-major, and at Qwen2.5-0.5B size (151936 x 896, 272 MB) the largest single
// read of a decode step. HBM-bound: every weight byte is read once.
//
// A wave walks 16-row tiles of W. Within a tile, lane (r16, rg) covers rows 4 rg .. 4 rg + 3 and
// the 8-k chunks r16, r16 + 16, ... of K (16 lanes span 128 k, 256 contiguous bytes of a row),
// so one 8-value read of x from LDS feeds four rows' 16-byte weight loads. A wave's jobs (tile,
// 128-k step) stream through a register ring P jobs deep that runs across tiles; at a tile's end
// the 16 lanes of each row add their sums (xor butterfly) and one lane stores. Workgroups stay
// resident and take tiles gw, gw + waves, ... so x is staged in LDS once per workgroup.
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

hipError_t launch_gemv_f16w(const F16wArgs& a, bool fast, int cu_count, hipStream_t stream)
{
    if (!fast) {
        dim3 grid((a.N + 255) / 256, a.M);
        hipLaunchKernelGGL(gemv_f16w_simple_kernel, grid, dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    const int tiles = (a.N + kRowsPerTile - 1) / kRowsPerTile;
    // resident workgroups (4 waves each, two per CU), each walking many tiles with x staged once
    const int grid = std::max(1, std::min((tiles + 3) / 4, 2 * cu_count));
    // up to 4 rows per launch (the decode lm_head is M = 1); more rows take further launches,
    // each reading the weights again
    for (int m0 = 0; m0 < a.M; m0 += 4) {
        F16wArgs p = a;
        p.M = std::min(4, a.M - m0);
        p.x = a.x + (size_t)m0 * a.K;
        p.y = a.y + (size_t)m0 * a.N;
        const size_t lds = gemv_f16w_lds(p.M, a.K);
        if (p.M == 1) hipLaunchKernelGGL(gemv_f16w_kernel<1>, dim3(grid), dim3(256), lds, stream, p);
        else hipLaunchKernelGGL(gemv_f16w_kernel<4>, dim3(grid), dim3(256), lds, stream, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ql
