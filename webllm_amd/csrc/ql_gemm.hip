// Prefill GEMM for GPTQ int4 linears, M > 16: y[M,N] = f16(x)[M,K] * f16(W)[N,K]^T (+ bias),
// fp32 accumulation. Same arithmetic as the reference's M > 1 path, gemm_nt_f16_from_f32.wgsl
// (x rounded to fp16 on load, fp16 weights from the load-time dequant), but the weights are
// dequantized from the packed int4 tiles into LDS inside the kernel, bit-identical to the
// load-time fp16 arena (dequant_word_perm in ql_device.h).
//
// Tile: 64 (M) x 64 (N) x 32 (K) per workgroup of 4 waves (2 x 2), each wave 32 x 32 as 2 x 2
// v_mfma_f32_16x16x32_f16 tiles. One K step is 4 packed qweight rows, which is one MFMA K block;
// each packed word dequantizes to exactly one lane's B fragment (8 k of one column), stored to
// LDS as 16 bytes. Activations are staged to LDS in the same permuted k order. Global loads for
// step i+1 are issued before the MFMAs of step i.
#include "ql_device.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int BM = 64;
constexpr int BN = 64;

struct Stage {
    uint4 a;       // 8 activations of one row (fp16, natural order) or f32 pair below
    float4 af0, af1;
    uint32_t w;    // one packed word
    uint32_t zz, ss;
};

__device__ __forceinline__ void load_stage(const GemmArgs& g, int m0, int n0, int k0, Stage& st)
{
    const int t = threadIdx.x;
    // activations: row r, chunk kq
    const int r = t >> 2, kq = t & 3;
    const int m = m0 + r;
    if (m < g.M) {
        if (g.x_dtype == 0) {
            const float4* src = reinterpret_cast<const float4*>(
                static_cast<const float*>(g.x) + (size_t)m * g.K + k0 + 8 * kq);
            st.af0 = src[0];
            st.af1 = src[1];
        } else {
            st.a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(g.x) +
                                                   (size_t)m * g.K + k0 + 8 * kq);
        }
    } else {
        st.a = uint4{0u, 0u, 0u, 0u};
        st.af0 = float4{0.f, 0.f, 0.f, 0.f};
        st.af1 = st.af0;
    }
    // weights: packed row kw, column c
    const int kw = t >> 6, c = t & 63;
    const int n = n0 + c;
    if (n < g.N) {
        const int p = (k0 >> 3) + kw;
        const int grp = k0 / g.group;
        st.w = g.qweight[(size_t)p * g.N + n];
        st.zz = zero_pair(zero_of(g.qzeros, grp, (g.N + 7) >> 3, n));
        st.ss = (uint32_t)g.scales[(size_t)grp * g.N + n] * 0x10001u;
    } else {
        st.w = 0u;
        st.zz = zero_pair(8u);
        st.ss = 0u;
    }
}

__device__ __forceinline__ void store_stage(const GemmArgs& g, const Stage& st, uint4* As, uint4* Bs)
{
    const int t = threadIdx.x;
    const int r = t >> 2, kq = t & 3;
    f16x8 h;
    if (g.x_dtype == 0) {
        const float v[8] = {st.af0.x, st.af0.y, st.af0.z, st.af0.w,
                            st.af1.x, st.af1.y, st.af1.z, st.af1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = (_Float16)v[perm_k(e)];
    } else {
        const f16x8 nat = __builtin_bit_cast(f16x8, st.a);
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = nat[perm_k(e)];
    }
    As[kq * BM + r] = __builtin_bit_cast(uint4, h);
    const int kw = t >> 6, c = t & 63;
    Bs[kw * BN + c] = __builtin_bit_cast(uint4, dequant_word_perm(st.w, st.zz, st.ss));
}

__global__ __launch_bounds__(256) void gemm_mfma_kernel(const GemmArgs g)
{
    __shared__ uint4 As[4 * BM];
    __shared__ uint4 Bs[4 * BN];
    const int n0 = blockIdx.x * BN;
    const int m0 = blockIdx.y * BM;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int j = lane & 15, kq = lane >> 4;

    f32x4 c[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) c[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    Stage st;
    load_stage(g, m0, n0, 0, st);
    for (int k0 = 0; k0 < g.K; k0 += 32) {
        store_stage(g, st, As, Bs);
        __syncthreads();
        if (k0 + 32 < g.K) load_stage(g, m0, n0, k0 + 32, st);
        f16x8 af[2], bf[2];
#pragma unroll
        for (int tm = 0; tm < 2; tm++)
            af[tm] = __builtin_bit_cast(f16x8, As[kq * BM + wm * 32 + tm * 16 + j]);
#pragma unroll
        for (int tn = 0; tn < 2; tn++)
            bf[tn] = __builtin_bit_cast(f16x8, Bs[kq * BN + wn * 32 + tn * 16 + j]);
#pragma unroll
        for (int tm = 0; tm < 2; tm++)
#pragma unroll
            for (int tn = 0; tn < 2; tn++) c[tm][tn] = mfma_16x16x32_f16(af[tm], bf[tn], c[tm][tn]);
        __syncthreads();
    }

#pragma unroll
    for (int tm = 0; tm < 2; tm++) {
#pragma unroll
        for (int tn = 0; tn < 2; tn++) {
            const int n = n0 + wn * 32 + tn * 16 + j;
            if (n >= g.N) continue;
            const float bias = g.bias ? g.bias[n] : 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 32 + tm * 16 + 4 * kq + r;
                if (m < g.M) g.y[(size_t)m * g.N + n] = g.bias ? c[tm][tn][r] + bias : c[tm][tn][r];
            }
        }
    }
}

}  // namespace

bool gemm_fast_ok(int M, int N, int K, int group)
{
    return M > 0 && N > 0 && K > 0 && K % 32 == 0 && group > 0 && group % 32 == 0 &&
           K % group == 0;
}

void gemm_grid(int M, int N, int* gx, int* gy, int* block)
{
    *gx = (N + BN - 1) / BN;
    *gy = (M + BM - 1) / BM;
    *block = 256;
}

hipError_t launch_gemm(const GemmArgs& a, hipStream_t stream)
{
    int gx, gy, block;
    gemm_grid(a.M, a.N, &gx, &gy, &block);
    hipLaunchKernelGGL(gemm_mfma_kernel, dim3(gx, gy), dim3(block), 0, stream, a);
    return hipGetLastError();
}

}  // namespace ql
