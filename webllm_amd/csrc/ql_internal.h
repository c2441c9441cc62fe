// Host-side interface between the C ABI (ql_api.hip) and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ql {

constexpr int kMaxBatch = 8;
constexpr int kGemvStripCols = 256;  // output columns per GEMV workgroup (4 waves x 64)
constexpr int kGemvMaxM = 16;      // rows handled by the GEMV path (2 MFMA row tiles)
constexpr int kCounterCapacity = 1 << 16;  // split-K arrival counters per context

// One GPTQ linear as the GEMV kernel sees it.
struct GemvLinear {
    const uint32_t* qweight;   // [K/8, N]
    const uint32_t* qzeros;    // [K/group, ceil(N/8)] or nullptr (zero 8)
    const uint16_t* scales;    // [K/group, N] fp16 bits
    const float* bias;         // [N] or nullptr
    const void* x;             // [M, K] f32 or f16
    float* y;                  // [M, N]
    float* partial;            // [split, M, N] (split > 1)
    uint32_t* counters;        // per-strip arrival counters (split > 1), zero between launches
    int N, K, group, split, strips, wg_begin;
};

struct GemvBatch {
    GemvLinear L[kMaxBatch];
    int count;
    int M;
    int x_dtype;
    int wg_total;
};

// GEMV planning shared by ql_plan_linear and the launcher.
struct GemvShape {
    int strips, groups, split, waves;
};
GemvShape gemv_shape(int M, int N, int K, int group);
bool gemv_fast_ok(int M, int N, int K, int group);
uint64_t gemv_partial_bytes(int M, int N, int split);

hipError_t launch_gemv_batch(const GemvBatch& b, hipStream_t stream);
hipError_t launch_gemv_simple(const GemvLinear& L, int M, int x_dtype, hipStream_t stream);

// GEMM (M > 16): y = f16(x) * f16(W)^T, fp32 accumulate.
struct GemmArgs {
    const uint32_t* qweight;
    const uint32_t* qzeros;
    const uint16_t* scales;
    const float* bias;
    const void* x;
    float* y;
    int M, N, K, group, x_dtype;
};
bool gemm_fast_ok(int M, int N, int K, int group);
void gemm_grid(int M, int N, int* gx, int* gy, int* block);
hipError_t launch_gemm(const GemmArgs& a, hipStream_t stream);
hipError_t launch_gemm_simple(const GemmArgs& a, hipStream_t stream);

// load-time unpack to fp16 [N, K]
struct UnpackArgs {
    const uint32_t* qweight;
    const uint32_t* qzeros;
    const uint16_t* scales;
    void* out;                 // fp16 [N,K] (launch_unpack) or fp32 [N,K] (launch_unpack_f32)
    int N, K, group;
};
hipError_t launch_unpack(const UnpackArgs& a, bool fast, hipStream_t stream);
hipError_t launch_unpack_f32(const UnpackArgs& a, hipStream_t stream);

}  // namespace ql
