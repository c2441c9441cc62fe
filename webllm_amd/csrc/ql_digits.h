// Activation digits for the int8-MFMA decode GEMV (shared by the per-linear and the persistent
// sequence kernels).
//
// A group of activations x (one quantization group of one row) is scaled by 2^(E+24), with E the
// group exponent (max|x| * 2^E < 64), rounded to an integer X, and split into four signed base-256
// digits b0..b3 (X = sum_i b_i 256^i). Each digit is one MFMA row, so v_mfma_i32_16x16x64_i8 gives
// exact int32 dot products with the weight nibbles; the group epilogue recombines them in fp32.
#pragma once

#include "ql_device.h"

namespace ql {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Load through the global address space (generic pointers compile to flat loads, which count
// against both the vector-memory and the LDS wait counters). T must be a scalar or a native
// (ext_vector_type) vector: HIP's uint4/uint2 are classes whose copy constructor takes a generic
// reference, which turns the load back into a flat one.
template <typename T>
__device__ __forceinline__ T ld_global(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(1))) T*)(p);
#else
    return *p;   // host pass: never executed
#endif
}
// a streaming load (nontemporal: the line is not kept for reuse)
template <typename T>
__device__ __forceinline__ T ld_stream(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T*)(p));
#else
    return *p;   // host pass: never executed
#endif
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Store through the global address space. A flat store still in flight makes the compiler wait
// for every outstanding vector-memory operation at the next wait it places (it cannot tell flat
// from LDS completions apart), which would drain the weight prefetch after each block's output.
template <typename T>
__device__ __forceinline__ void st_global(T* p, T v)
{
#if defined(__HIP_DEVICE_COMPILE__)
    *(__attribute__((address_space(1))) T*)(p) = v;
#else
    *p = v;      // host pass: never executed
#endif
}

// A pointer as a global-address-space pointer (device pass only; the host pass never runs it).
#if defined(__HIP_DEVICE_COMPILE__)
#define QL_GLOBAL(T, p) ((__attribute__((address_space(1))) T*)(p))
#else
#define QL_GLOBAL(T, p) (p)
#endif


__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c)
{
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Exponent E with max|x| * 2^E < 64 (E = 0 when all values are zero).
__device__ __forceinline__ int group_exponent(float amax)
{
    if (!(amax > 0.f)) return 0;
    int ex;
    (void)frexpf(amax, &ex);                 // amax < 2^ex
    const int E = 6 - ex;
    return E < -100 ? -100 : (E > 100 ? 100 : E);
}

__device__ __forceinline__ void load8(const void* x, int x_dtype, size_t base, float v[8])
{
    if (x_dtype == 0) {
        const f32x4* src = reinterpret_cast<const f32x4*>(static_cast<const float*>(x) + base);
        const f32x4 a0 = ld_global(src), a1 = ld_global(src + 1);
        v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
        v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    } else {
        const f16x8 h = __builtin_bit_cast(
            f16x8, ld_global(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(x) + base)));
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)h[e];
    }
}

// 4x4 byte transpose: out[i] = byte i of (a, b, c, d), packed low to high.
__device__ __forceinline__ void byte_transpose(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                               uint32_t out[4])
{
    const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a0 b0 a1 b1
    const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);   // a2 b2 a3 b3
    const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);
    const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);
    out[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);         // a0 b0 c0 d0
    out[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);         // a1 b1 c1 d1
    out[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
    out[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// Signed base-256 digits of round(v * scale): byte i of the result is digit i.
__device__ __forceinline__ uint32_t digits_of(float v, float scale)
{
    const int X = (int)rintf(v * scale);
    return ((uint32_t)X + 0x00808080u) ^ 0x00808080u;
}

// Activation digits for one 8-k chunk, owned by one of CPG lanes (CPG = group / 8, consecutive
// lanes) that together hold one quantization group of one row. Writes the chunk's digit rows
// (8 bytes each, k order {0,2,4,6,1,3,5,7}) and returns the group's {2^-E, Sx} to every lane.
// Butterfly reductions give every lane identical bits (IEEE addition is commutative).
template <int CPG>
__device__ __forceinline__ float2 prep_chunk(const float v[8], uint2* rows, int row_stride)
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
    const int E = group_exponent(amax);
    const float scale = ldexpf(1.f, E + 24);
    uint32_t ev[4], od[4];
    byte_transpose(digits_of(v[0], scale), digits_of(v[2], scale), digits_of(v[4], scale),
                   digits_of(v[6], scale), ev);
    byte_transpose(digits_of(v[1], scale), digits_of(v[3], scale), digits_of(v[5], scale),
                   digits_of(v[7], scale), od);
#pragma unroll
    for (int i = 0; i < 4; i++) rows[i * row_stride] = uint2{ev[i], od[i]};
    return float2{ldexpf(1.f, -E), sum};
}

}  // namespace ql
