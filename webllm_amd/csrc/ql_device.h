// Device-side helpers shared by the gfx950 kernels of libqlinear.
//
// GPTQ int4 layout (src/weights/quant.ts:6-12 of the reference): qweight int32 [K/8, N] with the
// low nibble holding the smallest input index; qzeros int32 [K/group, N/8] storing zero - 1;
// scales fp16 [K/group, N]. Dequantized weight W[n,k] = (q - z) * s.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ql {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x2 as_f16x2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// Two nibbles of one packed word as fp16 (1024 + q): nibble `i` in the low half and nibble
// `i + 4` in the high half. 0x6400 is fp16 1024.0, whose ulp is 1, so OR-ing a nibble into the
// mantissa gives exactly 1024 + q.
__device__ __forceinline__ uint32_t magic_pair(uint32_t w, int shift)
{
    return ((w >> shift) & 0x000F000Fu) | 0x64006400u;
}

// The same with the mask and the fp16 1024 pair in registers (mask uniform, magic per lane), so
// the and + or is one v_and_or_b32 (three-operand instructions take no literals on gfx950).
__device__ __forceinline__ uint32_t magic_pair_r(uint32_t w, int shift, uint32_t mask, uint32_t magic)
{
    return ((w >> shift) & mask) | magic;
}

__device__ __forceinline__ f16x8 dequant_word_perm_r(uint32_t w, uint32_t zz, uint32_t ss, uint32_t mask, uint32_t magic)
{
    const f16x2 z = as_f16x2(zz);
    const f16x2 s = as_f16x2(ss);
    const f16x2 p0 = (as_f16x2(magic_pair_r(w, 0, mask, magic)) - z) * s;
    const f16x2 p1 = (as_f16x2(magic_pair_r(w, 4, mask, magic)) - z) * s;
    const f16x2 p2 = (as_f16x2(magic_pair_r(w, 8, mask, magic)) - z) * s;
    const f16x2 p3 = (as_f16x2(magic_pair_r(w, 12, mask, magic)) - z) * s;
    return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// fp16 pair (1024 + z, 1024 + z) for a true zero point z in [1, 16].
__device__ __forceinline__ uint32_t zero_pair(uint32_t z) { return (0x6400u + z) * 0x00010001u; }

// (q - z) for the 8 nibbles of `w`, exact in fp16 (integers in [-16, 15]). Element order is
// k = {0,4,1,5,2,6,3,7}: the MFMA A operand (activations) is staged in the same order, so the
// dot product over k is unchanged.
__device__ __forceinline__ f16x8 centered_nibbles(uint32_t w, uint32_t zz)
{
    const f16x2 z = as_f16x2(zz);
    const f16x2 p0 = as_f16x2(magic_pair(w, 0)) - z;
    const f16x2 p1 = as_f16x2(magic_pair(w, 4)) - z;
    const f16x2 p2 = as_f16x2(magic_pair(w, 8)) - z;
    const f16x2 p3 = as_f16x2(magic_pair(w, 12)) - z;
    return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Order in which centered_nibbles() emits the 8 k offsets of a packed word.
__device__ __forceinline__ int perm_k(int e) { return ((e & 1) << 2) | (e >> 1); }

// Dequantized fp16 weights (q - z) * s for the 8 nibbles of `w`, rounded once to nearest-even.
// (q - z) is exact and the fp16 product of two fp16 values is rounded once, so each element
// equals RNE_f16((q - z) * s) — the value f32ToF16Bits(dequantizeGptqInt4(..)) produces.
// Same {0,4,1,5,2,6,3,7} element order as centered_nibbles().
__device__ __forceinline__ f16x8 dequant_word_perm(uint32_t w, uint32_t zz, uint32_t ss)
{
    const f16x2 z = as_f16x2(zz);
    const f16x2 s = as_f16x2(ss);
    const f16x2 p0 = (as_f16x2(magic_pair(w, 0)) - z) * s;
    const f16x2 p1 = (as_f16x2(magic_pair(w, 4)) - z) * s;
    const f16x2 p2 = (as_f16x2(magic_pair(w, 8)) - z) * s;
    const f16x2 p3 = (as_f16x2(magic_pair(w, 12)) - z) * s;
    return f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Same values in natural k order 0..7 (the [N,K] fp16 arena layout).
__device__ __forceinline__ f16x8 dequant_word_natural(uint32_t w, uint32_t zz, uint32_t ss)
{
    const f16x8 p = dequant_word_perm(w, zz, ss);
    return f16x8{p[0], p[2], p[4], p[6], p[1], p[3], p[5], p[7]};
}

// True zero point of column n from a qzeros word (stored zero + 1, quant.ts:99), or 8.
__device__ __forceinline__ uint32_t zero_of(const uint32_t* qzeros, int g, int n_cols8, int n)
{
    if (!qzeros) return 8u;
    const uint32_t zw = qzeros[(size_t)g * n_cols8 + (n >> 3)];
    return ((zw >> (4 * (n & 7))) & 15u) + 1u;
}

__device__ __forceinline__ f32x4 mfma_16x16x32_f16(f16x8 a, f16x8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

}  // namespace ql
