// Column strips for decode batches of M = 5..16 rows on weights streamed from HBM: the strip
// launch of ql_strip.hip for plans without padding, with an arithmetic laid out for few vector
// instructions per job.
//
// Same work split as strip_kernel (a workgroup owns strips of 8 whole 64-column blocks over all
// of K, one block per wave; K in chunks of 4 quantization groups staged as activation digits in
// double-buffered LDS; a 2-deep register ring of packed weights per wave), restricted to plans in
// which every linear has a multiple of 4 groups of 128 and a multiple of 512 columns, so every
// chunk has 4 jobs for every wave and no position is padding. What differs:
// * M 9..16 (L = 1): the four base-256 digits of every activation laid out digit-major: tile d
//   holds digit d of rows 0..15, so a lane holds the four digit sums of its 4 rows x 4 columns and
//   recombines them in its own registers; M 5..8 (L = 0): rows 4m + d in two 16-row tiles, as
//   strip_kernel. (Three digits, 24 bits of each group's range, measured 1.9e-5 against the
//   1e-5 + 1e-4 |ref| bar on the 7B down projections (K = 18944), so four are kept.)
// * one instruction per nibble half: the even-k nibbles are w & 0x0F0F0F0F (n, 0..15), the odd-k
//   ones (w ^ 0x88888888) & 0xF0F0F0F0 (16 (n - 8) as a signed byte, one v_bitop3_b32), whose
//   activation digits are formed at a 16 times smaller scale (26 bits of the chunk's range
//   instead of 30); the offset -8 joins the zero-point term through the odd k's own row sums;
// * one exponent per (chunk, row) instead of per (group, row): a chunk's jobs accumulate
//   s * digits in the exponent's units (v_fma_mix_f32 on the fp16 scale as loaded, no
//   conversion), and the chunk's sums join the outputs with one multiply-add by 2^-(E+8);
// * the zero-point term -s*(z+1)*sum(x_even) - s*(z-7)*sum(x_odd) goes through two
//   v_mfma_f32_16x16x4_f32 per column quarter and chunk (k = the chunk's 4 groups: A = the
//   groups' row sums, B = the lane's columns' -s*(z+1) or -s*(z-7)), which start the chunk's sums
//   (L = 1) instead of one FMA per output and job;
// * every LDS address is a lane constant plus a compile-time offset, and positions never branch;
// * the activation digits are computed once per (linear, chunk) by wide_digits_kernel, launched
//   just before, as images of the LDS chunk buffer; each strip's workgroup copies the image
//   instead of computing the digits itself (every strip of a linear used to recompute them: about
//   46 of the 7B step's 255 vector instructions per job at M=16). The 7B step at M=16: 792-799
//   against 827-832 us (the digits launch itself 24.7 us); M=8 unchanged within noise.
// Each job's epilogue is then, per output, two integer recombinations, two conversions, one FMA
// for the digit value and one mixed-precision multiply-add with the fp16 scale.
#include <type_traits>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kCG = kStripChunkGroups;   // quantization groups per chunk (4)
constexpr int kCols = kSeqTileCols;      // 64 output columns per block
constexpr int kW = 8;                    // waves: one block each
constexpr int kThreads = 64 * kW;
// M 9..16: each column quarter's MFMAs and epilogue form a scheduling region of their own (the
// 7B step at M=16 826-831 against 839-846 us with one region per job; 192 against 208 VGPRs)
#ifndef QL_WIDE_QREGION
#define QL_WIDE_QREGION 1
#endif
constexpr int kNB = 2;                   // 64-k blocks per 128-k group
constexpr int kBlocks = 8;               // blocks per strip
static_assert(kCG == 4, "chunks of 4 groups");

template <typename T>
__device__ __forceinline__ T tab(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    // tables are written once before any launch: constant address space, scalar loads
    return *(const __attribute__((address_space(4))) T*)(reinterpret_cast<uintptr_t>(p));
#else
    return *p;
#endif
}

__device__ __forceinline__ int sreg(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <typename T>
__device__ __forceinline__ const T* sptr(const T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const T*>((hi << 32) | lo);
}

// Buffer loads: a scalar resource per tensor, a 32-bit lane offset and a scalar offset, so no
// lane computes a 64-bit address. kNT: the streaming (nontemporal) policy.
constexpr int kNT = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
}

__device__ __forceinline__ f32x4 mfma_f32_4(float a, float b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Four digits per activation. L = 0: digit row 4m + d (m < 8) in tile m / 4 at row 4 (m % 4) + d;
// L = 1: tile d, row m (m < 16).
template <int L>
struct WideLayout {
    static constexpr int kDigits = 4;
    static constexpr int kTiles = L == 0 ? 2 : 4;       // 16-row tiles per (64-k block, quarter)
    static constexpr int kMaxM = L == 0 ? 8 : 16;
    static constexpr int kTileB = 16 * 16;              // 16 rows of 16 bytes
    static constexpr int kKqB = kTiles * kTileB;        // per lane group kq (16 k of the block)
    static constexpr int kBbB = 4 * kKqB;               // per 64-k block
    static constexpr int kGB = kNB * kBbB;              // per group
    static constexpr int kDigB = kCG * kGB;             // digits of one chunk
    // {sum x over even k, over odd k} per (group, row < 16), then 2^-(E+8) and 2^(E+8) per row
    static constexpr int kGstB = kCG * 16 * 8 + 2 * 16 * 4;
    static constexpr int kBufB = kDigB + kGstB;         // one chunk buffer
    static constexpr int kBiasB = 2 * kBlocks * kCols * 4;   // two strips' bias
    static constexpr int kZB = L == 0 ? kW * 16 * kCols * 4 : 0;   // zero-term transposition (L = 0)
    static constexpr int kLds = 2 * kBufB + kBiasB + kZB;
    // 8-value staging items per thread and chunk: kCG groups x kMaxM rows x 16 pieces of 8 k
    static constexpr int kH = (kCG * kMaxM * 16 + kThreads - 1) / kThreads;
    // a chunk buffer as 16-byte units, and the units each thread copies from its digit image
    static constexpr int kUnits = kBufB / 16;
    static constexpr int kHI = (kUnits + kThreads - 1) / kThreads;
    static_assert(kBufB % 16 == 0, "whole 16-byte units");
};

// Reductions over the 16 lanes of a row by DPP row rotations (every lane ends with the combined
// value; the sum's order is fixed per lane, so each run gives the same bits).
template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ void row_sums(float& a, float& b)
{
    // row_ror:8, row_ror:4, quad_perm [2,3,0,1], quad_perm [1,0,3,2]
    a += dpp<0x128>(a); b += dpp<0x128>(b);
    a += dpp<0x124>(a); b += dpp<0x124>(b);
    a += dpp<0x4E>(a);  b += dpp<0x4E>(b);
    a += dpp<0xB1>(a);  b += dpp<0xB1>(b);
}
// max over the wave's 64 lanes (exact; every lane ends with it)
__device__ __forceinline__ float wave_max(float a)
{
    a = fmaxf(a, dpp<0x128>(a));
    a = fmaxf(a, dpp<0x124>(a));
    a = fmaxf(a, dpp<0x4E>(a));
    a = fmaxf(a, dpp<0xB1>(a));
    a = fmaxf(a, __shfl_xor(a, 16));
    return fmaxf(a, __shfl_xor(a, 32));
}

// round(v) as an integer, halves rounded up (v_cvt_rpi_i32_f32: one instruction)
__device__ __forceinline__ int round_int(float v)
{
    int r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Signed base-256 digits of round(v * scale): byte i of the result is digit i.
__device__ __forceinline__ uint32_t digits4_of(float v, float scale)
{
    return ((uint32_t)round_int(v * scale) + 0x00808080u) ^ 0x00808080u;
}

// One wave stages one row's chunk: lane 16 gg + c holds the 8 values of piece c (k 8c .. 8c+7) of
// group gg. Returns the chunk's exponent E (max|x| * 2^E < 64 over the row's 512 values).
__device__ __forceinline__ int chunk_exponent(const float v[8])
{
    const float amax = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                             fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
    return group_exponent(wave_max(amax));
}

// Digits of one 8-k piece owned by one of 16 consecutive lanes (one DPP row) that hold one
// (group, row): for each of the four digits, its 16-byte-row halves (k order {0,2,4,6,1,3,5,7}) in
// row[d], and the group's {sum x over even k, over odd k} in sums. Even k: digits of
// round(x 2^(E+24)) (the weight operand is the nibble n); odd k: of round(x 2^(E+20)) (the weight
// operand is 16 (n - 8)), so both products carry 2^(E+24).
struct PieceDigits {
    uint2 row[4];
    float2 sums;
};
__device__ __forceinline__ PieceDigits piece_digits(const float v[8], int E)
{
    float se = (v[0] + v[2]) + (v[4] + v[6]);
    float so = (v[1] + v[3]) + (v[5] + v[7]);
    row_sums(se, so);
    const float scale = ldexpf(1.f, E + 24);
    const float sodd = ldexpf(1.f, E + 20);
    uint32_t ev[4], od[4];
    byte_transpose(digits4_of(v[0], scale), digits4_of(v[2], scale), digits4_of(v[4], scale),
                   digits4_of(v[6], scale), ev);
    byte_transpose(digits4_of(v[1], sodd), digits4_of(v[3], sodd), digits4_of(v[5], sodd),
                   digits4_of(v[7], sodd), od);
    PieceDigits p;
#pragma unroll
    for (int i = 0; i < 4; i++) p.row[i] = uint2{ev[i], od[i]};
    p.sums = float2{se, so};
    return p;
}

// Where digit d of piece c (k 8c .. 8c+7 of local group gg) of row m lies in a chunk buffer: 64-k
// block c / 8, lane group (c % 8) / 2 of its B operand, 8-byte half c % 2 of a 16-byte row; L = 1
// tile d, row m; L = 0 tile m / 4, row 4 (m % 4) + d. swz: the row index xor-ed with
// swz_of(kq, bb, gg) (the digits launch's LDS staging, so that the 64 lanes of a wave, one row's
// pieces, write distinct banks), or not (swz = false: the strips' own staging).
__device__ __forceinline__ int swz_of(int kq, int bb, int gg) { return kq + 4 * bb + 8 * (gg & 1); }
template <typename Lay, int L>
__device__ __forceinline__ int digit_offset(int gg, int c, int m, int d, bool swz)
{
    const int bb = c >> 3, kq = (c & 7) >> 1;
    const int tile = L == 0 ? m >> 2 : d;
    int row = L == 0 ? 4 * (m & 3) + d : m;
    if (swz) row ^= swz_of(kq, bb, gg);
    return gg * Lay::kGB + bb * Lay::kBbB + kq * Lay::kKqB + tile * Lay::kTileB + row * 16 + (c & 1) * 8;
}

// The activation digits of one chunk of one linear (workgroup j: image j), laid out as
// strip_wide_kernel's LDS chunk buffer: digits of every (group, row < M, 8-k piece) by
// stage_piece, zeros for rows M and up, then the row sums per (group, row) and 2^-(E+8), 2^(E+8)
// per row. Built in LDS, then copied out whole. Each strip of the linear copies the image instead
// of computing it. Wave w of pass h stages row 8h + w: its 64 lanes are the chunk's 4 groups x 16
// pieces, so the chunk's exponent is one wave reduction.
template <int L>
__global__ __launch_bounds__(kThreads) void wide_digits_kernel(const StripArgs a)
{
    using Lay = WideLayout<L>;
    extern __shared__ uint4 dyn_lds[];
    char* const lds = reinterpret_cast<char*>(dyn_lds);
    const int M = a.M;
    const int j = blockIdx.x;
    const int li = tab(a.dimg_lin + j);
    const int ch = j - tab(a.dimg_base + li);
    const SeqLinear* Lp = a.lin + li;
    const __amdgpu_buffer_rsrc_t rx = rsrc(sptr(tab(&Lp->x)));
    const int K = tab(&Lp->K);
    const int xdt = tab(&Lp->x_dtype);
    for (int o = threadIdx.x * 16; o < Lay::kBufB; o += kThreads * 16)
        *reinterpret_cast<uint4*>(lds + o) = uint4{0u, 0u, 0u, 0u};
    __syncthreads();
    const int items = kCG * M * 16;
    const int g0 = ch * kCG;
    float2* const gs = reinterpret_cast<float2*>(lds + Lay::kDigB);
    float* const ex = reinterpret_cast<float*>(lds + Lay::kDigB + kCG * 16 * 8);
#pragma unroll
    for (int h = 0; h < Lay::kH; h++) {
        const int idx = (int)threadIdx.x + kThreads * h;
        if (idx < items) {                        // whole waves: items is a multiple of 64
            const int item = idx >> 4, c = idx & 15;
            const int gg = item & 3, m = item >> 2;
            const uint32_t e = (uint32_t)m * (uint32_t)K + (uint32_t)((g0 + gg) * 128 + c * 8);
            float v[8];
            if (xdt == 0) {
                const f32x4 lo = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, e * 4u, 0, 0));
                const f32x4 hi = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, e * 4u + 16u, 0, 0));
                v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
                v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
            } else {
                const f16x8 hv = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, e * 2u, 0, 0));
#pragma unroll
                for (int q = 0; q < 8; q++) v[q] = (float)hv[q];
            }
            const int E = chunk_exponent(v);
            const PieceDigits pd = piece_digits(v, E);
#pragma unroll
            for (int d = 0; d < 4; d++)
                *reinterpret_cast<uint2*>(lds + digit_offset<Lay, L>(gg, c, m, d, true)) = pd.row[d];
            if (c == 0) gs[gg * 16 + m] = pd.sums;
            if ((idx & 63) == 0) {
                ex[m] = ldexpf(1.f, -E - 8);
                ex[16 + m] = ldexpf(1.f, E + 8);
            }
        }
    }
    __syncthreads();
    // out in the strips' layout: 16-byte unit u of the digits is (group, block, lane group, tile,
    // row) with the row fastest; its LDS copy sits at the swizzled row
    char* const dst = a.dimg + (size_t)j * Lay::kBufB;
    for (int o = threadIdx.x * 16; o < Lay::kBufB; o += kThreads * 16) {
        int src = o;
        if (o < Lay::kDigB) {
            const int u = o >> 4;
            const int rest = (u >> 4) / Lay::kTiles;       // (group, block, lane group)
            src = o ^ (swz_of(rest & 3, (rest >> 2) & 1, rest >> 3) << 4);
        }
        st_global(reinterpret_cast<u32x4*>(dst + o), *reinterpret_cast<const u32x4*>(lds + src));
    }
}

// Waves per SIMD the M 5..8 instance is compiled for. At 4 it fits 128 VGPRs (some spilled) and
// a CU holds two of its workgroups, planned as 512: the 7B step at M=8 measured 653 against
// 603-610 us with one workgroup per CU (2), so 2 is kept.
#ifndef QL_WIDE_OCC0
#define QL_WIDE_OCC0 2
#endif
// P: jobs in flight per wave (the register ring's depth): 2 for long strips over all of K, 4 (a
// chunk's every job) for the short K-part tasks, whose time is mostly round trips to HBM.
// S: where a chunk's activation digits come from. 0: the digit images of wide_digits_kernel;
// 1: computed while staging from fp32 activations formed through the linear's StripIn (as is,
// times the RMSNorm weight, or SiLU-mul of two producers), so a pass of a pass-by-pass sequence
// needs neither an elementwise launch nor a digits launch (an RMSNorm's 1/rms, one scalar per
// row, multiplies the sums in the part-sum launch: the linear commutes with it).
template <int L, int P, int S>
__global__ __launch_bounds__(kThreads, L == 0 ? QL_WIDE_OCC0 : 2) void strip_wide_kernel(const StripArgs a)
{
    static_assert(kCG % P == 0, "whole ring rounds per chunk");
    using Lay = WideLayout<L>;
    constexpr int KT = Lay::kTiles;
    extern __shared__ uint4 dyn_lds[];
    char* const lds = reinterpret_cast<char*>(dyn_lds);
    const int M = a.M;
    const int lane = threadIdx.x & 63;
    const int wave = sreg(threadIdx.x >> 6);
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int wg = blockIdx.x;
    // S = 1: workgroup w runs flat task w alone; its task, linear entry, staging and partial
    // offset are one record, so their loads do not wait on one another
    int tb = wg, te = wg + 1;
    if constexpr (S == 0) {
        tb = tab(a.task_begin + wg);
        te = tab(a.task_begin + wg + 1);
        if (tb >= te) return;
    }
    auto task_of = [&](int ti) {
        if constexpr (S == 1) return tab(&a.flat[ti].t);
        else return tab(a.tasks + ti);
    };
    auto lin_of = [&](int ti, const StripTask& t) -> const SeqLinear* {
        if constexpr (S == 1) return &a.flat[ti].L;
        else return a.lin + t.linear;
    };

    // chunk buffers (digits, then {2^-(E+8), sum x}), the strips' bias, the zero-term transposition
    auto gst = [&](int buf) { return reinterpret_cast<float2*>(lds + buf * Lay::kBufB + Lay::kDigB); };
    // 2^-(E+8) of row m at [m], 2^(E+8) at [16 + m]
    auto gex = [&](int buf) { return reinterpret_cast<float*>(lds + buf * Lay::kBufB + Lay::kDigB + kCG * 16 * 8); };
    float* const bias_base = reinterpret_cast<float*>(lds + 2 * Lay::kBufB);
    auto bias_lds = [&](int par) { return bias_base + par * (kBlocks * kCols); };


    if constexpr (S == 1) {
        // rows M and up of both chunk buffers stay zero (staging writes rows below M only)
        if (M < Lay::kMaxM) {
            for (int o = threadIdx.x * 16; o < 2 * Lay::kBufB; o += kThreads * 16)
                *reinterpret_cast<uint4*>(lds + o) = uint4{0u, 0u, 0u, 0u};
            __syncthreads();
        }
    }

    // ---- staging: the chunk being staged (task si, chunk sch): its digits into LDS ----
    struct Stage {
        int si, sch, ch0, chend, ngroups, ct, has_bias;
        __amdgpu_buffer_rsrc_t ri, rb, rz, rs;   // the linear's digit images (S = 1: x), bias (x without one), the wave block's zeros, scales
        uint32_t Gz, Gs;
        // S = 1: the second operand (SiLU-mul's up, RMSNorm's weight; x otherwise)
        __amdgpu_buffer_rsrc_t r2;
        int K, kind;
    };
    auto stage_open = [&](Stage& st, int ti) {
        const StripTask t = task_of(ti);
        const SeqLinear* Lp = lin_of(ti, t);
        st.si = ti;
        st.sch = st.ch0 = t.ch0;
        st.chend = t.ch0 + t.chunks;
        const float* b = tab(&Lp->bias);
        st.has_bias = b != nullptr;
        const void* dummy = a.dimg;                     // a global address for unused loads
        if constexpr (S == 0) {
            st.ri = rsrc(a.dimg + (size_t)tab(a.dimg_base + t.linear) * Lay::kBufB);
        } else {
            const StripIn in = tab(&a.flat[ti].in);
            const float* x = sptr(static_cast<const float*>(tab(&Lp->x)));
            st.ri = rsrc(x);
            st.K = tab(&Lp->K);
            st.kind = in.kind;
            st.r2 = rsrc(in.kind != 0 ? sptr(in.x2) : x);
            dummy = x;
        }
        st.rb = rsrc(b ? static_cast<const void*>(sptr(b) + t.ct * kCols) : dummy);
        st.ngroups = tab(&Lp->K) / 128;
        st.ct = t.ct;
        const int N = tab(&Lp->N);
        const uint32_t blk = (uint32_t)(t.ct + wave);
        st.rz = rsrc(reinterpret_cast<const char*>(sptr(tab(&Lp->qzeros))) + blk * (uint32_t)(kCols / 8) * 4u);
        st.rs = rsrc(reinterpret_cast<const char*>(sptr(tab(&Lp->scales))) + blk * (uint32_t)kCols * 2u);
        st.Gz = (((uint32_t)N + 7u) >> 3) * 4u;
        st.Gs = (uint32_t)N * 2u;
    };
    u32x4 xr[Lay::kHI];                     // S = 0: the chunk's image units of this thread
    u32x4 xs[Lay::kH][4];                   // S = 1: per item, x then the second operand (8 k each)
    float bv;                               // one bias value per thread (512 = a strip's columns)
    uint32_t zq;                            // zero word of group (chunk + kq), the lane's columns
    u32x2 sq;                               // scales of group (chunk + kq), the lane's 4 columns
    // step 1: unconditional loads, the same number on every path (threads past the image's units
    // or the chunk's items re-read the last one), so the wait before step 5 is exact
    auto stage_issue = [&](const Stage& st) {
        const int g0 = st.sch * kCG;
        if constexpr (S == 0) {
            const uint32_t img = (uint32_t)st.sch * (uint32_t)Lay::kBufB;
#pragma unroll
            for (int h = 0; h < Lay::kHI; h++) {
                const int u = min((int)threadIdx.x + kThreads * h, Lay::kUnits - 1);
                xr[h] = __builtin_amdgcn_raw_buffer_load_b128(st.ri, (uint32_t)u * 16u, img, 0);
            }
        } else {
            const int items = kCG * M * 16;
#pragma unroll
            for (int h = 0; h < Lay::kH; h++) {
                const int idx = min((int)threadIdx.x + kThreads * h, items - 1);
                const int item = idx >> 4, c = idx & 15;
                const int gg = item & 3, m = item >> 2;
                const uint32_t k = (uint32_t)((g0 + gg) * 128 + c * 8);
                const uint32_t e = (uint32_t)m * (uint32_t)st.K + k;
                xs[h][0] = __builtin_amdgcn_raw_buffer_load_b128(st.ri, e * 4u, 0, 0);
                xs[h][1] = __builtin_amdgcn_raw_buffer_load_b128(st.ri, e * 4u + 16u, 0, 0);
                const uint32_t e2 = st.kind == 1 ? k : e;       // the norm weight has no rows
                xs[h][2] = __builtin_amdgcn_raw_buffer_load_b128(st.r2, e2 * 4u, 0, 0);
                xs[h][3] = __builtin_amdgcn_raw_buffer_load_b128(st.r2, e2 * 4u + 16u, 0, 0);
            }
        }
        bv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(st.rb, st.has_bias ? threadIdx.x * 4u : 0u, 0, 0));
        zq = __builtin_amdgcn_raw_buffer_load_b32(st.rz, (uint32_t)kq * st.Gz + (uint32_t)(j >> 1) * 4u, (uint32_t)g0 * st.Gz, 0);
        sq = __builtin_amdgcn_raw_buffer_load_b64(st.rs, (uint32_t)kq * st.Gs + (uint32_t)j * 8u, (uint32_t)g0 * st.Gs, 0);
    };
    float nsz[4], nsz2[4];                  // -s (z+1), -s (z-7) of group (chunk + kq), the lane's columns
    // step 5: the staged image into buffer `buf`, its -s*z, the strip's bias
    auto stage_finish = [&](const Stage& st, int buf) {
        char* const dig = lds + buf * Lay::kBufB;
        if constexpr (S == 0) {
#pragma unroll
            for (int h = 0; h < Lay::kHI; h++) {
                const int u = (int)threadIdx.x + kThreads * h;
                if (u < Lay::kUnits) *reinterpret_cast<u32x4*>(dig + u * 16) = xr[h];
            }
        } else {
            const int items = kCG * M * 16;
            float2* const gs = gst(buf);
            float* const ex = gex(buf);
#pragma unroll
            for (int h = 0; h < Lay::kH; h++) {
                const int idx = (int)threadIdx.x + kThreads * h;
                if (idx < items) {                // whole waves (one row each): items is a multiple of 64
                    const int item = idx >> 4, c = idx & 15;
                    const int gg = item & 3, m = item >> 2;
                    const f32x4 x0 = __builtin_bit_cast(f32x4, xs[h][0]), x1 = __builtin_bit_cast(f32x4, xs[h][1]);
                    const f32x4 y0 = __builtin_bit_cast(f32x4, xs[h][2]), y1 = __builtin_bit_cast(f32x4, xs[h][3]);
                    float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    const float w2[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
                    if (st.kind == 2) {
                        // silu(g) * u = g / (1 + exp(-g)) * u, with the hardware exp2 and
                        // reciprocal (about 2 ulp; every strip of the pass forms these values, and
                        // expf with an IEEE division cost about 25 vector instructions per value)
#pragma unroll
                        for (int q = 0; q < 8; q++)
                            v[q] = v[q] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(v[q] * -1.44269504088896341f)) * w2[q];
                    } else if (st.kind == 1) {
#pragma unroll
                        for (int q = 0; q < 8; q++) v[q] = v[q] * w2[q];
                    }
                    const int E = chunk_exponent(v);
                    const PieceDigits pd = piece_digits(v, E);
#pragma unroll
                    for (int d = 0; d < 4; d++)
                        *reinterpret_cast<uint2*>(dig + digit_offset<Lay, L>(gg, c, m, d, false)) = pd.row[d];
                    if (c == 0) gs[gg * 16 + m] = pd.sums;
                    if ((idx & 63) == 0) {
                        ex[m] = ldexpf(1.f, -E - 8);
                        ex[16 + m] = ldexpf(1.f, E + 8);
                    }
                }
            }
        }
        // -s * z of the lane's columns 4j .. 4j+3 for group (chunk + kq), zero = stored + 1, for
        // the even k; the odd k's weight operand 16 (n - 8) moves their zero to z - 8
        const uint32_t zw = zq >> (16 * (j & 1));
        const uint32_t sw[4] = {sq.x & 0xffffu, sq.x >> 16, sq.y & 0xffffu, sq.y >> 16};
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
            const int zs = (int)((zw >> (4 * u)) & 15u);
            nsz[u] = -s * (float)(zs + 1);
            nsz2[u] = -s * (float)(zs - 7);
        }
        if (st.sch == st.ch0) bias_lds((st.si - tb) & 1)[threadIdx.x] = st.has_bias ? bv : 0.f;
    };
    auto stage_next = [&](Stage& st) {    // false past the last chunk of the last task
        if (st.sch + 1 < st.chend) {
            st.sch++;
            return true;
        }
        if (st.si + 1 >= te) return false;
        stage_open(st, st.si + 1);
        return true;
    };

    // ---- job stream: one job per group of each strip (the wave's block) ----
    uint4 wb[P][2 * kNB];
    uint2 sb[P];
    struct Cur {
        int ti, g, gend;            // the task's groups end at gend
        __amdgpu_buffer_rsrc_t rq, rs;   // the wave block's packed weights and scales
        uint32_t Gq, Gs;
        uint32_t lq[2 * kNB];       // the lane's packed rows 2kq, 2kq+1, 2kq+8, 2kq+9 of a group
    };
    const uint32_t ls = 8u * (uint32_t)j;
    auto open = [&](Cur& c, int ti) {
        const StripTask t = task_of(ti);
        const SeqLinear* Lp = lin_of(ti, t);
        c.ti = ti;
        c.g = t.ch0 * kCG;
        const int N = sreg(tab(&Lp->N));
        c.gend = (t.ch0 + t.chunks) * kCG;
        const uint32_t blk = (uint32_t)(t.ct + wave);
        c.rq = rsrc(reinterpret_cast<const char*>(sptr(tab(&Lp->qweight))) + blk * (uint32_t)kCols * 4u);
        c.rs = rsrc(reinterpret_cast<const char*>(sptr(tab(&Lp->scales))) + blk * (uint32_t)kCols * 2u);
        c.Gq = 16u * (uint32_t)N * 4u;
        c.Gs = (uint32_t)N * 2u;
#pragma unroll
        for (int r = 0; r < 2 * kNB; r++)
            c.lq[r] = ((uint32_t)(2 * kq + (r >> 1) * 8 + (r & 1)) * (uint32_t)N + 4u * (uint32_t)j) * 4u;
    };
    auto advance = [&](Cur& c) {
        if (c.g + 1 < c.gend) c.g++;
        else if (c.ti + 1 < te) open(c, c.ti + 1);
        // else: the stream has ended; stay on the last job (its reloads are never consumed)
    };
    auto fetch = [&](int d, const Cur& c) {
        const uint32_t gq = (uint32_t)c.g * c.Gq;
#pragma unroll
        for (int r = 0; r < 2 * kNB; r++)
            wb[d][r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(c.rq, c.lq[r], gq, kNT));
        sb[d] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(c.rs, ls, (uint32_t)c.g * c.Gs, 0));
    };

    // accumulators: L = 1 rows 4kq + r of column 4j + u: acc[u][r]; L = 0 rows 4t + kq: acc[u][t],
    // and the zero term in the MFMA layout (rows 4kq + r) in zacc, folded in at a strip's end.
    // cacc: the current chunk's sums in units of its exponent (acc's layout), folded into acc with
    // one multiply-add by 2^-(E+8) at the chunk's end.
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef typename std::conditional<L == 0, f32x2, f32x4>::type Acc;
    Acc acc[4], cacc[4];
    f32x4 zacc[L == 0 ? 4 : 1];
    auto clear = [&]() {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            acc[u] = Acc{};
            if constexpr (L == 0) zacc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };

    // lane-constant LDS offsets: the A operand row of this lane (row j of each tile, lane group kq)
    const int a_lane = kq * Lay::kKqB + j * 16;

    // one job: local group gg of the chunk in buffer `buf`, ring slot d
    auto consume = [&](int d, int buf, int gg) {
        const char* const dig = lds + buf * Lay::kBufB + gg * Lay::kGB + a_lane;
        i32x4 av[kNB][KT];
#pragma unroll
        for (int bb = 0; bb < kNB; bb++)
#pragma unroll
            for (int t = 0; t < KT; t++)
                av[bb][t] = *reinterpret_cast<const i32x4*>(dig + bb * Lay::kBbB + t * Lay::kTileB);
        // the scales of the lane's 4 columns, fp16 as loaded (the epilogue's v_fma_mix_f32 takes
        // them without a conversion)
        const uint2 sv = sb[d];
        const f16x2 s01 = __builtin_bit_cast(f16x2, sv.x), s23 = __builtin_bit_cast(f16x2, sv.y);
        const _Float16 s[4] = {s01[0], s01[1], s23[0], s23[1]};
        // the weight nibbles of 64-k block bb, column quarter u, as bytes: even k n, odd k 16 (n - 8)
        auto bq_of = [&](int bb, int u) {
            const uint4 w0 = wb[d][2 * bb], w1 = wb[d][2 * bb + 1];
            const uint32_t lo[4] = {w0.x, w0.y, w0.z, w0.w};
            const uint32_t hi[4] = {w1.x, w1.y, w1.z, w1.w};
            return i32x4{(int)(lo[u] & 0x0F0F0F0Fu), (int)((lo[u] ^ 0x88888888u) & 0xF0F0F0F0u),
                         (int)(hi[u] & 0x0F0F0F0Fu), (int)((hi[u] ^ 0x88888888u) & 0xF0F0F0F0u)};
        };
        if constexpr (L == 1) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                i32x4 c[4];
#pragma unroll
                for (int bb = 0; bb < kNB; bb++) {
                    const i32x4 bq = bq_of(bb, u);
#pragma unroll
                    for (int t = 0; t < 4; t++) c[t] = mfma_i8(av[bb][t], bq, bb == 0 ? i32x4{0, 0, 0, 0} : c[t]);
                }
                // tile t holds digit t: 2^8 * sum_d c_d 2^(8d-24) = (c0 + 2^8 c1) 2^-16 + (c2 + 2^8 c3)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int lo2 = c[0][r] + c[1][r] * 256;
                    const int hi2 = c[2][r] + c[3][r] * 256;
                    const float v = fmaf((float)lo2, 0x1p-16f, (float)hi2);
                    cacc[u][r] = fmaf((float)s[u], v, cacc[u][r]);
                }
#if QL_WIDE_QREGION
                asm volatile("" : "+v"(cacc[u]));
                __builtin_amdgcn_sched_barrier(0);
#endif
            }
            // keep this job's epilogue here: without a use, the compiler sinks every job's
            // epilogue to the end of the chunk and keeps all four jobs' MFMA results live
#pragma unroll
            for (int u = 0; u < 4; u++) asm volatile("" : "+v"(cacc[u]));
        } else {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                i32x4 c[2];
#pragma unroll
                for (int bb = 0; bb < kNB; bb++) {
                    const i32x4 bq = bq_of(bb, u);
#pragma unroll
                    for (int t = 0; t < 2; t++) c[t] = mfma_i8(av[bb][t], bq, bb == 0 ? i32x4{0, 0, 0, 0} : c[t]);
                }
                // digit products (|c| < 2^21, digit 3 most significant) in two exact integer
                // pairs: 2^8 * sum_d c_d 2^(8d-24) = (c0 + 2^8 c1) 2^-16 + (c2 + 2^8 c3)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int lo2 = c[t][0] + c[t][1] * 256;
                    const int hi2 = c[t][2] + c[t][3] * 256;
                    const float v = fmaf((float)lo2, 0x1p-16f, (float)hi2);
                    cacc[u][t] = fmaf((float)s[u], v, cacc[u][t]);
                }
            }
            // keep this job's epilogue here: without a use, the compiler sinks every job's
            // epilogue to the end of the chunk and keeps all four jobs' MFMA results live
#pragma unroll
            for (int u = 0; u < 4; u++) asm volatile("" : "+v"(cacc[u]));
        }
    };

    // The zero-point term of a chunk: rows i, columns 4j + u: sum over its 4 groups g of
    // sum_even[g][i] (-s (z+1))[g][col] + sum_odd[g][i] (-s (z-7))[g][col] (lane (kq, i) holds
    // A = the sums of group kq, row i; lane (kq, j) holds B of group kq, its column of quarter u).
    // L = 1: A in the chunk's exponent units, and the MFMAs start the chunk's sums (their
    // internal sum is not one IEEE rounding, so they never take a running sum as C: fed acc, they
    // lost up to 2.8e-5 over the 148 groups of a 7B down projection). L = 0: in the MFMA layout,
    // added to zacc; the chunk's sums start from zero.
    auto chunk_begin = [&](int buf) {
        const float2 sx = gst(buf)[kq * 16 + j];
        if constexpr (L == 1) {
            const float xi = gex(buf)[16 + j];
#pragma unroll
            for (int u = 0; u < 4; u++)
                cacc[u] = mfma_f32_4(sx.y * xi, nsz2[u], mfma_f32_4(sx.x * xi, nsz[u], f32x4{0.f, 0.f, 0.f, 0.f}));
        } else {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                cacc[u] = Acc{};
                zacc[u] += mfma_f32_4(sx.y, nsz2[u], mfma_f32_4(sx.x, nsz[u], f32x4{0.f, 0.f, 0.f, 0.f}));
            }
        }
    };
    // the chunk's sums into acc: times 2^-(E+8) of the row (L = 1: rows 4kq + r; L = 0: 4t + kq)
    auto chunk_end = [&](int buf) {
        const float* const ex = gex(buf);
        if constexpr (L == 1) {
            const f32x4 e = *reinterpret_cast<const f32x4*>(ex + 4 * kq);
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[u][r] = fmaf(e[r], cacc[u][r], acc[u][r]);
        } else {
            const float e0 = ex[kq], e1 = ex[4 + kq];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                acc[u][0] = fmaf(e0, cacc[u][0], acc[u][0]);
                acc[u][1] = fmaf(e1, cacc[u][1], acc[u][1]);
            }
        }
    };

    // the first chunk's image, then the ring's first P positions, in flight together
    Stage sg;
    stage_open(sg, tb);
    stage_issue(sg);
    Cur fc;
    open(fc, tb);
#pragma unroll
    for (int d = 0; d < P; d++) {
        fetch(d, fc);
        advance(fc);
    }
    stage_finish(sg, 0);
    __syncthreads();
    bool staging = stage_next(sg);
    clear();

    int buf = 0;
    for (int ti = tb; ti < te; ti++) {
        const StripTask t = task_of(ti);
        const SeqLinear* Lp = lin_of(ti, t);
        const int nch = t.ch0 + t.chunks;   // end of the task's chunks
        for (int ch = t.ch0; ch < nch; ch++) {
            stage_issue(sg);                 // past the last chunk: repeats it (never finished)
            chunk_begin(buf);
#pragma unroll
            for (int gg = 0; gg < kCG; gg++) {
                consume(gg % P, buf, gg);
                fetch(gg % P, fc);
                advance(fc);
            }
            chunk_end(buf);
            if (ch + 1 == nch) {
                // a whole task's outputs with the bias, or a K part's sums into its partial block
                const bool whole = t.parts <= 1;
                const int N = tab(&Lp->N);
                int64_t po = 0;
                if constexpr (S == 1) po = tab(&a.flat[ti].poff);
                else if (!whole) po = tab(a.poff + t.linear);
                float* const y = whole ? tab(&Lp->y) : a.partial + po + (size_t)t.part * M * N;
                const int col = (t.ct + wave) * kCols + 4 * j;
                const f32x4 bvv = whole ? *reinterpret_cast<const f32x4*>(bias_lds((ti - tb) & 1) + wave * kCols + 4 * j)
                                        : f32x4{0.f, 0.f, 0.f, 0.f};
                if constexpr (L == 1) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = 4 * kq + r;
                        if (m < M)
                            st_global(reinterpret_cast<f32x4*>(y + (size_t)m * N + col),
                                      f32x4{acc[0][r] + bvv.x, acc[1][r] + bvv.y, acc[2][r] + bvv.z, acc[3][r] + bvv.w});
                    }
                } else {
                    // the zero term from the MFMA layout (row 4kq + r) to the digit layout (row
                    // 4t + kq) through this wave's own LDS rows
                    float* const zl = reinterpret_cast<float*>(lds + 2 * Lay::kBufB + Lay::kBiasB) + wave * 16 * kCols;
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        *reinterpret_cast<f32x4*>(zl + (4 * kq + r) * kCols + 4 * j) =
                            f32x4{zacc[0][r], zacc[1][r], zacc[2][r], zacc[3][r]};
                    // a wave's LDS operations complete in order: the reads below see every lane's
                    // writes (the fences only keep the compiler from moving them)
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
                    __builtin_amdgcn_wave_barrier();
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
                    for (int tt = 0; tt < 2; tt++) {
                        const int m = 4 * tt + kq;
                        const f32x4 z = *reinterpret_cast<const f32x4*>(zl + m * kCols + 4 * j);
                        if (m < M)
                            st_global(reinterpret_cast<f32x4*>(y + (size_t)m * N + col),
                                      f32x4{acc[0][tt] + z.x + bvv.x, acc[1][tt] + z.y + bvv.y,
                                            acc[2][tt] + z.z + bvv.z, acc[3][tt] + z.w + bvv.w});
                    }
                }
                clear();
            }
            if (staging) stage_finish(sg, buf ^ 1);
            __syncthreads();
            buf ^= 1;
            if (staging) staging = stage_next(sg);
        }
    }
}

// The K parts of every split linear of a pass, summed with bias and residual: blockIdx.y is the
// entry; 4 lanes (a DPP quad) per 4 consecutive outputs (N % 4 == 0), lane r summing parts
// r, r + 4, ... in order, the quad's four sums then combined as (s0 + s1) + (s2 + s3), so every
// run adds in the same order. Up to 4 loads per lane are issued before their adds. With in_ssq
// set (the linear's input is RMSNorm'd: its strips staged x * w), the sum is multiplied by the
// row's 1 / rms before bias and residual. With ssq set (N % 256 == 0: a workgroup's 64 quads are
// 256 columns of one row), the workgroup also writes the sum of squares of its 256 outputs, in a
// fixed order, for a consumer that RMSNorms y.
__device__ __forceinline__ void part_sum_entry(const PartSum& e, int M)
{
    __shared__ float red[4];
    const int n4 = e.N / 4;
    const int i = (int)(blockIdx.x * 256 + threadIdx.x) >> 2;   // 4-value group over [M][N]
    const int r = threadIdx.x & 3;
    if (i >= M * n4) return;                  // whole quads (with ssq: whole workgroups) leave
    const int m = i / n4, c = (i - m * n4) * 4;
    const size_t stride = (size_t)M * e.N;
    const float* p = e.part0 + (size_t)m * e.N + c;
    // the bias, residual and (up to 16 blocks of) the input's sums of squares go out with the
    // parts, so the lane waits for memory once
    const f32x4 bv = e.bias ? ld_global(reinterpret_cast<const f32x4*>(e.bias + c)) : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 rv = e.res ? ld_global(reinterpret_cast<const f32x4*>(e.res + (size_t)m * e.N + c)) : f32x4{0.f, 0.f, 0.f, 0.f};
    const int nb = e.in_ssq ? e.K / 256 : 0;
    float sb[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int b = r + 4 * k;
        sb[k] = b < nb ? ld_global(e.in_ssq + (size_t)m * nb + b) : 0.f;
    }
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    int q = r;
    for (; q + 12 < e.parts; q += 16) {
        const f32x4 a0 = ld_global(reinterpret_cast<const f32x4*>(p + (size_t)q * stride));
        const f32x4 a1 = ld_global(reinterpret_cast<const f32x4*>(p + (size_t)(q + 4) * stride));
        const f32x4 a2 = ld_global(reinterpret_cast<const f32x4*>(p + (size_t)(q + 8) * stride));
        const f32x4 a3 = ld_global(reinterpret_cast<const f32x4*>(p + (size_t)(q + 12) * stride));
        v += a0;
        v += a1;
        v += a2;
        v += a3;
    }
    for (; q < e.parts; q += 4) v += ld_global(reinterpret_cast<const f32x4*>(p + (size_t)q * stride));
    // quad_perm [1,0,3,2] then [2,3,0,1]: every lane of the quad ends with (s0 + s1) + (s2 + s3)
    // (an add's two operands commute exactly). Each component is copied to a scalar first:
    // __builtin_bit_cast of a vector element subscript (v[k]) read element 0 whatever k.
    f32x4 t;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float sk = v[k];
        const float w = sk + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sk), 0xB1, 0xF, 0xF, false));
        t[k] = w + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, w), 0x4E, 0xF, 0xF, false));
    }
    if (e.in_ssq) {
        // the input row's sum of squares: lane r adds its 256-column blocks r, r + 4, ... in
        // order, then the quad as above (the same bits in every quad of the row)
        float ss = ((sb[0] + sb[1]) + sb[2]) + sb[3];
        for (int b = r + 16; b < nb; b += 4) ss += ld_global(e.in_ssq + (size_t)m * nb + b);
        const float w = ss + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, ss), 0xB1, 0xF, 0xF, false));
        const float tot = w + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, w), 0x4E, 0xF, 0xF, false));
        const float rstd = 1.0f / sqrtf(tot / (float)e.K + e.eps);
        t *= rstd;
    }
    if (e.bias) t += bv;
    if (e.res) t += rv;
    if (r == 0) st_global(reinterpret_cast<f32x4*>(e.y + (size_t)m * e.N + c), t);
    if (e.ssq) {
        // the quad's lanes hold the same t: the xor 1 and 2 steps double it exactly, so the
        // wave's butterfly ends with 4 x (the sum over its 16 quads), the same in every lane
        float s2 = fmaf(t.w, t.w, fmaf(t.z, t.z, fmaf(t.y, t.y, t.x * t.x)));
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) s2 += __shfl_xor(s2, o);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s2;
        __syncthreads();
        if (threadIdx.x == 0) e.ssq[(size_t)m * (e.N / 256) + c / 256] = ((red[0] + red[1]) + (red[2] + red[3])) * 0.25f;
    }
}

// NP sums of as many parts each, lane r of a DPP quad adding parts p[j] + q * stride for
// q = r, r + 4, ... in order (the loads of the NP sums in one loop, so that they go out together)
// and the quad then combining them as (s0 + s1) + (s2 + s3) with quad_perm [1,0,3,2] then
// [2,3,0,1]: every lane ends with the same bits, those of part_sum_entry's sums.
template <int NP>
__device__ __forceinline__ void quad_parts_sums(const float* const (&p)[NP], int parts, size_t stride, int r, f32x4 (&t)[NP])
{
    f32x4 v[NP];
#pragma unroll
    for (int j = 0; j < NP; j++) v[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    int q = r;
    for (; q + 12 < parts; q += 16) {
        f32x4 a[NP][4];
#pragma unroll
        for (int j = 0; j < NP; j++)
#pragma unroll
            for (int h = 0; h < 4; h++) a[j][h] = ld_global(reinterpret_cast<const f32x4*>(p[j] + (size_t)(q + 4 * h) * stride));
#pragma unroll
        for (int j = 0; j < NP; j++) {
            v[j] += a[j][0];
            v[j] += a[j][1];
            v[j] += a[j][2];
            v[j] += a[j][3];
        }
    }
    for (; q < parts; q += 4) {
        f32x4 a[NP];
#pragma unroll
        for (int j = 0; j < NP; j++) a[j] = ld_global(reinterpret_cast<const f32x4*>(p[j] + (size_t)q * stride));
#pragma unroll
        for (int j = 0; j < NP; j++) v[j] += a[j];
    }
#pragma unroll
    for (int j = 0; j < NP; j++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float sk = v[j][k];
            const float w = sk + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sk), 0xB1, 0xF, 0xF, false));
            t[j][k] = w + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, w), 0x4E, 0xF, 0xF, false));
        }
}

// silu(g) * u, as the SiLU-mul launch forms it (IEEE division, expf)
__device__ __forceinline__ float silu_mul1(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// An entry whose yglu is set: the gate linear's sums (+ bias, residual) into y, the up linear's
// (the b fields: as many parts, + bias) into yb, and silu(y) * yb into yglu, in place of a
// SiLU-mul launch of its own.
__device__ __forceinline__ void part_sum_glu_entry(const PartSum& e, int M)
{
    const int n4 = e.N / 4;
    const int i = (int)(blockIdx.x * 256 + threadIdx.x) >> 2;
    const int r = threadIdx.x & 3;
    if (i >= M * n4) return;
    const int m = i / n4, c = (i - m * n4) * 4;
    const size_t stride = (size_t)M * e.N;
    const size_t o = (size_t)m * e.N + c;
    const f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 bv = e.bias ? ld_global(reinterpret_cast<const f32x4*>(e.bias + c)) : z;
    const f32x4 rv = e.res ? ld_global(reinterpret_cast<const f32x4*>(e.res + o)) : z;
    const f32x4 ubv = e.bias_b ? ld_global(reinterpret_cast<const f32x4*>(e.bias_b + c)) : z;
    const float* const pp[2] = {e.part0 + o, e.part0b + o};
    f32x4 tu[2];
    quad_parts_sums<2>(pp, e.parts, stride, r, tu);
    f32x4 t = tu[0], u = tu[1];
    if (e.bias) t += bv;
    if (e.res) t += rv;
    if (e.bias_b) u += ubv;
    if (r == 0) {
        st_global(reinterpret_cast<f32x4*>(e.y + o), t);
        st_global(reinterpret_cast<f32x4*>(e.yb + o), u);
        st_global(reinterpret_cast<f32x4*>(e.yglu + o),
                  f32x4{silu_mul1(t.x, u.x), silu_mul1(t.y, u.y), silu_mul1(t.z, u.z), silu_mul1(t.w, u.w)});
    }
}

__global__ __launch_bounds__(256) void part_sum_kernel(const PartSum* entries, int M)
{
    part_sum_entry(entries[blockIdx.y], M);
}

__global__ __launch_bounds__(256) void part_sum_glu_kernel(const PartSum* entries, int M)
{
    part_sum_glu_entry(entries[blockIdx.y], M);
}

// the same with the entries in the kernel arguments (a batch of single-call linears)
__global__ __launch_bounds__(256) void part_sum_args_kernel(const PartSumArgs a)
{
    part_sum_entry(a.e[blockIdx.y], a.M);
}

}  // namespace

hipError_t launch_part_sums_args(const PartSumArgs& a, int max_n, hipStream_t stream)
{
    if (a.count < 1) return hipSuccess;
    const int threads = a.M * (max_n / 4) * 4;
    hipLaunchKernelGGL(part_sum_args_kernel, dim3((threads + 255) / 256, a.count), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_part_sums(const PartSum* entries_dev, int count, int M, int max_n, bool glu, hipStream_t stream)
{
    if (count < 1) return hipSuccess;
    const int threads = M * (max_n / 4) * 4;
    if (glu)
        hipLaunchKernelGGL(part_sum_glu_kernel, dim3((threads + 255) / 256, count), dim3(256), 0, stream, entries_dev, M);
    else
        hipLaunchKernelGGL(part_sum_kernel, dim3((threads + 255) / 256, count), dim3(256), 0, stream, entries_dev, M);
    return hipGetLastError();
}

bool strip_wide_eligible(const std::vector<SeqSpec>& lin, int M, const StripPlan& p, int min_m)
{
    if (!p.stream || p.split != 1 || M < min_m || M > kGemvMaxM) return false;
    for (const SeqSpec& s : lin)
        if (s.group != 128 || s.K % (128 * kCG) != 0 || s.N % (kBlocks * kCols) != 0) return false;
    return true;
}

int strip_wide_per_cu(int M)
{
    return M <= 8 && QL_WIDE_OCC0 >= 4 ? 2 : 1;
}

size_t strip_wide_lds(int M)
{
    return M <= 8 ? (size_t)WideLayout<0>::kLds : (size_t)WideLayout<1>::kLds;
}

size_t strip_wide_image_bytes(int M)
{
    return M <= 8 ? (size_t)WideLayout<0>::kBufB : (size_t)WideLayout<1>::kBufB;
}

hipError_t launch_strips_wide(const StripArgs& a, size_t lds, hipStream_t stream)
{
    void* args[] = {const_cast<StripArgs*>(&a)};
    if (a.in) {
        // activations staged through StripIn: no digit images (K-part plans only), one
        // workgroup per flat task
        if (a.ring != 4 || !a.flat) return hipErrorInvalidValue;
        const void* fn = a.M <= 8 ? reinterpret_cast<const void*>(&strip_wide_kernel<0, 4, 1>)
                                  : reinterpret_cast<const void*>(&strip_wide_kernel<1, 4, 1>);
        return hipLaunchKernel(fn, dim3(a.G), dim3(kThreads), args, lds, stream);
    }
    if (!a.dimg || a.dimg_count < 1) return hipErrorInvalidValue;
    const void* dfn = a.M <= 8 ? reinterpret_cast<const void*>(&wide_digits_kernel<0>)
                               : reinterpret_cast<const void*>(&wide_digits_kernel<1>);
    hipError_t e = hipLaunchKernel(dfn, dim3(a.dimg_count), dim3(kThreads), args, strip_wide_image_bytes(a.M), stream);
    if (e != hipSuccess) return e;
    const bool deep = a.ring == 4;
    const void* fn = a.M <= 8 ? (deep ? reinterpret_cast<const void*>(&strip_wide_kernel<0, 4, 0>)
                                      : reinterpret_cast<const void*>(&strip_wide_kernel<0, 2, 0>))
                              : (deep ? reinterpret_cast<const void*>(&strip_wide_kernel<1, 4, 0>)
                                      : reinterpret_cast<const void*>(&strip_wide_kernel<1, 2, 0>));
    return hipLaunchKernel(fn, dim3(a.G), dim3(kThreads), args, lds, stream);
}

}  // namespace ql
