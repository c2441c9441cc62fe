// Prefill GEMM for GPTQ int4 linears, M > 16: y[M,N] = f16(x)[M,K] * f16(W)[N,K]^T (+ bias, + res),
// fp32 accumulation. Same arithmetic as the reference's M > 1 path, gemm_nt_f16_from_f32.wgsl
// (x rounded to fp16 on load, fp16 weights from the load-time dequant), but the weights are
// dequantized from the packed int4 words inside the kernel, bit-identical to the load-time fp16
// arena (dequant_word_perm in ql_device.h).
//
// Work split: a workgroup (4 waves) owns BM rows x 256 columns and one K segment of whole
// quantization groups; each wave owns 64 of the columns for all BM rows. A K step is 32 k (one
// v_mfma_f32_16x16x32_f16 block = 4 packed qweight rows).
// * Weights never pass through LDS. Lane (j, kq) loads 16 bytes of packed row 4s + kq: the words
//   of columns 4j .. 4j+3 of its wave's strip, and each word is exactly the lane's B fragment (8 k
//   of one column) for one of the wave's 4 N tiles. N tile t therefore holds columns 4j + t,
//   which makes each lane's 4 outputs of a row adjacent (one 16-byte store).
// * Activations (shared by the 4 waves) are staged per step in LDS, double-buffered, rounded to
//   fp16 and permuted into the k order dequant_word_perm emits.
// * Each thread keeps D steps of loads in flight (a register ring, statically indexed).
// * With split > 1 K segments, each workgroup stores its partial tile with agent-scope stores and
//   bumps the tile's arrival counter; the last one adds the partials in ascending segment order
//   (deterministic, like the reference's gemm_gemv_split_reduce.wgsl:32-38) and resets the
//   counter, all in one launch.
// * Several linears can share one launch (q/k/v, gate/up): workgroups are numbered across them.
#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

#include <algorithm>

namespace ql {

namespace {

// Tunables (compile-time):
//   QL_GEMM_DEPTH       K steps of loads each thread keeps in flight (even)
//   QL_GEMM_TARGET_WGS  workgroups per CU a linear aims for when choosing the K split
//   QL_GEMM_MIN_STEPS   fewest K steps per segment (caps the split)
#ifndef QL_GEMM_DEPTH
#define QL_GEMM_DEPTH 8
#endif
#ifndef QL_GEMM_DEPTH_F32
#define QL_GEMM_DEPTH_F32 (QL_GEMM_DEPTH / 2)
#endif
#ifndef QL_GEMM_TARGET_WGS
#define QL_GEMM_TARGET_WGS 1
#endif
#ifndef QL_GEMM_MIN_STEPS
#define QL_GEMM_MIN_STEPS 8
#endif
static_assert(QL_GEMM_DEPTH % 4 == 0, "the LDS double buffer alternates with the ring slot");

constexpr int kCols = kGemmTileCols;   // 256 columns per workgroup, 64 per wave

constexpr int kSC1 = 16;               // buffer-op cache policy bit SC1 (agent coherence)

// qzeros word of a linear without qzeros: every stored zero 7 (true zero 8)
__device__ const uint32_t kSymZeros = 0x77777777u;

// 8 activations (natural k order) as fp16 in the order dequant_word_perm emits {0,4,1,5,2,6,3,7}
__device__ __forceinline__ u32x4 perm_f16(u32x4 nat)
{
    // nat holds (k0,k1) (k2,k3) (k4,k5) (k6,k7); want (k0,k4) (k1,k5) (k2,k6) (k3,k7)
    u32x4 r;
    r.x = __builtin_amdgcn_perm(nat.z, nat.x, 0x05040100u);   // lo halves: k0 | k4
    r.y = __builtin_amdgcn_perm(nat.z, nat.x, 0x07060302u);   // hi halves: k1 | k5
    r.z = __builtin_amdgcn_perm(nat.w, nat.y, 0x05040100u);   // k2 | k6
    r.w = __builtin_amdgcn_perm(nat.w, nat.y, 0x07060302u);   // k3 | k7
    return r;
}

// The same from 8 f32 activations (a: k0..k3, b: k4..k7), each rounded to fp16 (RNE). Written as
// one vector shuffle + conversion: building the result from four scalar (lo, hi) pair
// conversions is miscompiled for gfx950 by this toolchain (all four words come out equal to the
// first pair).
__device__ __forceinline__ u32x4 perm_f32(u32x4 a, u32x4 b)
{
    typedef float f32x8 __attribute__((ext_vector_type(8)));
    const f32x4 fa = __builtin_bit_cast(f32x4, a), fb = __builtin_bit_cast(f32x4, b);
    const f32x8 v = __builtin_shufflevector(fa, fb, 0, 4, 1, 5, 2, 6, 3, 7);
    return __builtin_bit_cast(u32x4, __builtin_convertvector(v, f16x8));
}

// An empty asm that claims to rewrite v, so nothing computed from v moves above this point
__device__ __forceinline__ void pin(u32x4& v)
{
    uint32_t e0 = v.x, e1 = v.y, e2 = v.z, e3 = v.w;
    asm volatile("" : "+v"(e0), "+v"(e1), "+v"(e2), "+v"(e3));
    v = u32x4{e0, e1, e2, e3};
}

// Stores a workgroup's BM x 256 tile: directly (split == 1) or, with a K split, as this segment's
// partial sums, the last segment to arrive adding all of them in ascending segment order.
// Lane (j, kq) holds rows 16 tm + 4 kq + r of columns ncol .. ncol + 3 (one per N tile).
template <int MT>
__device__ __forceinline__ void gemm_store(const GemmLinear& L, int M, int m0, int nt, int mt, int seg,
                                           int split, int ncol, bool col_ok, int kq, const f32x4 (&acc)[MT][4])
{
    constexpr int BM = MT * 16;
    const int N = L.N;
    if (split == 1) {
        if (!col_ok) return;
        f32x4 bias = f32x4{0.f, 0.f, 0.f, 0.f};
        if (L.bias) bias = ld_global(reinterpret_cast<const f32x4*>(L.bias + ncol));
#pragma unroll
        for (int tm = 0; tm < MT; tm++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * tm + 4 * kq + r;
                if (m < M) {
                    f32x4 v = f32x4{acc[tm][0][r] + bias.x, acc[tm][1][r] + bias.y, acc[tm][2][r] + bias.z,
                                    acc[tm][3][r] + bias.w};
                    if (L.res) v += ld_global(reinterpret_cast<const f32x4*>(L.res + (size_t)m * N + ncol));
                    st_global(reinterpret_cast<f32x4*>(L.y + (size_t)m * N + ncol), v);
                }
            }
        return;
    }
    // Partial sums go through buffer stores / loads with the SC1 cache policy: the coherence
    // point of agent-scope accesses (another XCD's workgroup adds them up). Unlike atomics they
    // can all be in flight at once. The host keeps split * M * N * 4 below 2 GiB.
    const __amdgpu_buffer_rsrc_t part = __builtin_amdgcn_make_buffer_rsrc(L.partial, 0, 0x7FFFFFFF, 0x00020000);
    const uint32_t plane = (uint32_t)M * (uint32_t)N * 4u;   // bytes per segment
    if (col_ok) {
#pragma unroll
        for (int tm = 0; tm < MT; tm++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * tm + 4 * kq + r;
                if (m < M)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        f32x4{acc[tm][0][r], acc[tm][1][r], acc[tm][2][r], acc[tm][3][r]}, part,
                        ((uint32_t)m * (uint32_t)N + (uint32_t)ncol) * 4u, seg * plane, kSC1);
            }
    }
    if (L.defer) return;   // a part-sum launch adds the segments
    // this wave's partial stores are complete before the workgroup signals arrival
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ uint32_t is_last;
    __syncthreads();
    const int tile = nt * L.tiles_m + mt;
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&L.counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t last = prev == (uint32_t)(split - 1);
        if (last) __hip_atomic_store(&L.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = last;
    }
    __syncthreads();
    if (!is_last) return;
    // the tile's sums in ascending segment order: a thread owns PER 4-column pieces, and each
    // segment's loads for all of them are issued together (one round trip per segment)
    // a thread owns PER 4-column pieces, reduced HALF at a time with two segments' loads in flight
    constexpr int PER = BM * (kCols / 4) / 256;
    constexpr int HALF = PER / 2;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        f32x4 sum[HALF];
        bool ok[HALF];
        int col[HALF];
        uint32_t off[HALF];
#pragma unroll
        for (int i = 0; i < HALF; i++) {
            const int idx = threadIdx.x + 256 * (h * HALF + i);
            const int m = m0 + idx / (kCols / 4);
            const int n = nt * kCols + 4 * (idx % (kCols / 4));
            ok[i] = m < M && n < N;
            col[i] = n;
            off[i] = ok[i] ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * 4u : 0u;
            sum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        int sg = 0;
        for (; sg + 2 <= split; sg += 2) {
            f32x4 v0[HALF], v1[HALF];
#pragma unroll
            for (int i = 0; i < HALF; i++) {
                v0[i] = __builtin_amdgcn_raw_buffer_load_b128(part, off[i], sg * plane, kSC1);
                v1[i] = __builtin_amdgcn_raw_buffer_load_b128(part, off[i], (sg + 1) * plane, kSC1);
            }
#pragma unroll
            for (int i = 0; i < HALF; i++) sum[i] = sum[i] + v0[i] + v1[i];
        }
        if (sg < split) {
#pragma unroll
            for (int i = 0; i < HALF; i++) sum[i] += __builtin_amdgcn_raw_buffer_load_b128(part, off[i], sg * plane, kSC1);
        }
#pragma unroll
        for (int i = 0; i < HALF; i++) {
            if (!ok[i]) continue;
            f32x4 v = sum[i];
            if (L.bias) v += ld_global(reinterpret_cast<const f32x4*>(L.bias + col[i]));
            if (L.res) v += ld_global(reinterpret_cast<const f32x4*>(L.res + off[i] / 4u));
            st_global(reinterpret_cast<f32x4*>(L.y + off[i] / 4u), v);
        }
    }
}

template <int BM, bool XF32, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BM == 64 ? 2 : 1)))
void gemm_kernel(const GemmBatch b)
{
    constexpr int MT = BM / 16;              // M tiles per wave
    constexpr int AC = BM * 4 / 256;         // 8-k activation chunks per thread per step
    constexpr int AV = XF32 ? 2 : 1;         // 16-byte loads per chunk
    // [buffer][k block][row], fp16 in dequant order; one spare row per k block keeps the 4 k
    // blocks of a row (written by adjacent threads) in different banks
    __shared__ u32x4 As[2][4][BM + 1];

    // workgroup -> (linear, N tile, M tile, segment); consecutive numbers share an XCD (the
    // hardware deals workgroups out to the 8 XCDs in turn), so a strip's M tiles and segments
    // meet its weights in one L2
    const int bid = blockIdx.x;
    const int n8 = b.wg_total / 8 * 8;
    const int wg = bid < n8 ? (bid % 8) * (n8 / 8) + bid / 8 : bid;
    int li = 0;
    while (li + 1 < b.count && wg >= b.L[li + 1].wg_begin) li++;
    const GemmLinear& L = b.L[li];
    const int N = L.N, K = L.K, M = b.M;
    int local = wg - L.wg_begin;
    const int split = L.split;
    const int seg = local % split;
    local /= split;
    const int mt = local % L.tiles_m;
    const int nt = local / L.tiles_m;
    const int groups = K / L.group;
    const int spg = L.group / 32;                           // K steps per group
    const int ga = seg * groups / split, gb = (seg + 1) * groups / split;
    const int s0 = ga * spg, S = (gb - ga) * spg;           // this segment's steps

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kq = lane >> 4;
    const int ncol = nt * kCols + wave * 64 + 4 * j;        // this lane's 4 columns
    const bool col_ok = ncol < N;                           // N % 4 == 0: all 4 or none
    const int nc = col_ok ? ncol : 0;                       // loads stay inside the tensors
    const int m0 = mt * BM;
    const int NZ = (N + 7) >> 3;
    const uint32_t zshift = 4 * (nc & 7);                   // 0 or 16

    const uint32_t* qw = L.qweight + nc + (size_t)kq * N;
    const uint16_t* sc = L.scales + nc;
    // every load is unconditional (a conditional one makes the compiler drain the whole ring)
    const uint32_t* qz = L.qzeros ? L.qzeros + (nc >> 3) : &kSymZeros;
    const int zstride = L.qzeros ? NZ : 0;

    // activation chunk c = threadIdx.x + 256 a: row c / 4, k block c % 4 (rows past M read row
    // M - 1; their results land in rows that are never stored)
    const void* xb = L.x;
    size_t xrow[AC];
    int arow[AC], akb[AC];
#pragma unroll
    for (int a = 0; a < AC; a++) {
        const int c = threadIdx.x + 256 * a;
        arow[a] = c >> 2;
        akb[a] = c & 3;
        xrow[a] = (size_t)min(m0 + arow[a], M - 1) * K + 8 * akb[a];
    }

    u32x4 wq[D], xa[D][AC * AV];
    u32x2 sv[D];
    uint32_t zv[D];
    auto load = [&](int d, int s) {
        const int sa = s0 + s;
        const int g = sa / spg;
        wq[d] = ld_global(reinterpret_cast<const u32x4*>(qw + (size_t)sa * 4 * N));
        sv[d] = ld_global(reinterpret_cast<const u32x2*>(sc + (size_t)g * N));
        zv[d] = ld_global(qz + (size_t)g * zstride);
#pragma unroll
        for (int a = 0; a < AC; a++) {
            if (XF32) {
                const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(xb) + xrow[a] + 32 * sa);
                xa[d][2 * a] = ld_global(p);
                xa[d][2 * a + 1] = ld_global(p + 1);
            } else {
                xa[d][a] = ld_global(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(xb) + xrow[a] + 32 * sa));
            }
        }
    };

    f32x4 acc[MT][4];
#pragma unroll
    for (int tm = 0; tm < MT; tm++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[tm][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // one K step: this step's activations into LDS buffer d & 1 (its last readers finished
    // before the previous step's barrier), then 4 x MT MFMAs
    auto step = [&](int d) {
        // pin the raw activations and packed words here: otherwise the f32 -> f16 conversion
        // and the dequantization of all D steps are hoisted to the top of the ring's round,
        // whose first wait then drains every load in flight (vmcnt(0) once per D steps)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int a = 0; a < AC * AV; a++) pin(xa[d][a]);
        pin(wq[d]);
        {
            uint32_t s0 = sv[d].x, s1 = sv[d].y, z0 = zv[d];
            asm volatile("" : "+v"(s0), "+v"(s1), "+v"(z0));
            sv[d] = u32x2{s0, s1};
            zv[d] = z0;
        }
#pragma unroll
        for (int a = 0; a < AC; a++)
            As[d & 1][akb[a]][arow[a]] = XF32 ? perm_f32(xa[d][2 * a], xa[d][2 * a + 1]) : perm_f16(xa[d][a]);
        __syncthreads();
        f16x8 bf[4];
        const uint32_t zw = zv[d] >> zshift;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t sbits = (t < 2 ? sv[d].x : sv[d].y) >> (16 * (t & 1)) & 0xFFFFu;
            bf[t] = dequant_word_perm(wq[d][t], zero_pair(((zw >> (4 * t)) & 15u) + 1u), sbits * 0x10001u);
        }
#pragma unroll
        for (int tm = 0; tm < MT; tm++) {
            const f16x8 af = __builtin_bit_cast(f16x8, As[d & 1][kq][16 * tm + j]);
#pragma unroll
            for (int t = 0; t < 4; t++) acc[tm][t] = mfma_16x16x32_f16(af, bf[t], acc[tm][t]);
        }
    };
    // ring of D steps; loads past the segment's end repeat its last step (never consumed)
#pragma unroll
    for (int d = 0; d < D; d++) load(d, min(d, S - 1));
    int s = 0;
    for (; s + D <= S; s += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            step(d);
            load(d, min(s + d + D, S - 1));
        }
    }
#pragma unroll
    for (int d = 0; d < D; d++)
        if (s + d < S) step(d);

    gemm_store<MT>(L, M, m0, nt, mt, seg, split, ncol, col_ok, kq, acc);
}

// The same tiles for f16 activations and groups that are a multiple of 128, in 128-k chunks (4 MFMA
// k blocks). Per chunk:
// * the activations of the chunk (BM rows x 128 k) go to LDS once, behind one barrier, from a
//   2-slot register ring whose refill is issued as soon as a slot is written to LDS;
// * scale and zero pairs are prepared once (one group covers the whole chunk);
// * each k block reads all MT of its A fragments into registers one block ahead of its MFMAs,
//   and each k block's packed words are refilled (2-slot ring) as soon as they are dequantized.
// One wave per SIMD (BM = 128) or two (BM = 64): the accumulators take 128 / 64 registers.
template <int BM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BM == 64 ? 2 : 1)))
void gemm_chunk_kernel(const GemmBatch b)
{
    constexpr int MT = BM / 16;              // M tiles per wave
    constexpr int AC = BM / 16;              // 16-byte activation pieces per thread per chunk
    // [buffer][k block][k quarter][row], fp16 in dequant order; the spare row staggers banks
    __shared__ u32x4 As[2][4][4][BM + 1];

    const int bid = blockIdx.x;
    const int n8 = b.wg_total / 8 * 8;
    const int wg = bid < n8 ? (bid % 8) * (n8 / 8) + bid / 8 : bid;
    int li = 0;
    while (li + 1 < b.count && wg >= b.L[li + 1].wg_begin) li++;
    const GemmLinear& L = b.L[li];
    const int N = L.N, K = L.K, M = b.M;
    int local = wg - L.wg_begin;
    const int split = L.split;
    const int seg = local % split;
    local /= split;
    const int mt = local % L.tiles_m;
    const int nt = local / L.tiles_m;
    const int groups = K / L.group;
    const int cpg = L.group / 128;                          // chunks per group
    const int ga = seg * groups / split, gb = (seg + 1) * groups / split;
    const int c0 = ga * cpg, S = (gb - ga) * cpg;           // this segment's chunks

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kq = lane >> 4;
    const int ncol = nt * kCols + wave * 64 + 4 * j;
    const bool col_ok = ncol < N;
    const int nc = col_ok ? ncol : 0;
    const int m0 = mt * BM;
    const int NZ = (N + 7) >> 3;
    const uint32_t zshift = 4 * (nc & 7);

    const uint32_t* qw = L.qweight + nc + (size_t)kq * N;
    const uint16_t* sc = L.scales + nc;
    const uint32_t* qz = L.qzeros ? L.qzeros + (nc >> 3) : &kSymZeros;
    const int zstride = L.qzeros ? NZ : 0;

    // activation piece a: row c / 16, 8-k piece c % 16 (k block (c % 16) / 4, quarter c % 4)
    const uint16_t* xb = static_cast<const uint16_t*>(L.x);
    size_t xrow[AC];
    int arow[AC], apc[AC];
#pragma unroll
    for (int a = 0; a < AC; a++) {
        const int c = threadIdx.x + 256 * a;
        arow[a] = c >> 4;
        apc[a] = c & 15;
        xrow[a] = (size_t)min(m0 + arow[a], M - 1) * K + 8 * apc[a];
    }

    u32x4 xa[2][AC];
    u32x4 wq[2][4];
    u32x2 sv[2];
    uint32_t zv[2];
    auto load_x = [&](int d, int c) {
        const size_t k0 = (size_t)(c0 + c) * 128;
#pragma unroll
        for (int a = 0; a < AC; a++) xa[d][a] = ld_global(reinterpret_cast<const u32x4*>(xb + xrow[a] + k0));
    };
    auto load_w = [&](int d, int kb, int c) {
        const int p = (c0 + c) * 16 + 4 * kb;           // packed row of k quarter 0
        wq[d][kb] = ld_global(reinterpret_cast<const u32x4*>(qw + (size_t)p * N));
    };
    auto load_sz = [&](int d, int c) {
        const int g = (c0 + c) / cpg;
        sv[d] = ld_global(reinterpret_cast<const u32x2*>(sc + (size_t)g * N));
        zv[d] = ld_global(qz + (size_t)g * zstride);
    };

    f32x4 acc[MT][4];
#pragma unroll
    for (int tm = 0; tm < MT; tm++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[tm][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // chunk c from ring slot d (= c & 1); loads past the segment's end repeat its last chunk
    auto chunk = [&](int d, int c) {
        // keep each chunk's work in its own region: hoisting the next chunk's scale/zero work
        // above this point would wait for loads issued just before
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int a = 0; a < AC; a++) pin(xa[d][a]);
#pragma unroll
        for (int a = 0; a < AC; a++) As[d][apc[a] >> 2][apc[a] & 3][arow[a]] = perm_f16(xa[d][a]);
        load_x(d, min(c + 2, S - 1));
        uint32_t zz[4], ss[4];
        {
            const uint32_t zw = zv[d] >> zshift;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                zz[t] = zero_pair(((zw >> (4 * t)) & 15u) + 1u);
                ss[t] = (((t < 2 ? sv[d].x : sv[d].y) >> (16 * (t & 1))) & 0xFFFFu) * 0x10001u;
            }
        }
        load_sz(d, min(c + 2, S - 1));
        __syncthreads();
        u32x4 af[2][MT];
#pragma unroll
        for (int tm = 0; tm < MT; tm++) af[0][tm] = As[d][0][kq][16 * tm + j];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            if (kb < 3) {
#pragma unroll
                for (int tm = 0; tm < MT; tm++) af[(kb + 1) & 1][tm] = As[d][kb + 1][kq][16 * tm + j];
            }
            f16x8 bf[4];
#pragma unroll
            for (int t = 0; t < 4; t++) bf[t] = dequant_word_perm(wq[d][kb][t], zz[t], ss[t]);
            load_w(d, kb, min(c + 2, S - 1));
#pragma unroll
            for (int tm = 0; tm < MT; tm++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    acc[tm][t] = mfma_16x16x32_f16(__builtin_bit_cast(f16x8, af[kb & 1][tm]), bf[t], acc[tm][t]);
        }
    };

#pragma unroll
    for (int d = 0; d < 2; d++) {
        const int c = min(d, S - 1);
        load_x(d, c);
#pragma unroll
        for (int kb = 0; kb < 4; kb++) load_w(d, kb, c);
        load_sz(d, c);
    }
    int c = 0;
    for (; c + 2 <= S; c += 2) {
        chunk(0, c);
        chunk(1, c + 1);
    }
    if (c < S) chunk(0, c);

    gemm_store<MT>(L, M, m0, nt, mt, seg, split, ncol, col_ok, kq, acc);
}

template <int BM, bool XF32>
hipError_t launch_bm(const GemmBatch& b, hipStream_t stream)
{
    // f32 activations take twice the registers per step
    constexpr int D = XF32 ? QL_GEMM_DEPTH_F32 : QL_GEMM_DEPTH;
    hipLaunchKernelGGL((gemm_kernel<BM, XF32, D>), dim3(b.wg_total), dim3(256), 0, stream, b);
    return hipGetLastError();
}

}  // namespace

bool gemm_fast_ok(int M, int N, int K, int group)
{
    return M > kGemvMaxM && N > 0 && K > 0 && N % 4 == 0 && group >= 32 && group % 32 == 0 && K % group == 0;
}

GemmShape gemm_shape(int M, int N, int K, int group, int cu_count)
{
    GemmShape s;
    s.tiles_n = (N + kCols - 1) / kCols;
    // 128-row tiles once they alone give every CU a workgroup, else 64; groups of 128 or 256 run
    // the chunked kernel, whose 64-row instance keeps two waves per SIMD (its 128-row form would
    // spill into the accumulation registers)
    s.bm = group % 128 != 0 && (long)s.tiles_n * ((M + 127) / 128) >= cu_count ? 128 : 64;
    s.tiles_m = (M + s.bm - 1) / s.bm;
    const int tiles = s.tiles_n * s.tiles_m;
    const int groups = K / group;
    const int steps_per_group = group / 32;
    const int max_split = std::max(1, groups * steps_per_group / QL_GEMM_MIN_STEPS);
    // a K split pays for its partial-sum round trip only when the tiles leave most CUs idle
    const int want = tiles * 2 >= cu_count ? 1 : (QL_GEMM_TARGET_WGS * cu_count + tiles - 1) / tiles;
    s.split = std::max(1, std::min({want, max_split, groups}));
    // partial sums are addressed with 32-bit byte offsets
    while (s.split > 1 && (uint64_t)s.split * M * N * 4 >= (1ull << 31)) s.split--;
    return s;
}

uint64_t gemm_partial_bytes(int M, int N, int split)
{
    return split > 1 ? (uint64_t)split * M * N * 4 : 0;
}

hipError_t launch_gemm_batch(const GemmBatch& b, hipStream_t stream)
{
    if (b.count < 1 || b.count > kMaxBatch || b.wg_total < 1) return hipErrorInvalidValue;
    const int bm = b.bm;
    for (int i = 1; i < b.count; i++)
        if (b.L[i].wg_begin <= b.L[i - 1].wg_begin) return hipErrorInvalidValue;
    bool chunked = b.x_dtype != 0;          // f16 activations, groups of 128 or 256
    for (int i = 0; i < b.count; i++) chunked &= b.L[i].group % 128 == 0;
    if (chunked) {
        if (bm != 64) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gemm_chunk_kernel<64>, dim3(b.wg_total), dim3(256), 0, stream, b);
        return hipGetLastError();
    }
    if (bm == 64) return b.x_dtype == 0 ? launch_bm<64, true>(b, stream) : launch_bm<64, false>(b, stream);
    if (bm == 128) return b.x_dtype == 0 ? launch_bm<128, true>(b, stream) : launch_bm<128, false>(b, stream);
    return hipErrorInvalidValue;
}

}  // namespace ql
