// Linear sequences: the decode linears of a forward (M = 1..16 rows) in ONE persistent launch.
//
// The reference records every dispatch of a forward into one command batch and separates
// dependent dispatches with pass breaks (src/gpu/pipeline.ts:71-116, src/model/qwen.ts:382-387,
// :556-559); each pass break drains the GPU. Here the whole sequence is one kernel whose
// workgroups stay resident and order the work themselves:
//
// * Work is cut into tasks, planned on the host and dealt to workgroups round-robin pass by
//   pass: GEMV tiles (64 output columns x a K segment of whole groups; the four waves split the
//   segment and add their sums through LDS in a fixed order) and, for linears split across
//   workgroups, reductions of the segments' partial sums (ascending segment order). A workgroup
//   runs its list in order; every task waits only on tasks of earlier passes (a reduction on its
//   own pass's tiles), so with all workgroups resident the earliest unfinished task can run.
// * Results travel as 8-byte words (value bits | epoch << 32) written with single-copy-atomic
//   stores. A reader polls the words it needs until every epoch matches, so producers need no
//   fence, counter or flag, and a reader pays one round trip when its input is already there.
// * The epoch is this run's ticket: each workgroup takes one from one of 32 sub-counters at start
//   (run r gives every workgroup r). Nothing is cleared between runs, so a captured graph can
//   replay the launch.
// * Weights do not depend on activations: a workgroup starts loading its next tile's packed
//   words before it waits for that tile's inputs, so the memory pipe stays busy across passes.
// * Every wait is bounded. A wait that runs out sets a shared abort word and an error code; every
//   other wait sees the abort word and returns, so the grid always drains.
#include <algorithm>
#include <cstdio>
#include <string>
#include <vector>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

// Tunables (compile-time):
//   QL_SEQ_PREFETCH      groups each wave keeps in flight (jobs per wave padded to a multiple)
//   QL_SEQ_PREFETCH_WIDE the same for M > 8 (one workgroup per CU leaves registers for more)
//   QL_SEQ_WAVES         waves per workgroup for M <= 8 with groups of at most 128 (8 or 4)
//   QL_SEQ_CLASS_CUT     1: a streaming pass gives every workgroup an equal share of each
//                        (K, N) shape class; 0: one cut over all the pass's linears
//   QL_SEQ_STREAM_KB     weight KiB per workgroup from which a pass is planned for streaming
//                        (several evenly split blocks per workgroup) instead of one block each
//   QL_SEQ_MIN_GROUPS    fewest groups per K segment when a linear is split across workgroups
//   QL_SEQ_WHOLE_GROUPS  a latency-bound linear of at most this many groups is not split along K
//                        (walking its groups costs less than the reduction's round trip: 7B o,
//                        28 groups, measured faster whole; 0.5B down, 38 groups, split)
//   QL_SEQ_WG_PER_CU     resident workgroups per CU the grid is sized for
//   QL_SEQ_PRO_CHUNKS    8-value input chunks per lane whose loads a tile's prologue issues together
//   QL_SEQ_SENTINEL      1: a tile first polls one word per 64-value input chunk (wave 0), then
//                        loads its input; 0: every lane polls its own input words (one round trip
//                        less per dependent pass; measured faster on 0.5B- and 7B-shaped chains)
//   QL_SEQ_BLOCK_MODE    1: tiles of fewer groups than waves may run in block mode (below)
//   QL_SEQ_TILE_COST_MALL block-groups a tile's fixed work (prologue, pipeline drain) is priced
//                        at when a streaming pass whose weights fit the MALL is cut into runs
//   QL_SEQ_TILE_COST     the same for passes streamed from HBM with M > 1 (M = 1 measured best
//                        with equal block-groups per run: 0)
#ifndef QL_SEQ_BLOCK_MODE
#define QL_SEQ_BLOCK_MODE 1
#endif
#ifndef QL_SEQ_TILE_COST_MALL
#define QL_SEQ_TILE_COST_MALL 64
#endif
#ifndef QL_SEQ_TILE_COST
#define QL_SEQ_TILE_COST 48
#endif
#ifndef QL_SEQ_SENTINEL
#define QL_SEQ_SENTINEL 0
#endif
#ifndef QL_SEQ_PREFETCH
#define QL_SEQ_PREFETCH 2
#endif
#ifndef QL_SEQ_PREFETCH_WIDE
#define QL_SEQ_PREFETCH_WIDE 4
#endif
#ifndef QL_SEQ_CLASS_CUT
#define QL_SEQ_CLASS_CUT 0
#endif
#ifndef QL_SEQ_WAVES
#define QL_SEQ_WAVES 8
#endif
#ifndef QL_SEQ_PRO_CHUNKS
#define QL_SEQ_PRO_CHUNKS 1
#endif
#ifndef QL_SEQ_STREAM_KB
#define QL_SEQ_STREAM_KB 32
#endif
#ifndef QL_SEQ_MIN_GROUPS
#define QL_SEQ_MIN_GROUPS 4
#endif
#ifndef QL_SEQ_WHOLE_GROUPS
#define QL_SEQ_WHOLE_GROUPS 32
#endif
#ifndef QL_SEQ_WG_PER_CU
#define QL_SEQ_WG_PER_CU 2
#endif
constexpr int kMinGroups = QL_SEQ_MIN_GROUPS;
// Dynamic LDS (activation digits) per workgroup. Every variant runs one workgroup per CU (160 KB
// of LDS), of which the reduction ring takes up to 32 KB and the staged bias 16 KB.
size_t lds_budget(int, int) { return (size_t)104 << 10; }
constexpr int kCols = kSeqTileCols;     // 64 output columns per tile
constexpr int kSumBatch = 16;           // partial sums a reduction loads per round trip
// a pass with at least this many weight bytes per workgroup streams from HBM (7B-shaped linears)
// rather than waiting on latency (0.5B-shaped linears, MALL-resident)
constexpr uint64_t kStreamBytes = (uint64_t)QL_SEQ_STREAM_KB << 10;
// weight bytes of a pass that stay resident in MI355X's 256 MB MALL across steps (with room
// for activations and the exchange buffers)
constexpr uint64_t kMallBytes = 192ull << 20;

size_t lds_per_group(int M, int group) { return (size_t)(group / 64) * 4 * (4 * M) * 16 + 8 * (size_t)M; }

// The task and linear tables are written once, before any launch: reading them through the
// constant address space lets the compiler use scalar loads, which do not wait behind the
// vector-memory queue (the weight prefetch).
template <typename T>
__device__ __forceinline__ T ld_const(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    // through an integer: a direct cast of a kernel argument's pointer is folded back into the
    // global address space, where loads that follow any store are vector loads
    return *(const __attribute__((address_space(4))) T*)(reinterpret_cast<uintptr_t>(p));
#else
    return *p;   // host pass: never executed
#endif
}


// A pointer every lane holds, moved to scalar registers.
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const T*>((hi << 32) | lo);
}

// The epoch-tagged exchange words, as single-copy-atomic 32/64-bit global accesses.
__device__ __forceinline__ uint32_t ld_word(const uint32_t* p)
{
    return __hip_atomic_load(QL_GLOBAL(const uint32_t, p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_ll(const uint64_t* p)
{
    return __hip_atomic_load(QL_GLOBAL(const uint64_t, p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ll(uint64_t* p, float v, uint32_t e)
{
    __hip_atomic_store(QL_GLOBAL(uint64_t, p), (uint64_t)__float_as_uint(v) | ((uint64_t)e << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ void raise_abort(const SeqArgs& a, uint32_t code)
{
    uint32_t expected = 0u;
    __hip_atomic_compare_exchange_strong(QL_GLOBAL(uint32_t, a.err), &expected, code, __ATOMIC_RELAXED,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(QL_GLOBAL(uint32_t, a.abort), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called between polls of a wait loop; false when the wait must give up.
__device__ __forceinline__ bool keep_waiting(const SeqArgs& a, uint32_t& n)
{
    if ((++n & 63) == 0) {
        if (ld_word(a.abort) != 0) return false;
        if (n >= a.spin_limit) {
            raise_abort(a, kSeqErrTimeout);
            return false;
        }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

// Waits until all `cnt` (<= MAXN) words at p, p + stride, ... carry epoch e (loads issued
// together: one round trip) and adds their values to *sum in order.
template <int MAXN>
__device__ bool sum_ll(const uint64_t* p, size_t stride, int cnt, uint32_t e, const SeqArgs& a,
                       float* sum)
{
    uint64_t w[MAXN];
#pragma unroll
    for (int k = 0; k < MAXN; k++) w[k] = k < cnt ? ld_ll(p + k * stride) : (uint64_t)e << 32;
    uint32_t n = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < MAXN; k++) ready = ready && (uint32_t)(w[k] >> 32) == e;
        if (ready) break;
        if (!keep_waiting(a, n)) return false;
#pragma unroll
        for (int k = 0; k < MAXN; k++)
            if ((uint32_t)(w[k] >> 32) != e) w[k] = ld_ll(p + k * stride);
    }
    float s = *sum;
#pragma unroll
    for (int k = 0; k < MAXN; k++)
        if (k < cnt) s += __uint_as_float((uint32_t)w[k]);
    *sum = s;
    return true;
}

// One lane per word: waits until the word at p + lane * stride (lane < cnt) carries epoch e.
// Readers poll one word per producer chunk this way before loading the chunks in bulk, so a
// waiting workgroup costs the memory system a few loads per poll, not its whole input.
__device__ bool wait_words(const uint64_t* p, size_t stride, int cnt, int lane, uint32_t e,
                           const SeqArgs& a)
{
    for (int c = lane; c < cnt; c += 64) {
        uint32_t n = 0;
        while ((uint32_t)(ld_ll(p + c * stride) >> 32) != e)
            if (!keep_waiting(a, n)) return false;
    }
    return true;
}

// Eight consecutive values of a producer's output: issue the loads now, finish later, so the
// next chunk's loads can be in flight while this one is turned into digits.
__device__ __forceinline__ void issue8_ll(const uint64_t* p, uint64_t w[8])
{
#pragma unroll
    for (int k = 0; k < 8; k++) w[k] = ld_ll(p + k);
}

// Waits until all eight words carry epoch e (re-polling stragglers) and unpacks the values.
__device__ bool finish8_ll(const uint64_t* p, uint32_t e, uint64_t w[8], float v[8], const SeqArgs& a)
{
    uint32_t n = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int k = 0; k < 8; k++) ready = ready && (uint32_t)(w[k] >> 32) == e;
        if (ready) break;
        if (!keep_waiting(a, n)) return false;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if ((uint32_t)(w[k] >> 32) != e) w[k] = ld_ll(p + k);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = __uint_as_float((uint32_t)w[k]);
    return true;
}

// Block mode for a tile of `nblk` blocks over a segment of `gseg` groups on W waves (see the
// kernel): segments shorter than W groups, when the busiest wave has no more jobs than under the
// K split plus a quarter job per block for the ring. The planner and the kernel use the same rule.
__host__ __device__ constexpr bool block_mode_for(int gseg, int nblk, int W)
{
    return QL_SEQ_BLOCK_MODE && gseg < W &&
           4 * ((nblk + W - 1) / W * gseg) <= 4 * (nblk * ((gseg + W - 1) / W)) + nblk;
}

// One wave's view of a tile for its weight loads: the tile's blocks ct .. ct+nblk-1 and the
// wave's groups g0 .. g0+wcount-1 of the tile's K segment. Every field is wave-uniform, so
// selecting one view or another stays scalar.
struct FetchSrc {
    const uint32_t* qweight;
    const uint32_t* qzeros;
    const uint16_t* scales;
    int N, ct, nblk, g0, wcount;
    int b0, bs;                 // the wave's first block of the tile and its block step
};

template <int T, int NB, int RG, int kP, int W, bool BMODE, bool FU>
__global__ __launch_bounds__(64 * W) void seq_kernel(const SeqArgs a)
{
    constexpr int kThreads = 64 * W;
    // dynamic LDS: activation digits [block][kq][row] (16 B), then {2^-E, Sx}[group][m]
    extern __shared__ uint4 dyn_lds[];
    // Ring of RG slots for the waves' sums of a 64-column block, [slot][wave][m][column]. Each
    // wave writes its sums and counts itself in (ring_arrive); the last to arrive adds the W sums
    // in wave order, stores the block and marks the slot free (ring_done = the block's sequence
    // number). Waves therefore never wait for each other between blocks, only for a slot a full
    // ring behind.
    __shared__ float red[RG][W][4 * T][kCols];
    __shared__ int ring_arrive[RG];
    __shared__ int ring_done[RG];
    // the bias of a tile's columns, staged by the prologue (tiles that write whole outputs)
    __shared__ float bias_lds[kSeqBiasBlocks * kCols];
    __shared__ uint32_t sh_epoch;
    __shared__ int sh_bad;
    // fused RMSNorm: 1/rms of each input row of the current task's linear (written by the last
    // wave before a barrier, read by every wave after it)
    __shared__ float sh_rstd[FU ? 4 * T : 1];

    const int wg = blockIdx.x;
    const int lane = threadIdx.x & 63;
    // wave-uniform (scalar) so that per-wave branches stay scalar: an exec-masked branch around
    // the MFMA loop makes the compiler drain every load in flight
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int M = a.M;
    const int R = 4 * M;
    constexpr int GK = NB * 64;
    constexpr int CPG = NB * 8;             // lanes per (group, row) in the prologue

    const int tb = ld_const(a.task_begin + wg);
    const int te = ld_const(a.task_begin + wg + 1);
    const int first = ld_const(a.first_tile + wg);

    // Two ways to share a tile among the waves:
    // * K split: the waves split the segment into contiguous parts of floor or ceil(gseg / W)
    //   groups (wave w takes local groups [w*gseg/W, (w+1)*gseg/W)) and every block's W partial
    //   sums meet in the LDS ring;
    // * block mode: wave w takes blocks w, w + W, ... over the whole segment and stores each
    //   block's sums itself (no ring, no wave without work while nblk >= W).
    // Block mode (block_mode_for) serves short segments: K = 896 has 7 groups for 8 waves. On
    // longer segments the K split measured faster even at equal job counts. Its code is only in
    // the BMODE instance, which the launcher picks for plans that have such tiles: the extra
    // registers slow the latency-bound tiles of other plans.
    auto wave_lo = [&](int gseg) { return wave * gseg / W; };
    auto block_mode = [&](int gseg, int nblk) { return BMODE && block_mode_for(gseg, nblk, W); };
    auto src_of = [&](int ti) {
        // uniform index: the table reads become scalar loads, which the weight prefetch does
        // not have to drain before the fields are used
        const SeqTask t = ld_const(a.tasks + __builtin_amdgcn_readfirstlane(ti));
        const SeqLinear* L = a.lin + t.linear;
        FetchSrc f;
        f.qweight = uniform_ptr(ld_const(&L->qweight));
        f.qzeros = uniform_ptr(ld_const(&L->qzeros));
        f.scales = uniform_ptr(ld_const(&L->scales));
        f.N = __builtin_amdgcn_readfirstlane(ld_const(&L->N));
        const int gseg = t.g1 - t.g0;
        if (block_mode(gseg, t.nblk)) {
            f.g0 = t.g0;
            f.wcount = gseg;
            f.b0 = wave;
            f.bs = W;
        } else {
            f.g0 = t.g0 + wave_lo(gseg);
            f.wcount = t.g0 + (wave + 1) * gseg / W - f.g0;
            f.b0 = 0;
            f.bs = 1;
        }
        f.ct = t.ct;
        f.nblk = t.nblk;
        return f;
    };

    // Fused residual of output (m, n) of linear L: an external input or a producer's output word
    // (waited for like any input; the producer ran in an earlier pass).
    auto residual = [&](const SeqFuseLin* F, int m, int n, int N, uint32_t e, bool& ok) -> float {
        const int rs = ld_const(&F->res_src);
        if (rs < 0) return ld_global(uniform_ptr(ld_const(&F->res)) + (size_t)m * N + n);
        const uint64_t* w = uniform_ptr(ld_const(&a.lin[rs].y_ll)) + (size_t)m * N + n;
        uint64_t v = ld_ll(w);
        uint32_t polls = 0;
        while ((uint32_t)(v >> 32) != e && ok) {
            if (!keep_waiting(a, polls)) ok = false;
            else v = ld_ll(w);
        }
        return __uint_as_float((uint32_t)v);
    };

    // The sum of squares of one stored row of a 64-column block (lane = column, 0 past N), for a
    // consumer that normalizes this output: one epoch word per (row, block), added over the
    // wave's lanes in a fixed order.
    auto emit_ssq = [&](uint64_t* ssq, int N, int m, int blk, float v, uint32_t e) {
        float q = v * v;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o);
        if (lane == 0) st_ll(ssq + (size_t)m * ((N + kCols - 1) / kCols) + blk, q, e);
    };

    // Fused RMSNorm: 1/rms of each input row of linear L into sh_rstd, computed by the calling wave
    // alone (before a barrier that publishes it). With a producer that emits sums of squares (one
    // word per row and 64-column block), lane l adds the row's words l, l + 64, ... and an xor
    // butterfly adds the lanes; all rows' loads go out together, so this costs one round trip.
    // Otherwise (an external input) the row itself is read. The order of additions is fixed, so
    // every task and every run gets the same values.
    auto rows_rstd = [&](const SeqLinear& L, const SeqFuseLin* F, uint32_t e, bool& ok) {
        const float eps = ld_const(&F->norm_eps);
        const uint64_t* pss = L.src >= 0 ? ld_const(&a.fl[L.src].ssq) : nullptr;
        float ss[4 * T];
#pragma unroll
        for (int m = 0; m < 4 * T; m++) ss[m] = 0.f;
        if (pss) {
            pss = uniform_ptr(pss);
            const int nbk = L.K / kCols;
            for (int c0 = 0; c0 < nbk && ok; c0 += 64) {
                const int c = c0 + lane;
                uint64_t w[4 * T];
#pragma unroll
                for (int m = 0; m < 4 * T; m++)
                    w[m] = m < M && c < nbk ? ld_ll(pss + (size_t)m * nbk + c) : (uint64_t)e << 32;
                uint32_t polls = 0;
                for (;;) {
                    bool ready = true;
#pragma unroll
                    for (int m = 0; m < 4 * T; m++) ready = ready && (uint32_t)(w[m] >> 32) == e;
                    if (ready) break;
                    if (!keep_waiting(a, polls)) {
                        ok = false;
                        break;
                    }
#pragma unroll
                    for (int m = 0; m < 4 * T; m++)
                        if ((uint32_t)(w[m] >> 32) != e) w[m] = ld_ll(pss + (size_t)m * nbk + c);
                }
#pragma unroll
                for (int m = 0; m < 4 * T; m++)
                    if (m < M && c < nbk) ss[m] += __uint_as_float((uint32_t)w[m]);
            }
        } else {
            const uint64_t* pll = L.src >= 0 ? uniform_ptr(ld_const(&a.lin[L.src].y_ll)) : nullptr;
            const int cpr = L.K / 8;
            for (int m = 0; m < M; m++) {
                // the row's sum in a scalar, then into ss[m] by compile-time indices (a runtime
                // index into a register array would put ss in scratch memory)
                float rs = 0.f;
                for (int c = lane; c < cpr && ok; c += 64) {
                    const size_t xo = (size_t)m * L.K + (size_t)c * 8;
                    float v[8];
                    if (pll) {
                        uint64_t w[8];
                        issue8_ll(pll + xo, w);
                        ok = finish8_ll(pll + xo, e, w, v, a);
                    } else {
                        load8(L.x, L.x_dtype, xo, v);
                    }
#pragma unroll
                    for (int k = 0; k < 8; k++) rs = fmaf(v[k], v[k], rs);
                }
#pragma unroll
                for (int mm = 0; mm < 4 * T; mm++)
                    if (mm == m) ss[mm] += rs;
            }
        }
#pragma unroll
        for (int m = 0; m < 4 * T; m++) {
            float q = ss[m];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o);
            if (lane == 0 && m < M) sh_rstd[m] = (float)(1.0 / sqrt((double)q / (double)L.K + (double)eps));
        }
    };

    // Software pipeline over each wave's job stream. In a tile, the wave's job k is block
    // k / wcount, group g0 + k % wcount (blocks in order); the stream is padded to a multiple of
    // kP (at least kP) and continues into the next tile, so slot d always holds a job k with
    // k % kP == d and the loads stay kP jobs ahead across blocks and tiles. Padding loads
    // re-read the tile's first job (cached) and are never consumed. Loads are unconditional, so
    // the compiler waits for exactly the slot it consumes. Base pointers sit in scalar registers
    // and offsets stay 32-bit (every GPTQ tensor is far below 4 GiB).
    uint4 wb[kP][2 * NB];
    uint32_t zb[kP];
    uint2 sb[kP];
    // One wave's fetch cursor over a tile's jobs: scalar bases and byte offsets of the cursor's
    // group (one add per job), lane offsets of the cursor's block (recomputed per block; a
    // partial last block clamps its columns to the linear's last four). Past the tile's last job
    // the cursor stays there, so padding loads re-read cached data.
    struct Stream {
        const char* qw;
        const char* qz;
        const char* sc;
        uint32_t gq, gz, gs;               // byte offsets of the cursor's group
        uint32_t Gq, Gz, Gs;               // byte strides from one group to the next
        int b, bs, gi, wcount, nblk, ct, N;
        uint32_t lq[2 * NB], lz, ls;       // lane offsets of the cursor's block
    };
    auto set_lanes = [&](Stream& st) {
        const int nc = (st.ct + st.b) * kCols + 4 * j;
        const uint32_t n = (uint32_t)(nc < st.N ? nc : st.N - 4);
#pragma unroll
        for (int r = 0; r < 2 * NB; r++)
            st.lq[r] = ((uint32_t)(2 * kq + (r >> 1) * 8 + (r & 1)) * (uint32_t)st.N + n) * 4u;
        st.ls = n * 2u;
        st.lz = (n >> 3) * 4u;
    };
    auto open_stream = [&](const FetchSrc& f) {
        Stream st;
        st.qw = reinterpret_cast<const char*>(uniform_ptr(f.qweight));
        st.qz = reinterpret_cast<const char*>(uniform_ptr(f.qzeros));   // never null
        st.sc = reinterpret_cast<const char*>(uniform_ptr(f.scales));
        st.N = __builtin_amdgcn_readfirstlane(f.N);
        st.ct = __builtin_amdgcn_readfirstlane(f.ct);
        st.nblk = __builtin_amdgcn_readfirstlane(f.nblk);
        st.wcount = __builtin_amdgcn_readfirstlane(f.wcount);
        const uint32_t g0 = (uint32_t)__builtin_amdgcn_readfirstlane(f.g0);
        st.Gq = (uint32_t)(NB * 8) * (uint32_t)st.N * 4u;
        st.Gs = (uint32_t)st.N * 2u;
        st.Gz = (((uint32_t)st.N + 7u) >> 3) * 4u;
        st.gq = g0 * st.Gq;
        st.gs = g0 * st.Gs;
        st.gz = g0 * st.Gz;
        st.b = __builtin_amdgcn_readfirstlane(f.b0);
        st.bs = __builtin_amdgcn_readfirstlane(f.bs);
        st.gi = 0;
        set_lanes(st);
        return st;
    };
    auto advance = [&](Stream& st) {
        if (st.gi + 1 < st.wcount) {
            st.gi++;
            st.gq += st.Gq;
            st.gs += st.Gs;
            st.gz += st.Gz;
        } else if (st.wcount > 0 && st.b + st.bs < st.nblk) {
            // back to the wave's first group, on to the wave's next block
            const uint32_t back = (uint32_t)(st.wcount - 1);
            st.gi = 0;
            st.gq -= back * st.Gq;
            st.gs -= back * st.Gs;
            st.gz -= back * st.Gz;
            st.b += st.bs;
            set_lanes(st);
        }
    };
    auto fetch = [&](int d, const Stream& st) {
        // scalar base + 32-bit lane offset: one load instruction each
        const char* q = st.qw + st.gq;
#pragma unroll
        for (int r = 0; r < 2 * NB; r++)
            wb[d][r] = __builtin_bit_cast(uint4, ld_global(reinterpret_cast<const u32x4*>(q + st.lq[r])));
        zb[d] = ld_global(reinterpret_cast<const uint32_t*>(st.qz + st.gz + st.lz));
        sb[d] = __builtin_bit_cast(uint2, ld_global(reinterpret_cast<const u32x2*>(st.sc + st.gs + st.ls)));
    };

    // the first tile's first kP stream positions
    if (first >= 0) {
        Stream st = open_stream(src_of(first));
#pragma unroll
        for (int d = 0; d < kP; d++) {
            fetch(d, st);
            advance(st);
        }
    }

    if (threadIdx.x == 0) {
        const int sub = wg % kSeqTickets;
        const uint32_t members = (uint32_t)((a.G - 1 - sub) / kSeqTickets + 1);
        const unsigned long long old = __hip_atomic_fetch_add(QL_GLOBAL(unsigned long long, a.tickets + sub * 8), 1ull, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
        sh_epoch = (uint32_t)(old / members) + 1u;
        sh_bad = 0;
    }
    if (threadIdx.x < RG) {
        ring_arrive[threadIdx.x] = 0;
        ring_done[threadIdx.x] = (int)threadIdx.x - RG;   // as if blocks -RG .. -1 were done
    }
    __syncthreads();
    const uint32_t e = __builtin_amdgcn_readfirstlane(sh_epoch);   // uniform: scalar control flow
    int bseq = 0;              // this workgroup's blocks so far (ring position), across tiles

    for (int ti = tb; ti < te; ti++) {
        const SeqTask task = ld_const(a.tasks + ti);
        const SeqLinear L = ld_const(a.lin + task.linear);
        const int N = L.N;
        bool ok = true;

        if (task.kind == kSeqReduce) {
            // blocks ct .. ct+nblk-1: each the sum of its parts (consecutive pool slots, ascending
            // K order), plus bias. Each lane polls the parts of its own outputs as it loads them
            // (with QL_SEQ_SENTINEL, wave 0 first waits for one word of every slot).
            const int np = task.parts;
            const size_t slot_words = (size_t)M * kCols;
            const SeqFuseLin* F = FU ? a.fl + task.linear : nullptr;
            const int fz = FU ? task.fuse : 0;                  // carried by the task: no table read
            uint64_t* const fssq = FU && (fz & kFuseSsq) ? ld_const(&F->ssq) : nullptr;
            if constexpr (FU)
                if ((fz & kFuseNorm) && wave == W - 1) rows_rstd(L, F, e, ok);
            if (QL_SEQ_SENTINEL && wave == 0) {
                for (int l = lane; l < task.nblk * np && ok; l += 64) {
                    const int b = l / np;
                    const uint64_t* w0 = a.part + (size_t)(task.slot + b * task.stride + (l - b * np)) * slot_words;
                    uint32_t polls = 0;
                    while ((uint32_t)(ld_ll(w0) >> 32) != e)
                        if (!keep_waiting(a, polls)) {
                            ok = false;
                            break;
                        }
                }
            }
            if (!ok) sh_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
            // output (m, nn) of block b: its parts added in K order, then the epilogue
            // rstd * sum + (bias + residual); stored, and returned for the block's sum of squares
            auto reduce_one = [&](int b, int r, int m, int nn) -> float {
                const uint64_t* src = a.part + (size_t)(task.slot + b * task.stride) * slot_words + r;
                // the residual's load goes out with the parts' (its producer ran passes earlier)
                float add = L.bias ? ld_global(L.bias + nn) : 0.f;
                uint64_t rw = 0;
                const uint64_t* rp = nullptr;
                if constexpr (FU)
                    if (fz & kFuseRes) {
                        const int rs = ld_const(&F->res_src);
                        if (rs < 0) add += ld_global(uniform_ptr(ld_const(&F->res)) + (size_t)m * N + nn);
                        else {
                            rp = uniform_ptr(ld_const(&a.lin[rs].y_ll)) + (size_t)m * N + nn;
                            rw = ld_ll(rp);
                        }
                    }
                float sum = 0.f;
                for (int s0 = 0; s0 < np && ok; s0 += kSumBatch)
                    ok = sum_ll<kSumBatch>(src + (size_t)s0 * slot_words, slot_words, min(kSumBatch, np - s0),
                                           e, a, &sum);
                if constexpr (FU)
                    if (rp) {
                        uint32_t polls = 0;
                        while ((uint32_t)(rw >> 32) != e && ok) {
                            if (!keep_waiting(a, polls)) ok = false;
                            else rw = ld_ll(rp);
                        }
                        add += __uint_as_float((uint32_t)rw);
                    }
                if (!ok) return 0.f;
                if constexpr (FU)
                    if (fz & kFuseNorm) sum *= sh_rstd[m];
                sum += add;
                st_global(L.y + (size_t)m * N + nn, sum);
                st_ll(L.y_ll + (size_t)m * N + nn, sum, e);
                return sum;
            };
            for (int idx = threadIdx.x; idx < task.nblk * M * kCols; idx += kThreads) {
                const int b = idx / (M * kCols);
                const int r = idx - b * (M * kCols);
                const int m = r / kCols;
                const int nn = (task.ct + b) * kCols + (r - m * kCols);
                if constexpr (FU)
                    if (fssq) {
                        // one wave holds one (block, row): its 64 lanes are the block's columns
                        const float v = nn < N && ok ? reduce_one(b, r, m, nn) : 0.f;
                        emit_ssq(fssq, N, m, task.ct + b, v, e);
                        continue;
                    }
                if (nn >= N || !ok) continue;
                reduce_one(b, r, m, nn);
            }
            if (!ok) sh_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
            continue;
        }

        // ---- GEMV tile: blocks ct .. ct + nblk - 1 (64 columns each) over the segment [g0, g1) ----
        const int gseg = task.g1 - task.g0;
        const bool bmode = block_mode(gseg, task.nblk);
        const int wfirst = bmode ? 0 : wave_lo(gseg);                   // this wave's first group
        const int wcount = bmode ? gseg : (wave + 1) * gseg / W - wfirst; // and its number of groups
        // the wave's blocks: all of them (K split) or every W-th from its own index
        const int nbw = !bmode ? task.nblk : wave < task.nblk ? (task.nblk - 1 - wave) / W + 1 : 0;
        const bool P = L.src >= 0;
        const uint64_t* p_ll = P ? ld_const(&a.lin[L.src].y_ll) : nullptr;
        // fused staging: x -> rmsnorm(x) * w (NORM) or silu(x) * x2 (GLU)
        const SeqFuseLin* F = FU ? a.fl + task.linear : nullptr;
        const int fz = FU ? task.fuse : 0;                      // carried by the task: no table read
        const bool NORM = FU && (fz & kFuseNorm);
        const bool GLU = FU && (fz & kFuseGlu);
        const int src2 = GLU ? ld_const(&F->src2) : -1;
        const bool P2 = GLU && src2 >= 0;
        const uint64_t* p2_ll = P2 ? ld_const(&a.lin[src2].y_ll) : nullptr;
        // this tile's and the next tile's views, read now so that their table loads overlap the
        // prologue (without a next tile the stream's tail re-reads this tile)
        const FetchSrc cs = src_of(ti);
        const FetchSrc ns = task.next_tile >= 0 ? src_of(task.next_tile) : cs;

        // the segment's activation digits (shared by all blocks of the tile), from the external
        // input or from the producer's output words: wave 0 first waits for one word of each
        // 64-value chunk of the segment (one producer block's columns)
        if ((P || P2) && QL_SEQ_SENTINEL) {
            if (wave == 0) {
                const int c0 = task.g0 * GK / kCols;
                const int c1 = task.g1 * GK / kCols;
                if (P) ok = wait_words(p_ll + (size_t)c0 * kCols, kCols, c1 - c0, lane, e, a);
                if (P2 && ok) ok = wait_words(p2_ll + (size_t)c0 * kCols, kCols, c1 - c0, lane, e, a);
            }
            if (!ok) sh_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
        }
        uint4* xd = dyn_lds;
        float2* gst = reinterpret_cast<float2*>(dyn_lds + gseg * NB * 4 * R);
        // A tile that writes whole outputs finishes them where it stores them:
        // y = rstd * sum + (bias + residual) (rstd with a fused RMSNorm, the residual with a fused
        // add), then the block sums of squares for a consumer that normalizes y. The prologue
        // stages what that needs, in the round trip of the tile's own input: bias + residual
        // per (block, row, column) in bias_lds (rows only with a residual; the planner keeps
        // nblk * rows within kSeqBiasBlocks), taken from the highest threads down because the
        // input chunks occupy the lowest; and 1/rms per row in sh_rstd, from the last wave.
        const bool RES = FU && task.slot < 0 && (fz & kFuseRes);
        const int Mr = RES ? M : 1;
        {
            if (task.slot < 0 && (L.bias || RES))
                for (int idx = kThreads - 1 - (int)threadIdx.x; idx < task.nblk * Mr * kCols; idx += kThreads) {
                    const int b = idx / (Mr * kCols);
                    const int r = idx - b * (Mr * kCols);
                    const int m = r / kCols;
                    const int col = (task.ct + b) * kCols + (r - m * kCols);
                    float v = col < N && L.bias ? ld_global(L.bias + col) : 0.f;
                    if constexpr (FU)
                        if (RES && col < N) v += residual(F, m, col, N, e, ok);
                    bias_lds[idx] = v;
                }
            if constexpr (FU)
                if (NORM && task.slot < 0 && wave == W - 1) rows_rstd(L, F, e, ok);
            // QL_SEQ_PRO_CHUNKS chunks per trip: their input loads are all issued before any is used
            const int items = gseg * M;
            constexpr int H = QL_SEQ_PRO_CHUNKS;
            for (int base = 0; base < items * CPG; base += kThreads * H) {
                uint64_t w[H][8];
                float v[H][8];
                size_t xo[H];
                bool live[H];
#pragma unroll
                for (int h = 0; h < H; h++) {
                    const int idx = base + kThreads * h + threadIdx.x;
                    const int item = idx / CPG;
                    live[h] = item < items;
                    const int c = idx - item * CPG;
                    const int gg = item / M;
                    const int m = item - gg * M;
                    xo[h] = (size_t)m * L.K + (size_t)(task.g0 + gg) * GK + (size_t)c * 8;
                    if (live[h]) {
                        if (P) issue8_ll(p_ll + xo[h], w[h]);
                        else load8(L.x, L.x_dtype, xo[h], v[h]);
                    }
                }
                // the fused second operand (GLU) and norm weights of the same chunks
                uint64_t w2[FU ? H : 1][8];
                float v2[FU ? H : 1][8];
                if constexpr (FU) {
#pragma unroll
                    for (int h = 0; h < H; h++) {
                        if (!live[h]) continue;
                        if (P2) issue8_ll(p2_ll + xo[h], w2[h]);
                        else if (GLU) load8(uniform_ptr(ld_const(&F->x2)), 0, xo[h], v2[h]);
                        else if (NORM) {
                            const int idx = base + kThreads * h + threadIdx.x;
                            const int item = idx / CPG;
                            const int c = idx - item * CPG;
                            const int gg = item / M;
                            load8(uniform_ptr(ld_const(&F->norm_w)), 0, (size_t)(task.g0 + gg) * GK + (size_t)c * 8, v2[h]);
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < H; h++) {
                    const int idx = base + kThreads * h + threadIdx.x;
                    const int item = idx / CPG;                 // uniform per CPG lanes
                    if (!live[h]) continue;
                    const int c = idx - item * CPG;
                    const int gg = item / M;
                    const int m = item - gg * M;
                    if (P) {
                        if (ok) ok = finish8_ll(p_ll + xo[h], e, w[h], v[h], a);
                        if (!ok) {
#pragma unroll
                            for (int k = 0; k < 8; k++) v[h][k] = 0.f;
                        }
                    }
                    if constexpr (FU) {
                        if (P2) {
                            if (ok) ok = finish8_ll(p2_ll + xo[h], e, w2[h], v2[h], a);
                            if (!ok) {
#pragma unroll
                                for (int k = 0; k < 8; k++) v2[h][k] = 0.f;
                            }
                        }
                        if (GLU) {
                            // siluMulRef: silu(g) * u = g / (1 + exp(-g)) * u
#pragma unroll
                            for (int k = 0; k < 8; k++) v[h][k] = v[h][k] / (1.f + expf(-v[h][k])) * v2[h][k];
                        } else if (NORM) {
                            // x * w here; the row's 1/rms, a scalar, multiplies the dot products
                            // when the outputs are stored (the linear commutes with it), so the
                            // tile need not wait for the whole row before it starts
#pragma unroll
                            for (int k = 0; k < 8; k++) v[h][k] = v[h][k] * v2[h][k];
                        }
                    }
                    const int blk = gg * NB + (c >> 3);
                    const int ckq = (c & 7) >> 1;
                    uint2* rows = reinterpret_cast<uint2*>(&xd[(blk * 4 + ckq) * R + 4 * m]) + (c & 1);
                    const float2 st = prep_chunk<CPG>(v[h], rows, 2);
                    if (c == 0) gst[gg * M + m] = st;
                }
            }
        }
        if (!ok) sh_bad = 1;
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
        uint64_t* const fssq = FU && task.slot < 0 && (fz & kFuseSsq) ? ld_const(&F->ssq) : nullptr;
        // one finished output: rstd * sum + staged (bias + residual), stored as value and word
        auto finish = [&](int b, int m, int nc, float v) -> float {
            if constexpr (FU)
                if (NORM) v *= sh_rstd[m];
            if (L.bias || RES) v += bias_lds[(b * Mr + (RES ? m : 0)) * kCols + lane];
            st_global(L.y + (size_t)m * N + nc, v);
            st_ll(L.y_ll + (size_t)m * N + nc, v, e);
            return v;
        };

        float acc[4][T];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int t = 0; t < T; t++) acc[u][t] = 0.f;
            auto consume = [&](int gg, const uint4* w, uint32_t zn, uint2 sv) {
                i32x4 c[4][T];
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int t = 0; t < T; t++) c[u][t] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int bb = 0; bb < NB; bb++) {
                    i32x4 av[T];
#pragma unroll
                    for (int t = 0; t < T; t++) {
                        const int row = 16 * t + j;
                        av[t] = row < R ? __builtin_bit_cast(i32x4, xd[((gg * NB + bb) * 4 + kq) * R + row])
                                        : i32x4{0, 0, 0, 0};
                    }
                    const uint4 w0 = w[2 * bb], w1 = w[2 * bb + 1];
                    const uint32_t lo[4] = {w0.x, w0.y, w0.z, w0.w};
                    const uint32_t hi[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const i32x4 bq = i32x4{(int)(lo[u] & 0x0F0F0F0Fu), (int)((lo[u] >> 4) & 0x0F0F0F0Fu),
                                               (int)(hi[u] & 0x0F0F0F0Fu), (int)((hi[u] >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
                        for (int t = 0; t < T; t++) c[u][t] = mfma_i8(av[t], bq, c[u][t]);
                    }
                }
                const uint32_t zw = zn >> (4 * ((4 * j) & 7));
                const uint32_t sw[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
                float2 st[T];
#pragma unroll
                for (int t = 0; t < T; t++) {
                    const int m = 4 * t + kq;
                    st[t] = m < M ? gst[gg * M + m] : float2{0.f, 0.f};
                    st[t].x *= 0x1p-8f;       // the digit pairs below carry a factor 2^8
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
                    const float sz = s * (float)(((zw >> (4 * u)) & 15u) + 1u);
#pragma unroll
                    for (int t = 0; t < T; t++) {
                        // digit products (|c| < 2^18, digit 3 most significant) in two exact
                        // integer pairs: 2^8 * sum_d c_d 2^(8d-24) = (c0 + 2^8 c1) 2^-16 + (c2 + 2^8 c3)
                        const int lo = c[u][t][0] + c[u][t][1] * 256;
                        const int hi = c[u][t][2] + c[u][t][3] * 256;
                        const float v = fmaf((float)lo, 0x1p-16f, (float)hi);
                        acc[u][t] = fmaf(s * st[t].x, v, acc[u][t]);
                        acc[u][t] = fmaf(-sz, st[t].y, acc[u][t]);
                    }
                }
            };

        // Publishes this wave's sums of block b; the last wave to arrive adds the W sums in wave
        // order and stores the block (lane = column, rows m).
        auto publish = [&](int b) {
            const int rs = bseq % RG;
            {
                // the slot is free once the block a full ring back has been stored
                uint32_t polls = 0;
                while (__hip_atomic_load(&ring_done[rs], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < bseq - RG)
                    if (!keep_waiting(a, polls)) {
                        ok = false;
                        break;
                    }
            }
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int u = 0; u < 4; u++) red[rs][wave][4 * t + kq][4 * j + u] = acc[u][t];
            // LDS executes a wave's operations in order: the sums land before the arrival is
            // counted (the fence only keeps the compiler from reordering them)
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            int arrived = 0;
            if (lane == 0)
                arrived = __hip_atomic_fetch_add(&ring_arrive[rs], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            arrived = __builtin_amdgcn_readfirstlane(arrived);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if (arrived == W - 1) {
                const int ncol = (task.ct + b) * kCols + lane;
                for (int m = 0; m < M; m++) {
                    float v = 0.f;
                    if (ncol < N) {
                        v = red[rs][0][m][lane];
#pragma unroll
                        for (int w = 1; w < W; w++) v += red[rs][w][m][lane];
                        if (task.slot < 0) v = finish(b, m, ncol, v);
                        else st_ll(a.part + ((size_t)(task.slot + b * task.stride) * M + m) * kCols + lane, v, e);
                    }
                    if constexpr (FU)
                        if (fssq) emit_ssq(fssq, N, m, task.ct + b, v, e);
                }
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                if (lane == 0) {
                    ring_arrive[rs] = 0;
                    __hip_atomic_store(&ring_done[rs], bseq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
            bseq++;
        };

        // block mode: this wave's complete sums of block b, stored directly. Lane (j, kq) holds
        // columns 4j .. 4j+3 of row 4t + kq; a cross-lane exchange gives lane l column l, so each
        // row of the block goes out as one 64-lane store like the ring's (a consumer polls one
        // word per block and expects the others with it).
        auto store_block = [&](int b) {
            const int nc = (task.ct + b) * kCols + lane;
            const int u = lane & 3;
#pragma unroll
            for (int t = 0; t < T; t++) {
#pragma unroll
                for (int mm = 0; mm < 4; mm++) {
                    const int m = 4 * t + mm;
                    if (m >= M) break;
                    const int src = 16 * mm + (lane >> 2);
                    const float s0 = __shfl(acc[0][t], src), s1 = __shfl(acc[1][t], src);
                    const float s2 = __shfl(acc[2][t], src), s3 = __shfl(acc[3][t], src);
                    float v = u == 0 ? s0 : u == 1 ? s1 : u == 2 ? s2 : s3;
                    if (nc < N) {
                        if (task.slot < 0) v = finish(b, m, nc, v);
                        else st_ll(a.part + ((size_t)(task.slot + b * task.stride) * M + m) * kCols + lane, v, e);
                    } else {
                        v = 0.f;
                    }
                    if constexpr (FU)
                        if (fssq) emit_ssq(fssq, N, m, task.ct + b, v, e);
                }
            }
        };

        // the wave's job stream over the tile (see the pipeline note above): positions 0..kP-1 are
        // in flight; the last iteration refills from the next tile
        const int njobs = nbw * wcount;
        const int njobs_p = njobs > kP ? (njobs + kP - 1) / kP * kP : kP;
        Stream fs = open_stream(cs);
#pragma unroll
        for (int d = 0; d < kP; d++) advance(fs);
        int cb = 0, cg = 0;                // block and group of the next job consumed
        auto consume_job = [&](int d) {
            consume(wfirst + cg, wb[d], zb[d], sb[d]);
            if (++cg == wcount) {
                if (bmode)
                    store_block(wave + cb * W);
                else
                    publish(cb);
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int t = 0; t < T; t++) acc[u][t] = 0.f;
                cg = 0;
                cb++;
            }
        };
        int k = 0;
        for (; k + kP < njobs_p; k += kP) {
#pragma unroll
            for (int d = 0; d < kP; d++) {
                if (k + d < njobs) consume_job(d);
                fetch(d, fs);
                advance(fs);
            }
        }
        {
            Stream nx = open_stream(ns);
#pragma unroll
            for (int d = 0; d < kP; d++) {
                if (k + d < njobs) consume_job(d);
                fetch(d, nx);
                advance(nx);
            }
        }
        // a wave without groups in this tile still counts itself in for every block
        if (!bmode && wcount == 0)
            for (int b = 0; b < task.nblk; b++) publish(b);
        if (!ok) sh_bad = 1;
        // the next tile's prologue rewrites the digits and the staged epilogue
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
    }
}

struct SeqKernel {
    const void* fn;
    int threads;
};

// Eight waves per workgroup (one workgroup per CU) where two waves per SIMD fit the registers:
// a single workgroup keeps its waves in step through the per-block barriers, where two
// co-resident workgroups drift apart (the older one's waves win issue). Otherwise four waves.
template <int T, bool BM, bool FU>
SeqKernel kernel_for(int nb)
{
    constexpr int RG = T == 1 ? 4 : 2;      // reduction ring slots (32 KB of LDS with 8 waves)
    // deeper prefetch for M > 8 except with 256-wide groups (it would spill registers)
    constexpr int P = T == 4 ? QL_SEQ_PREFETCH_WIDE : QL_SEQ_PREFETCH;
    constexpr int W = T <= 2 ? QL_SEQ_WAVES : 4;
    switch (nb) {
    case 1: return {reinterpret_cast<const void*>(&seq_kernel<T, 1, RG, P, W, BM, FU>), 64 * W};
    case 2: return {reinterpret_cast<const void*>(&seq_kernel<T, 2, RG, P, W, BM, FU>), 64 * W};
    case 4: return {reinterpret_cast<const void*>(&seq_kernel<T, 4, RG, QL_SEQ_PREFETCH, 4, BM, FU>), 256};
    default: return {nullptr, 0};
    }
}

template <bool FU>
SeqKernel seq_kernel_for_fu(int M, int group, bool bmode)
{
    const int nb = group / 64;
    if (M <= 4) return bmode ? kernel_for<1, true, FU>(nb) : kernel_for<1, false, FU>(nb);
    if (M <= 8) return bmode ? kernel_for<2, true, FU>(nb) : kernel_for<2, false, FU>(nb);
    return bmode ? kernel_for<4, true, FU>(nb) : kernel_for<4, false, FU>(nb);
}

SeqKernel seq_kernel_for(int M, int group, bool bmode = false, bool fused = false)
{
    return fused ? seq_kernel_for_fu<true>(M, group, bmode) : seq_kernel_for_fu<false>(M, group, bmode);
}

}  // namespace

size_t seq_lds_budget(int M, int group) { return lds_budget(M, group); }

// Most groups one tile may cover: its activation digits fit the LDS budget and, in a latency-bound
// pass, its prologue stays within 4 input chunks per lane (one round of loads).
static int max_tile_groups(const SeqSpec& s, int M, bool latency)
{
    const int max_g = std::max<int>(1, (int)(lds_budget(M, s.group) / lds_per_group(M, s.group)));
    const int max_p = std::max(1, 4 * seq_kernel_for(M, s.group).threads / (M * (s.group / 64) * 8));
#ifdef QL_SEQ_MAX_TILE_GROUPS
    return std::min(QL_SEQ_MAX_TILE_GROUPS, latency ? std::min(max_g, max_p) : max_g);
#else
    return latency ? std::min(max_g, max_p) : max_g;
#endif
}

// K segments of a linear in a latency-bound pass: about `units` (block, segment) items for the
// whole linear, at least kMinGroups groups each, within the tile limit.
static int latency_split(const SeqSpec& s, int M, double units)
{
    const int ct = (s.N + kCols - 1) / kCols;
    const int groups = s.K / s.group;
    int S = (int)(units / ct + 0.5);
    S = std::min(S, std::max(1, groups / kMinGroups));
    if (groups <= QL_SEQ_WHOLE_GROUPS) S = 1;
    const int mg = max_tile_groups(s, M, true);
    S = std::max({S, 1, (groups + mg - 1) / mg});
    return std::min({S, groups, kSeqMaxSplit});
}

// Rows per block a tile writing whole outputs of this linear stages in LDS for its epilogue: one
// (the bias) or M (bias + residual of a fused add); none without either.
static int staged_rows(const SeqSpec& s, int M)
{
    return (s.fuse & kFuseRes) ? M : s.has_bias ? 1 : 0;
}

namespace {

// Groups [g0, g1) of column block c of linear `lin`.
struct Piece {
    int lin, c, g0, g1;
};

// Deals a pass's items to `runs` workgroups (run w -> workgroup (cursor + w) % grid) so that
// every run carries the same number of block-groups to within one group. With `split`, an item
// that straddles a run boundary is cut at the group nearest to it. Without, items stay whole:
// one per run when they are no more than the runs, else each goes to the run holding its
// midpoint.
void cut_runs(const std::vector<Piece>& items, int runs, bool split, std::vector<std::vector<Piece>>* out)
{
    out->assign(runs, {});
    if (!split && items.size() <= (size_t)runs) {
        for (size_t k = 0; k < items.size(); k++) (*out)[k].push_back(items[k]);
        return;
    }
    uint64_t total = 0;
    for (const Piece& it : items) total += (uint64_t)(it.g1 - it.g0);
    if (total == 0 || runs == 0) return;
    // boundary of run w: total * (w + 1) / runs, in exact integer arithmetic
    auto bound = [&](int w) { return (total * (uint64_t)(w + 1) + runs / 2) / (uint64_t)runs; };
    uint64_t acc = 0;
    int w = 0;
    for (const Piece& it : items) {
        const uint64_t len = (uint64_t)(it.g1 - it.g0);
        if (!split) {
            const uint64_t mid2 = 2 * acc + len;          // twice the item's midpoint
            while (w + 1 < runs && mid2 > 2 * bound(w)) w++;
            (*out)[w].push_back(it);
            acc += len;
            continue;
        }
        int g = it.g0;
        while (g < it.g1) {
            while (w + 1 < runs && acc >= bound(w)) w++;
            const uint64_t room = w + 1 < runs ? bound(w) - acc : UINT64_MAX;
            const int take = (int)std::min<uint64_t>(room, (uint64_t)(it.g1 - g));
            (*out)[w].push_back(Piece{it.lin, it.c, g, g + take});
            g += take;
            acc += (uint64_t)take;
        }
    }
}


// Split runs priced with a fixed cost per tile: a run costs its block-groups plus `tile_cost`
// for each tile it starts (a new linear, or a piece of a block cut along K, which is a tile of
// its own). Finds the smallest cap on a run's cost that a greedy fill of `runs` runs meets
// (binary search), so workgroups with many small linears get fewer block-groups.
void cut_runs_priced(const std::vector<Piece>& items, int runs, uint64_t tile_cost,
                     std::vector<std::vector<Piece>>* out)
{
    uint64_t total = 0;
    for (const Piece& it : items) total += (uint64_t)(it.g1 - it.g0);
    // short runs: the price stays below a quarter of the mean run, so that runs still get cut
    // inside blocks rather than leave workgroups without work
    if (runs > 0) tile_cost = std::min<uint64_t>(tile_cost, total / (uint64_t)runs / 4);
    if (total == 0 || runs == 0 || tile_cost == 0) {
        cut_runs(items, runs, true, out);
        return;
    }
    // greedy fill under `cap`; false when it needs more than `runs` runs
    auto fill = [&](uint64_t cap, std::vector<std::vector<Piece>>* res) {
        if (res) res->assign(runs, {});
        int w = 0;
        uint64_t cost = 0;
        int prev_lin = -1;
        bool prev_part = false, empty = true;
        for (const Piece& it : items) {
            int g = it.g0;
            while (g < it.g1) {
                const int rest = it.g1 - g;
                const bool part_start = g != it.g0;
                const bool new_tile = empty || prev_lin != it.lin || prev_part || part_start;
                const uint64_t nt = new_tile ? tile_cost : 0;
                if (cost + nt + (uint64_t)rest <= cap) {
                    if (res) (*res)[w].push_back(Piece{it.lin, it.c, g, it.g1});
                    cost += nt + (uint64_t)rest;
                    prev_lin = it.lin;
                    prev_part = part_start;
                    empty = false;
                    g = it.g1;
                    continue;
                }
                // the cap falls inside this piece: take what fits (as a K part, its own tile)
                const uint64_t room = cap > cost + tile_cost ? cap - cost - tile_cost : 0;
                if (room > 0) {
                    const int take = (int)std::min<uint64_t>(room, (uint64_t)rest);
                    if (res) (*res)[w].push_back(Piece{it.lin, it.c, g, g + take});
                    g += take;
                } else if (empty) {
                    return false;              // not even one group fits: cap too small
                }
                if (++w >= runs) return false;
                cost = 0;
                empty = true;
                prev_lin = -1;
                prev_part = false;
            }
        }
        return true;
    };
    uint64_t lo = (total + runs - 1) / runs, hi = total + tile_cost * (uint64_t)(items.size() + 1);
    while (lo < hi) {
        const uint64_t mid = lo + (hi - lo) / 2;
        if (fill(mid, nullptr)) hi = mid;
        else lo = mid + 1;
    }
    fill(lo, out);
}
}  // namespace

void plan_seq(const std::vector<SeqSpec>& lin, int M, int grid, SeqPlanOut* out)
{
    SeqPlanOut& p = *out;
    p = SeqPlanOut{};
    p.grid = grid;
    const int n = (int)lin.size();
    // the fuse bits every task of a linear carries: its own, and kFuseSsq when a consumer
    // normalizes its output (the same rule that gives it a sums-of-squares buffer)
    std::vector<int32_t> task_fuse(n);
    for (int i = 0; i < n; i++) task_fuse[i] = lin[i].fuse;
    for (int c = 0; c < n; c++)
        if ((lin[c].fuse & kFuseNorm) && lin[c].src >= 0) task_fuse[lin[c].src] |= kFuseSsq;
    p.pass_of.assign(n, 0);
    for (int i = 0; i < n; i++) {
        // after every producer the linear reads: its input, the GLU operand, the residual
        int pass = 0;
        for (const int src : {lin[i].src, lin[i].src2, lin[i].res_src})
            if (src >= 0) pass = std::max(pass, p.pass_of[src] + 1);
        p.pass_of[i] = pass;
        p.passes = std::max(p.passes, p.pass_of[i] + 1);
    }
    std::vector<std::vector<SeqTask>> per_wg(grid);
    int cursor = 0;
    for (int pass = 0; pass < p.passes; pass++) {
        std::vector<int> ids;
        uint64_t bytes = 0;
        for (int i = 0; i < n; i++)
            if (p.pass_of[i] == pass) {
                ids.push_back(i);
                bytes += lin[i].weight_bytes;
            }
        // A pass whose weights are small per workgroup is latency-bound: about one (block,
        // K segment) item per workgroup. A streaming pass is cut into equal runs of block-groups
        // on every workgroup; blocks are split along K only where the LDS limit forces it or a
        // run boundary falls inside them. A linear with forced segments is walked in chunks of
        // blocks, all segments of a chunk before the next, so a block's parts mostly share a run.
        const bool streaming = bytes / (uint64_t)grid >= kStreamBytes;
        // Items of a set of linears: (linear, block, K segment) in linear order; a linear with
        // forced segments is walked in chunks of blocks (about one run's worth), all segments of
        // a chunk before the next, so a block's parts mostly share a run.
        auto build_items = [&](const std::vector<int>& set, double budget, std::vector<Piece>* items) {
            for (int i : set) {
                const SeqSpec& s = lin[i];
                const int ct = (s.N + kCols - 1) / kCols;
                const int groups = s.K / s.group;
                const int mgs = max_tile_groups(s, M, false);
                const int S = streaming ? std::min((groups + mgs - 1) / mgs, groups)
                                        : latency_split(s, M, (double)grid * s.weight_bytes / std::max<uint64_t>(1, bytes));
                auto seg = [&](int k, int* g0, int* g1) {
                    *g0 = (int)((int64_t)groups * k / S);
                    *g1 = (int)((int64_t)groups * (k + 1) / S);
                };
                int g0, g1;
                if (!streaming) {
                    for (int k = 0; k < S; k++) {
                        seg(k, &g0, &g1);
                        for (int c = 0; c < ct; c++) items->push_back(Piece{i, c, g0, g1});
                    }
                } else {
                    const int chunk = S == 1 ? ct : std::max(1, (int)(budget / groups));
                    for (int c0 = 0; c0 < ct; c0 += chunk)
                        for (int k = 0; k < S; k++) {
                            seg(k, &g0, &g1);
                            for (int c = c0; c < std::min(ct, c0 + chunk); c++) items->push_back(Piece{i, c, g0, g1});
                        }
                }
            }
        };
        auto units_of = [&](int i) { return (uint64_t)((lin[i].N + kCols - 1) / kCols) * (lin[i].K / lin[i].group); };
        std::vector<std::vector<Piece>> run_pieces;
        int runs = grid;
        if (!streaming) {
            std::vector<Piece> items;
            build_items(ids, 0.0, &items);
            runs = (int)std::min<size_t>(items.size(), (size_t)grid);
            cut_runs(items, runs, false, &run_pieces);
        } else {
            // Shape classes (K, N): every workgroup gets an equal share of each class, so every
            // workgroup carries the same mix of shapes. Shapes stream at different rates when
            // they share the memory system, and equal mixes finish together. Classes below 16
            // block-groups per workgroup are cut together.
            std::vector<std::pair<std::pair<int, int>, std::vector<int>>> classes;
            std::vector<int> small;
            for (int i : ids) {
                const std::pair<int, int> key{lin[i].K, lin[i].N};
                size_t c = 0;
                while (c < classes.size() && classes[c].first != key) c++;
                if (c == classes.size()) classes.push_back({key, {}});
                classes[c].second.push_back(i);
            }
            std::vector<std::vector<int>> sets;
            for (auto& c : classes) {
                uint64_t u = 0;
                for (int i : c.second) u += units_of(i);
                if (QL_SEQ_CLASS_CUT && u >= 16 * (uint64_t)grid) sets.push_back(c.second);
                else small.insert(small.end(), c.second.begin(), c.second.end());
            }
            if (!small.empty()) {
                std::sort(small.begin(), small.end());
                sets.push_back(small);
            }
            run_pieces.assign(grid, {});
            // a tile's fixed cost in block-groups: higher where the weights stream from the MALL
            // (a block-group takes about half the time it takes from HBM)
            const uint64_t tile_cost = bytes <= kMallBytes ? QL_SEQ_TILE_COST_MALL : M == 1 ? 0 : QL_SEQ_TILE_COST;
            std::vector<std::vector<std::vector<Piece>>> per_set(sets.size());
            for (size_t c = 0; c < sets.size(); c++) {
                uint64_t u = 0;
                for (int i : sets[c]) u += units_of(i);
                std::vector<Piece> items;
                build_items(sets[c], (double)u / grid, &items);
                cut_runs_priced(items, grid, tile_cost, &per_set[c]);
            }
            // each run takes the sets in a rotated order, so the chip-wide mix stays even in time
            for (int r = 0; r < grid; r++)
                for (size_t c = 0; c < sets.size(); c++) {
                    const auto& v = per_set[(c + r) % sets.size()][r];
                    run_pieces[r].insert(run_pieces[r].end(), v.begin(), v.end());
                }
        }

        // parts of each block, in ascending K order; slots for blocks of more than one part
        std::vector<std::vector<std::vector<Piece>>> parts(n);   // [linear][block] -> pieces
        for (int i : ids) parts[i].assign((lin[i].N + kCols - 1) / kCols, {});
        for (const auto& r : run_pieces)
            for (const Piece& q : r) parts[q.lin][q.c].push_back(q);
        std::vector<std::vector<int64_t>> base(n);
        for (int i : ids) {
            base[i].assign(parts[i].size(), -1);
            for (size_t c = 0; c < parts[i].size(); c++) {
                auto& v = parts[i][c];
                std::sort(v.begin(), v.end(), [](const Piece& a, const Piece& b) { return a.g0 < b.g0; });
                p.max_split = std::max(p.max_split, (int)v.size());
                if (v.size() > 1) {
                    base[i][c] = (int64_t)p.slots;
                    p.slots += v.size();
                }
            }
        }
        auto slot_of = [&](const Piece& q) -> int64_t {
            const int64_t b = base[q.lin][q.c];
            if (b < 0) return -1;
            const auto& v = parts[q.lin][q.c];
            for (size_t r = 0; r < v.size(); r++)
                if (v[r].g0 == q.g0) return b + (int64_t)r;
            return -1;
        };

        // tiles: consecutive pieces of a run merged while they continue the same columns and
        // K range and their slots advance by a fixed stride. A split block is reduced by the run
        // that computes its last part (the latest in that run): right after that tile when all of
        // the block's parts are in this run (no wait on another workgroup), otherwise after all of
        // the run's tiles of the pass.
        struct Host { int run; uint64_t pos; bool local; };
        std::vector<std::vector<Host>> host(n);
        std::vector<std::vector<int>> owner(n);      // run of the block's parts, -2 when several
        for (int i : ids) {
            host[i].assign(parts[i].size(), Host{-1, 0, false});
            owner[i].assign(parts[i].size(), -1);
        }
        for (int r = 0; r < runs; r++)
            for (const Piece& q : run_pieces[r]) {
                int& o = owner[q.lin][q.c];
                o = (o == -1 || o == r) ? r : -2;
            }
        std::vector<std::vector<std::pair<size_t, int>>> after(runs);   // (tile end index, block)
        for (int r = 0; r < runs; r++) {
            const auto& v = run_pieces[r];
            uint64_t pos = 0;                 // block-groups of the run up to the current tile's end
            for (size_t k = 0; k < v.size();) {
                const Piece& a = v[k];
                const int64_t s0 = slot_of(a);
                int64_t stride = 0;
                size_t e = k + 1;
                while (e < v.size()) {
                    const Piece& b = v[e];
                    if (b.lin != a.lin || b.c != a.c + (int)(e - k) || b.g0 != a.g0 || b.g1 != a.g1) break;
                    const int64_t sb = slot_of(b);
                    if ((s0 < 0) != (sb < 0)) break;
                    if (s0 >= 0) {
                        const int64_t d = sb - slot_of(v[e - 1]);
                        if (e == k + 1) stride = d;
                        else if (d != stride) break;
                    }
                    e++;
                }
                pos += (uint64_t)(e - k) * (uint64_t)(a.g1 - a.g0);
                for (size_t x = k; x < e; x++) {
                    const Piece& q = v[x];
                    if (base[q.lin][q.c] < 0) continue;
                    Host& h = host[q.lin][q.c];
                    if (h.run < 0 || pos >= h.pos) h = Host{r, pos, owner[q.lin][q.c] == r};
                }
                k = e;
            }
        }
        // emit: tiles in run order with local reductions after the tile that completes them, then
        // the run's remaining reductions
        auto emit_reduces = [&](int w, int r, int i, const std::vector<int>& blocks) {
            for (size_t k = 0; k < blocks.size();) {
                const int c = blocks[k];
                const int np = (int)parts[i][c].size();
                size_t e = k + 1;
                while (e < blocks.size() && e - k < 8 && blocks[e] == blocks[e - 1] + 1 &&
                       (int)parts[i][blocks[e]].size() == np && base[i][blocks[e]] == base[i][blocks[e - 1]] + np)
                    e++;
                per_wg[w].push_back(SeqTask{i, kSeqReduce, c, (int)(e - k), 0, 0, (int32_t)base[i][c], np, np, -1, task_fuse[i], 0});
                p.reduces++;
                k = e;
            }
            (void)r;
        };
        for (int r = 0; r < runs; r++) {
            const auto& v = run_pieces[r];
            const int w = (cursor + r) % grid;
            for (size_t k = 0; k < v.size();) {
                const Piece& a = v[k];
                const int64_t s0 = slot_of(a);
                int64_t stride = 0;
                size_t e = k + 1;
                while (e < v.size()) {
                    const Piece& b = v[e];
                    if (b.lin != a.lin || b.c != a.c + (int)(e - k) || b.g0 != a.g0 || b.g1 != a.g1) break;
                    const int64_t sb = slot_of(b);
                    if ((s0 < 0) != (sb < 0)) break;
                    if (s0 < 0 && (e - k + 1) * (size_t)staged_rows(lin[a.lin], M) > (size_t)kSeqBiasBlocks) break;
                    if (s0 >= 0) {
                        const int64_t d = sb - slot_of(v[e - 1]);
                        if (e == k + 1) stride = d;
                        else if (d != stride) break;
                    }
                    e++;
                }
                per_wg[w].push_back(SeqTask{a.lin, kSeqTile, a.c, (int)(e - k), a.g0, a.g1, (int32_t)s0,
                                            (int32_t)stride, 0, -1, task_fuse[a.lin], 0});
                p.tiles++;
                p.max_gseg = std::max(p.max_gseg, a.g1 - a.g0);
                // blocks whose parts all sit in this run and end with this tile
                std::vector<int> done;
                for (size_t x = k; x < e; x++) {
                    const Piece& q = v[x];
                    const Host& h = host[q.lin][q.c];
                    if (base[q.lin][q.c] >= 0 && h.run == r && h.local && parts[q.lin][q.c].back().g0 <= q.g0 &&
                        parts[q.lin][q.c].back().g1 == q.g1)
                        done.push_back(q.c);
                }
                if (!done.empty()) emit_reduces(w, r, a.lin, done);
                k = e;
            }
            for (int i : ids) {
                std::vector<int> rest;
                for (int c = 0; c < (int)parts[i].size(); c++)
                    if (base[i][c] >= 0 && host[i][c].run == r && !host[i][c].local) rest.push_back(c);
                if (!rest.empty()) emit_reduces(w, r, i, rest);
            }
        }
        cursor = (cursor + runs) % grid;
    }
    p.task_begin.assign(grid + 1, 0);
    p.first_tile.assign(grid, -1);
    for (int w = 0; w < grid; w++) {
        uint64_t units = 0;
        for (const SeqTask& t : per_wg[w])
            if (t.kind == kSeqTile) units += (uint64_t)t.nblk * (uint64_t)(t.g1 - t.g0);
        p.total_units += units;
        p.busiest_units = std::max(p.busiest_units, units);
        p.task_begin[w] = (int32_t)p.tasks.size();
        int prev = -1;
        for (const SeqTask& t : per_wg[w]) {
            const int idx = (int)p.tasks.size();
            p.tasks.push_back(t);
            if (t.kind == kSeqTile) {
                if (prev >= 0) p.tasks[prev].next_tile = idx;
                else p.first_tile[w] = idx;
                prev = idx;
            }
        }
    }
    p.task_begin[grid] = (int32_t)p.tasks.size();
    const int group = lin.empty() ? 128 : lin[0].group;
    p.lds_bytes = (uint64_t)std::max(1, p.max_gseg) * lds_per_group(M, group);
    const int W = seq_kernel_for(M, group).threads / 64;
    for (const SeqTask& t : p.tasks)
        if (t.kind == kSeqTile && block_mode_for(t.g1 - t.g0, t.nblk, W)) p.block_mode = true;
}

std::string verify_seq_plan(const std::vector<SeqSpec>& lin, int M, const SeqPlanOut& p)
{
    char msg[256];
    const int n = (int)lin.size();
    struct Part { int g0; int64_t slot; int wg; int task; };
    std::vector<std::vector<int>> cover(n);                  // [i][c * groups + g] -> tile
    std::vector<std::vector<int>> reduced(n);
    std::vector<std::vector<std::vector<Part>>> written(n);   // [i][c] -> parts
    for (int i = 0; i < n; i++) {
        const int ct = (lin[i].N + kCols - 1) / kCols;
        cover[i].assign((size_t)ct * (lin[i].K / lin[i].group), -1);
        reduced[i].assign(ct, 0);
        written[i].assign(ct, {});
    }
    if ((int)p.task_begin.size() != p.grid + 1 || p.task_begin[p.grid] != (int)p.tasks.size())
        return "task_begin does not bound the task list";
    // pass 1: tiles (coverage, LDS, chain links), pass order within each workgroup
    for (int w = 0; w < p.grid; w++) {
        int last_pass = -1, prev_tile = -1;
        for (int t = p.task_begin[w]; t < p.task_begin[w + 1]; t++) {
            const SeqTask& k = p.tasks[t];
            if (k.linear < 0 || k.linear >= n) return "task names no linear";
            const SeqSpec& s = lin[k.linear];
            const int groups = s.K / s.group, ct = (s.N + kCols - 1) / kCols;
            const int pass = p.pass_of[k.linear];
            if (pass < last_pass) {
                snprintf(msg, sizeof msg, "workgroup %d: pass %d after pass %d", w, pass, last_pass);
                return msg;
            }
            last_pass = pass;
            if (k.nblk < 1 || k.ct < 0 || k.ct + k.nblk > ct) return "task blocks outside the linear";
            if (k.kind == kSeqReduce) continue;
            if (k.kind != kSeqTile) return "unknown task kind";
            if (prev_tile < 0 ? p.first_tile[w] != t : p.tasks[prev_tile].next_tile != t)
                return "first_tile / next_tile chain broken";
            prev_tile = t;
            if (k.g0 < 0 || k.g1 > groups || k.g0 >= k.g1) return "tile groups outside K";
            if ((uint64_t)(k.g1 - k.g0) * lds_per_group(M, s.group) > p.lds_bytes) return "tile exceeds the LDS plan";
            if (k.slot < 0 && k.nblk * staged_rows(s, M) > kSeqBiasBlocks)
                return "tile with a staged epilogue exceeds the staged blocks";
            for (int b = 0; b < k.nblk; b++) {
                for (int g = k.g0; g < k.g1; g++) {
                    int& cv = cover[k.linear][(size_t)(k.ct + b) * groups + g];
                    if (cv >= 0) {
                        snprintf(msg, sizeof msg, "linear %d block %d group %d computed twice", k.linear, k.ct + b, g);
                        return msg;
                    }
                    cv = t;
                }
                const int64_t slot = k.slot < 0 ? -1 : (int64_t)k.slot + (int64_t)b * k.stride;
                if (slot >= (int64_t)p.slots) return "tile slot outside the pool";
                written[k.linear][k.ct + b].push_back(Part{k.g0, slot, w, t});
            }
        }
        if (prev_tile >= 0 ? p.tasks[prev_tile].next_tile != -1 : p.first_tile[w] != -1)
            return "first_tile / next_tile chain broken";
    }
    // every group computed; a block of one part written whole, others in consecutive slots in K order
    for (int i = 0; i < n; i++) {
        const SeqSpec& s = lin[i];
        const int groups = s.K / s.group, ct = (s.N + kCols - 1) / kCols;
        for (size_t x = 0; x < cover[i].size(); x++)
            if (cover[i][x] < 0) {
                snprintf(msg, sizeof msg, "linear %d block %d group %d not computed", i, (int)(x / groups), (int)(x % groups));
                return msg;
            }
        for (int c = 0; c < ct; c++) {
            auto& v = written[i][c];
            std::sort(v.begin(), v.end(), [](const Part& a, const Part& b) { return a.g0 < b.g0; });
            if (v.size() == 1) {
                if (v[0].slot >= 0) return "whole block routed through a reduction";
                continue;
            }
            if ((int)v.size() > kSeqMaxSplit) return "more parts than the kernel supports";
            for (size_t r = 0; r < v.size(); r++)
                if (v[r].slot != v[0].slot + (int64_t)r) return "parts not in consecutive slots in K order";
        }
    }
    // pass 2: reductions. Each reads exactly its blocks' parts; one that precedes some of its
    // workgroup's tiles of the same pass reads only parts that workgroup already wrote (so a
    // reduction never waits on a workgroup that could be waiting on it)
    for (int w = 0; w < p.grid; w++) {
        // index of the workgroup's last tile of the pass that each task belongs to (lists are
        // ordered by pass, so one backward scan finds it)
        std::vector<int> last_tile(p.task_begin[w + 1] - p.task_begin[w], -1);
        for (int t = p.task_begin[w + 1] - 1, cur_pass = -1, last = -1; t >= p.task_begin[w]; t--) {
            const SeqTask& k = p.tasks[t];
            const int pass = p.pass_of[k.linear];
            if (pass != cur_pass) {
                cur_pass = pass;
                last = -1;
            }
            if (k.kind == kSeqTile && last < 0) last = t;
            last_tile[t - p.task_begin[w]] = last;
        }
        for (int t = p.task_begin[w]; t < p.task_begin[w + 1]; t++) {
            const SeqTask& k = p.tasks[t];
            if (k.kind != kSeqReduce) continue;
            const bool tiles_after = last_tile[t - p.task_begin[w]] > t;
            for (int b = 0; b < k.nblk; b++) {
                const int c = k.ct + b;
                if (reduced[k.linear][c]++) return "block reduced twice";
                const auto& v = written[k.linear][c];
                if (v.size() < 2 || (int)v.size() != k.parts || v[0].slot != (int64_t)k.slot + (int64_t)b * k.stride)
                    return "reduction slots differ from the parts written";
                if (tiles_after)
                    for (const Part& q : v)
                        if (q.wg != w || q.task > t) {
                            snprintf(msg, sizeof msg, "workgroup %d: reduction of linear %d block %d may wait on a later tile",
                                     w, k.linear, c);
                            return msg;
                        }
            }
        }
    }
    for (int i = 0; i < n; i++)
        for (size_t c = 0; c < written[i].size(); c++)
            if (written[i][c].size() > 1 && reduced[i][c] != 1) {
                snprintf(msg, sizeof msg, "linear %d block %zu: %zu parts, reduced %d times", i, c, written[i][c].size(),
                         reduced[i][c]);
                return msg;
            }
    return "";
}

hipError_t seq_blocks_per_cu(int M, int group, bool fused, int* blocks)
{
    // the smaller occupancy of the two instances (with and without block mode)
    int b[2] = {0, 0};
    for (int i = 0; i < 2; i++) {
        const SeqKernel k = seq_kernel_for(M, group, i == 1, fused);
        if (!k.fn) return hipErrorInvalidValue;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b[i], k.fn, k.threads, lds_budget(M, group));
        if (e != hipSuccess) return e;
    }
    *blocks = std::min(b[0], b[1]);
    return hipSuccess;
}

int seq_wg_per_cu() { return QL_SEQ_WG_PER_CU; }

hipError_t launch_seq(const SeqArgs& a, size_t lds, hipStream_t stream)
{
    const SeqKernel k = seq_kernel_for(a.M, a.group, a.block_mode != 0, a.fused != 0);
    if (!k.fn) return hipErrorInvalidValue;
    void* args[] = {const_cast<SeqArgs*>(&a)};
    return hipLaunchKernel(k.fn, dim3(a.G), dim3(k.threads), args, lds, stream);
}

}  // namespace ql
