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
#include <vector>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

// Tunables (compile-time):
//   QL_SEQ_PREFETCH      groups each wave keeps in flight (jobs per wave padded to a multiple)
//   QL_SEQ_STREAM_KB     weight KiB per workgroup from which a pass is planned for streaming
//                        (several evenly split blocks per workgroup) instead of one block each
//   QL_SEQ_MIN_GROUPS    fewest groups per K segment when a linear is split across workgroups
//   QL_SEQ_WG_PER_CU     resident workgroups per CU the grid is sized for
//   QL_SEQ_PRO_CHUNKS    8-value input chunks per lane whose loads a tile's prologue issues together
//   QL_SEQ_SENTINEL      1: a tile first polls one word per 64-value input chunk (wave 0), then
//                        loads its input; 0: every lane polls its own input words
#ifndef QL_SEQ_SENTINEL
#define QL_SEQ_SENTINEL 1
#endif
#ifndef QL_SEQ_PREFETCH
#define QL_SEQ_PREFETCH 2
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
#ifndef QL_SEQ_WG_PER_CU
#define QL_SEQ_WG_PER_CU 2
#endif
constexpr int kP = QL_SEQ_PREFETCH;
constexpr int kMinGroups = QL_SEQ_MIN_GROUPS;
constexpr size_t kLdsBudget = 49152;
constexpr int kCols = kSeqTileCols;     // 64 output columns per tile
constexpr int kSumBatch = 16;           // partial sums a reduction loads per round trip
constexpr int kWaves = 4;
// a pass with at least this many weight bytes per workgroup streams from HBM (7B-shaped linears)
// rather than waiting on latency (0.5B-shaped linears, MALL-resident)
constexpr uint64_t kStreamBytes = (uint64_t)QL_SEQ_STREAM_KB << 10;

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

// Where a wave's packed-weight loads come from for one 64-column block of a tile: this wave's
// groups [g0, glast] of the tile's segment (a wave without groups re-reads the segment start;
// its jobs are never consumed). Every field is wave-uniform; the lane's column is derived from
// blk at each fetch, so selecting one source or another stays scalar.
struct FetchSrc {
    const uint32_t* qweight;
    const uint32_t* qzeros;
    const uint16_t* scales;
    int N, g0, glast, blk;
};

template <int T, int NB, int RB>
__global__ __launch_bounds__(256) void seq_kernel(const SeqArgs a)
{
    // dynamic LDS: activation digits [block][kq][row] (16 B), then {2^-E, Sx}[group][m]
    extern __shared__ uint4 dyn_lds[];
    // the four waves' sums of one 64-column block, [buffer][wave][m][column]; with two buffers
    // consecutive blocks alternate and need one barrier each
    __shared__ float red[RB][kWaves][4 * T][kCols];
    __shared__ uint32_t sh_epoch;
    __shared__ int sh_bad;

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

    // groups of a tile's segment per wave (the waves split the segment into contiguous parts)
    auto per_wave = [](int gseg) { return (gseg + kWaves - 1) / kWaves; };
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
        const int q = per_wave(t.g1 - t.g0);
        const int g0 = t.g0 + wave * q;
        const int g1 = min(t.g1, g0 + q);
        f.g0 = g1 > g0 ? g0 : t.g0;
        f.glast = g1 > g0 ? g1 - 1 : t.g0;
        f.blk = t.ct;
        return f;
    };

    // software pipeline over the workgroup's blocks: slot d holds job (i + d) of the current
    // block; refills run past the block's end into the next block (or the next tile's first
    // block). Loads are unconditional (clamped to the wave's groups), so the compiler waits for
    // exactly the slot it consumes. Base pointers sit in scalar registers and offsets stay
    // 32-bit (every GPTQ tensor is far below 4 GiB).
    uint4 wb[kP][2 * NB];
    uint32_t zb[kP];
    uint2 sb[kP];
    auto fetch = [&](int d, const FetchSrc& f, int job) {
        // the bases are uniform; saying so here keeps them in scalar registers however the
        // source was selected (a base in vector registers costs 64-bit address math per load and
        // makes the compiler drain the loads in flight)
        const uint32_t* qw = uniform_ptr(f.qweight);
        const uint32_t* qz = uniform_ptr(f.qzeros);   // never null
        const uint16_t* sc = uniform_ptr(f.scales);
        const int Ns = __builtin_amdgcn_readfirstlane(f.N);
        const uint32_t N = (uint32_t)Ns;
        const int g = __builtin_amdgcn_readfirstlane(min(f.g0 + job, f.glast));
        const int nc = __builtin_amdgcn_readfirstlane(f.blk) * kCols + 4 * j;
        const uint32_t n = (uint32_t)(nc < Ns ? nc : Ns - 4);
        // byte offsets in 32 bits: scalar base + 32-bit vector offset is one load instruction
        const uint32_t row0 = ((uint32_t)(g * NB * 8 + 2 * kq) * N + n) * 4u;
#pragma unroll
        for (int r = 0; r < 2 * NB; r++)
            wb[d][r] = __builtin_bit_cast(uint4, ld_global(reinterpret_cast<const u32x4*>(
                reinterpret_cast<const char*>(qw) + (row0 + (uint32_t)((r >> 1) * 8 + (r & 1)) * N * 4u))));
        zb[d] = ld_global(reinterpret_cast<const uint32_t*>(
            reinterpret_cast<const char*>(qz) + ((uint32_t)g * ((N + 7) >> 3) + (n >> 3)) * 4u));
        sb[d] = __builtin_bit_cast(uint2, ld_global(reinterpret_cast<const u32x2*>(
            reinterpret_cast<const char*>(sc) + ((uint32_t)g * N + n) * 2u)));
    };

    FetchSrc cur{};
    if (first >= 0) {
        cur = src_of(first);
#pragma unroll
        for (int d = 0; d < kP; d++) fetch(d, cur, d);
    }

    if (threadIdx.x == 0) {
        const int sub = wg % kSeqTickets;
        const uint32_t members = (uint32_t)((a.G - 1 - sub) / kSeqTickets + 1);
        const unsigned long long old = __hip_atomic_fetch_add(QL_GLOBAL(unsigned long long, a.tickets + sub * 8), 1ull, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
        sh_epoch = (uint32_t)(old / members) + 1u;
        sh_bad = 0;
    }
    __syncthreads();
    const uint32_t e = __builtin_amdgcn_readfirstlane(sh_epoch);   // uniform: scalar control flow
    int rbuf = 0;                                                 // reduction buffer in use

    for (int ti = tb; ti < te; ti++) {
        const SeqTask task = ld_const(a.tasks + ti);
        const SeqLinear L = ld_const(a.lin + task.linear);
        const int N = L.N;
        bool ok = true;

        if (task.kind == kSeqReduce) {
            // split-K partial sums of one 64-column block, added in ascending segment order
            const size_t stride = (size_t)M * N;
            if (wave == 0)
                ok = wait_words(L.part_ll + (size_t)task.ct * kCols, stride, L.S, lane, e, a);
            if (!ok) sh_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
            for (int idx = threadIdx.x; idx < M * kCols; idx += 256) {
                const int m = idx / kCols;
                const int nn = task.ct * kCols + (idx - m * kCols);
                if (nn >= N || !ok) continue;
                float sum = 0.f;
                for (int s0 = 0; s0 < L.S && ok; s0 += kSumBatch)
                    ok = sum_ll<kSumBatch>(L.part_ll + (size_t)(s0 * M + m) * N + nn, stride,
                                           min(kSumBatch, L.S - s0), e, a, &sum);
                if (!ok) continue;
                if (L.bias) sum += ld_global(L.bias + nn);
                st_global(L.y + (size_t)m * N + nn, sum);
                st_ll(L.y_ll + (size_t)m * N + nn, sum, e);
            }
            if (!ok) sh_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
            continue;
        }

        // ---- GEMV tile: blocks ct .. ct + nblk - 1 (64 columns each) over the segment [g0, g1) ----
        const int gseg = task.g1 - task.g0;
        const int q = per_wave(gseg);
        const int jpw = (q + kP - 1) / kP * kP;
        const int wcount = max(0, min(q, gseg - wave * q));   // this wave's groups
        const bool P = L.src >= 0;
        const uint64_t* p_ll = P ? ld_const(&a.lin[L.src].y_ll) : nullptr;
        // the next tile's source, read now so that its table loads overlap the prologue
        const FetchSrc next_tile = task.next_tile >= 0 ? src_of(task.next_tile) : cur;

        // the segment's activation digits (shared by all blocks of the tile), from the external
        // input or from the producer's output words: wave 0 first waits for one word of each
        // 64-value chunk of the segment (one producer block's columns)
        if (P && QL_SEQ_SENTINEL) {
            if (wave == 0) {
                const int c0 = task.g0 * GK / kCols;
                const int c1 = task.g1 * GK / kCols;
                ok = wait_words(p_ll + (size_t)c0 * kCols, kCols, c1 - c0, lane, e, a);
            }
            if (!ok) sh_bad = 1;
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(sh_bad)) return;
        }
        uint4* xd = dyn_lds;
        float2* gst = reinterpret_cast<float2*>(dyn_lds + gseg * NB * 4 * R);
        {
            // QL_SEQ_PRO_CHUNKS chunks per trip: their input loads are all issued before any is used
            const int items = gseg * M;
            constexpr int H = QL_SEQ_PRO_CHUNKS;
            for (int base = 0; base < items * CPG; base += 256 * H) {
                uint64_t w[H][8];
                float v[H][8];
                size_t xo[H];
                bool live[H];
#pragma unroll
                for (int h = 0; h < H; h++) {
                    const int idx = base + 256 * h + threadIdx.x;
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
#pragma unroll
                for (int h = 0; h < H; h++) {
                    const int idx = base + 256 * h + threadIdx.x;
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

        for (int b = 0; b < task.nblk; b++) {
            const int blk = task.ct + b;
            FetchSrc nxt = next_tile;
            if (b + 1 < task.nblk) {
                nxt = cur;
                nxt.blk = blk + 1;
            }
            const int n = blk * kCols + 4 * j;
            const bool col_ok = n < N;
            // this thread's bias values for the block's output stores, loaded ahead of the
            // weight prefetch so the stores do not wait for the prefetch to land
            float bias_v[T];
#pragma unroll
            for (int k = 0; k < T; k++) {
                const int idx = threadIdx.x + 256 * k;
                const int nn = blk * kCols + (idx - idx / kCols * kCols);
                bias_v[k] = (L.S == 1 && L.bias) ? ld_global(L.bias + (nn < N ? nn : 0)) : 0.f;
            }
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
                const uint32_t zw = zn >> (4 * (n & 7));
                const uint32_t sw[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
                float2 st[T];
#pragma unroll
                for (int t = 0; t < T; t++) {
                    const int m = 4 * t + kq;
                    st[t] = m < M ? gst[gg * M + m] : float2{0.f, 0.f};
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
                    const float sz = s * (float)(((zw >> (4 * u)) & 15u) + 1u);
#pragma unroll
                    for (int t = 0; t < T; t++) {
                        float v = fmaf((float)c[u][t][0], 0x1p-8f, (float)c[u][t][1]);
                        v = fmaf(v, 0x1p-8f, (float)c[u][t][2]);
                        v = fmaf(v, 0x1p-8f, (float)c[u][t][3]);
                        acc[u][t] = fmaf(s * st[t].x, v, acc[u][t]);
                        acc[u][t] = fmaf(-sz, st[t].y, acc[u][t]);
                    }
                }
            };

            // slot d is consumed before it is refilled: the refill then lands in the same
            // registers, so the compiler waits only for the slot it is about to use (no register
            // rotation at the back-edge, which would drain every load in flight). Every iteration
            // but the last refills from this block; the last one starts the next block.
            auto step = [&](int i, const FetchSrc& f, int job0) {
#pragma unroll
                for (int d = 0; d < kP; d++) {
                    const uint2 sv = col_ok ? sb[d] : uint2{0u, 0u};
                    if (i + d < wcount) consume(wave * q + i + d, wb[d], zb[d], sv);
                    fetch(d, f, job0 + d);
                }
            };
            int i = 0;
            for (; i + kP < jpw; i += kP) step(i, cur, i + kP);
            step(i, nxt, 0);
            cur = nxt;

            // the four waves' sums of each (row, column), added in wave order
            if (RB == 1) __syncthreads();          // the previous block's readers are done
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int u = 0; u < 4; u++) red[rbuf][wave][4 * t + kq][4 * j + u] = acc[u][t];
            __syncthreads();
#pragma unroll
            for (int k = 0; k < T; k++) {
                const int idx = threadIdx.x + 256 * k;
                const int m = idx / kCols;                  // < 4T: inside `red`
                const int col = idx - m * kCols;
                const int nn = blk * kCols + col;
                if (m < M && nn < N) {
                    float v = ((red[rbuf][0][m][col] + red[rbuf][1][m][col]) + red[rbuf][2][m][col]) +
                              red[rbuf][3][m][col];
                    if (L.S == 1) {
                        v += bias_v[k];
                        st_global(L.y + (size_t)m * N + nn, v);
                        st_ll(L.y_ll + (size_t)m * N + nn, v, e);
                    } else {
                        st_ll(L.part_ll + ((size_t)task.seg * M + m) * N + nn, v, e);
                    }
                }
            }
            rbuf = (rbuf + 1) % RB;
        }
        // the next tile's prologue rewrites the digits
        __syncthreads();
    }
}

template <int T>
const void* kernel_for(int nb)
{
    constexpr int RB = T == 4 ? 1 : 2;      // M > 8: one reduction buffer keeps LDS for 2 WGs/CU
    switch (nb) {
    case 1: return reinterpret_cast<const void*>(&seq_kernel<T, 1, RB>);
    case 2: return reinterpret_cast<const void*>(&seq_kernel<T, 2, RB>);
    case 4: return reinterpret_cast<const void*>(&seq_kernel<T, 4, RB>);
    default: return nullptr;
    }
}

const void* seq_kernel_for(int M, int group)
{
    const int nb = group / 64;
    if (M <= 4) return kernel_for<1>(nb);
    if (M <= 8) return kernel_for<2>(nb);
    return kernel_for<4>(nb);
}

}  // namespace

size_t seq_lds_budget() { return kLdsBudget; }

// K segments of one linear for a pass whose share is `units` 64-column blocks
static int split_for(const SeqSpec& s, int M, double units)
{
    const int ct = (s.N + kCols - 1) / kCols;
    const int groups = s.K / s.group;
    int S = (int)(units / ct + 0.5);
    S = std::min(S, std::max(1, groups / kMinGroups));
    // the segment's digits fit the LDS budget, and the prologue stays within 4 chunks per lane
    const int max_g = std::max<int>(1, (int)(kLdsBudget / lds_per_group(M, s.group)));
    const int max_p = std::max(1, 4 * 256 / (M * (s.group / 64) * 8));
    S = std::max({S, 1, (groups + max_g - 1) / max_g, (groups + max_p - 1) / max_p});
    return std::min({S, groups, kSeqMaxSplit});
}

void plan_seq(const std::vector<SeqSpec>& lin, int M, int grid, SeqPlanOut* out)
{
    SeqPlanOut& p = *out;
    p = SeqPlanOut{};
    p.grid = grid;
    const int n = (int)lin.size();
    p.pass_of.assign(n, 0);
    p.split.assign(n, 1);
    for (int i = 0; i < n; i++) {
        p.pass_of[i] = lin[i].src >= 0 ? p.pass_of[lin[i].src] + 1 : 0;
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
        // Splits: a pass whose weights are small per workgroup is latency-bound and gets about one
        // block per workgroup; a streaming pass gets the smallest multiple k of the grid whose
        // blocks divide evenly enough (the busiest workgroup carries at most ~15% above average).
        const bool streaming = bytes / (uint64_t)grid >= kStreamBytes;
        std::vector<int> best;
        double best_bal = -1.0;
        for (int k = 1; k <= (streaming ? 8 : 1); k++) {
            std::vector<int> S(ids.size());
            uint64_t U = 0;
            for (size_t x = 0; x < ids.size(); x++) {
                const SeqSpec& s = lin[ids[x]];
                S[x] = split_for(s, M, (double)k * grid * s.weight_bytes / std::max<uint64_t>(1, bytes));
                U += (uint64_t)((s.N + kCols - 1) / kCols) * S[x];
            }
            const double per = (double)U / grid;
            const double bal = per >= 1.0 ? per / std::ceil(per) : 1.0;
            if (bal > best_bal + 1e-9) {
                best_bal = bal;
                best = S;
            }
            if (bal >= 0.85) break;
        }
        // rows of blocks: (linear, segment) in order; cut into `grid` nearly equal runs
        struct Row { int lin, seg, g0, g1, blocks; };
        std::vector<Row> rows;
        uint64_t U = 0;
        for (size_t x = 0; x < ids.size(); x++) {
            const int i = ids[x];
            const SeqSpec& s = lin[i];
            const int S = best[x];
            const int groups = s.K / s.group;
            const int ct = (s.N + kCols - 1) / kCols;
            p.split[i] = S;
            p.max_split = std::max(p.max_split, S);
            for (int seg = 0; seg < S; seg++) {
                const int g0 = (int)((int64_t)groups * seg / S);
                const int g1 = (int)((int64_t)groups * (seg + 1) / S);
                p.max_gseg = std::max(p.max_gseg, g1 - g0);
                rows.push_back(Row{i, seg, g0, g1, ct});
                U += ct;
            }
        }
        const int runs = (int)std::min<uint64_t>(U, (uint64_t)grid);
        size_t r = 0;
        uint64_t row_start = 0;
        for (int w = 0; w < runs; w++) {
            uint64_t lo = U * w / runs, hi = U * (w + 1) / runs;
            const int dst = (cursor + w) % grid;
            while (lo < hi) {
                while (row_start + rows[r].blocks <= lo) row_start += rows[r++].blocks;
                const Row& row = rows[r];
                const uint64_t end = std::min<uint64_t>(hi, row_start + row.blocks);
                per_wg[dst].push_back(SeqTask{row.lin, kSeqTile, (int)(lo - row_start), row.seg,
                                              row.g0, row.g1, -1, (int)(end - lo)});
                p.tiles++;
                lo = end;
            }
        }
        cursor = (cursor + runs) % grid;
        // reductions of split linears: one per 64-column block, after the pass's tiles
        for (int i : ids) {
            if (p.split[i] == 1) continue;
            const int ct = (lin[i].N + kCols - 1) / kCols;
            for (int c = 0; c < ct; c++) {
                per_wg[cursor].push_back(SeqTask{i, kSeqReduce, c, 0, 0, 0, -1, 1});
                cursor = (cursor + 1) % grid;
                p.reduces++;
            }
        }
    }
    p.task_begin.assign(grid + 1, 0);
    p.first_tile.assign(grid, -1);
    for (int w = 0; w < grid; w++) {
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
}

hipError_t seq_blocks_per_cu(int M, int group, int* blocks)
{
    const void* k = seq_kernel_for(M, group);
    if (!k) return hipErrorInvalidValue;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, k, 256, kLdsBudget);
}

int seq_wg_per_cu() { return QL_SEQ_WG_PER_CU; }

hipError_t launch_seq(const SeqArgs& a, size_t lds, hipStream_t stream)
{
    const void* k = seq_kernel_for(a.M, a.group);
    if (!k) return hipErrorInvalidValue;
    void* args[] = {const_cast<SeqArgs*>(&a)};
    return hipLaunchKernel(k, dim3(a.G), dim3(256), args, lds, stream);
}

}  // namespace ql
