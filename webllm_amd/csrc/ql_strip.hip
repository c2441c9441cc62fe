// Column strips: independent decode linears (M = 2..16 rows, each on its own input) in ONE
// persistent launch, without K splits.
//
// A sequence whose linears do not feed each other (the reference's q/k/v or gate/up batches,
// src/model/qwen.ts:411-413, :464-465, or a whole step of independent linears) is one pass. For
// M > 1 the activation digits of a quantization group take 2*M KiB of LDS, so a tile of the
// dependency-ordered sequence kernel covers only a few groups and splits long K into parts whose
// partial sums cost HBM traffic. Here a workgroup instead owns a strip of whole 64-column blocks
// over ALL of K:
// * each consumer wave owns BPW blocks of the strip and keeps their sums in registers;
// * K is walked in chunks of kCG groups; one producer wave turns the next chunk's activations
//   into base-256 digits (ql_digits.h) in a double-buffered LDS area while the consumers run the
//   current chunk, and one barrier per chunk hands the buffers over;
// * each consumer streams its jobs (one quantization group x its BPW blocks) through a register
//   ring P jobs deep that runs across chunks, barriers and strips; the producer's loads use its
//   own wave's counters, so waiting for them never drains the consumers' weight loads;
// * strips are dealt to workgroups on the host (longest first onto the least loaded), so every
//   workgroup streams about the same number of weight bytes.
// Arithmetic is the decode kernels' exact int8-digit MFMA product and fp32 group epilogue, so
// outputs equal the sequence kernel's bit for bit.
#include <algorithm>
#include <cstdlib>
#include <functional>
#include <queue>
#include <vector>

#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

namespace ql {

namespace {

constexpr int kCG = kStripChunkGroups;   // quantization groups per chunk
constexpr int kCols = kSeqTileCols;      // 64 output columns per block

template <typename T>
__device__ __forceinline__ T ld_table(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    // tables are written once before any launch: constant address space, scalar loads
    return *(const __attribute__((address_space(4))) T*)(reinterpret_cast<uintptr_t>(p));
#else
    return *p;
#endif
}

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <typename T>
__device__ __forceinline__ const T* uni_ptr(const T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const T*>((hi << 32) | lo);
}

// LDS bytes of one chunk buffer: digits [group][k block][k quarter][digit row] (16 B each), then
// {2^-E, sum x} per (group, row)
__host__ __device__ constexpr size_t strip_buf_bytes(int M, int NB)
{
    return (size_t)kCG * NB * 4 * (4 * M) * 16 + (size_t)kCG * M * 8;
}

constexpr int kMaxStripBlocks = 8;       // most blocks in one strip

// T: 16-row MFMA tiles of digit rows (4 per activation row); NB: 64-k blocks per group;
// W: waves; BPW: blocks per wave; P: jobs in flight per wave.
//
// Every chunk runs the same fixed sequence, so the number of loads between any two points is
// known when the kernel is compiled and every wait names exactly the loads it needs:
//   1. issue the next chunk's activation loads (this wave's share) and a bias load;
//   2. kCG job positions (a job: one group x the wave's blocks; positions past the chunk's groups,
//      or of a wave without blocks, are padding whose loads are never consumed), each consuming
//      its ring slot and refilling it P positions ahead;
//   3. after the strip's last chunk, store the strip's outputs;
//   4. wait for step 1's loads (the kCG positions' loads stay in flight), turn them into digits
//      in the other LDS buffer, stage the next strip's bias with its first chunk;
//   5. one barrier.
// Waves per SIMD that the M 5..8 instance reading MALL-resident weights is compiled for (at most
// 128 VGPRs): 4 lets a CU hold both of its workgroups (the 0.5B step at M=8: 48.7 against
// 53.6 us). The streaming instance keeps the compiler's choice (143 VGPRs): capped at 128 it
// spills and the 7B step at M=8 takes 773 against 664 us (711 with two workgroups per CU).
#ifndef QL_STRIP_OCC2
#define QL_STRIP_OCC2 4
#endif
template <int T, int NB, int W, int BPW, int P, int S, bool NT>
__global__ __launch_bounds__(64 * W, (T == 2 && !NT) ? QL_STRIP_OCC2 : 1) void strip_kernel(const StripArgs a)
{
    // S waves share each block (S > 1: waves take alternate groups of every chunk and add their
    // sums in LDS at the strip's end, in part order); QP positions per chunk for each wave
    static_assert(S == 1 || BPW == 1, "split blocks hold one block per wave");
    constexpr int QP = kCG / S;
    static_assert(QP * S == kCG && QP % P == 0, "a chunk's positions fill whole ring rounds");
    constexpr int WB = W / S;                // waves per part = blocks per strip / BPW
    // The M 5..8 instance on MALL-resident weights is compiled for four waves per SIMD (at most
    // 128 VGPRs). It computes one column quarter's sums at a time and keeps one lane offset for
    // its weight loads, which frees the registers it would otherwise spill (the 0.5B step at M=8:
    // 42.3 against 48.3 us). The other instances keep all quarters' sums and per-row offsets,
    // which measured 1-2 % faster for them (the 7B step at M = 1, 8, 16).
    constexpr bool kLean = T == 2 && !NT;
    extern __shared__ uint4 dyn_lds[];
    constexpr int GK = NB * 64;              // k per group
    constexpr int CPG = NB * 8;              // lanes per (group, row) when staging
    constexpr int kThreads = 64 * W;
    // most 8-activation items one thread stages per chunk (M <= 4T)
    constexpr int H = (kCG * 4 * T * CPG + kThreads - 1) / kThreads;
    const int M = a.M;
    const int R = 4 * M;
    const int lane = threadIdx.x & 63;
    const int wave = uni(threadIdx.x >> 6);
    const int bw = wave % WB;                // the wave's block slot in the strip
    const int sp = wave / WB;                // the wave's part: groups sp, sp + S, ... of a chunk
    const int j = lane & 15;
    const int kq = lane >> 4;
    const int wg = blockIdx.x;
    const int tb = ld_table(a.task_begin + wg);
    const int te = ld_table(a.task_begin + wg + 1);
    if (tb >= te) return;
    const size_t buf_bytes = strip_buf_bytes(M, NB);
    auto digits = [&](int buf) { return reinterpret_cast<uint4*>(reinterpret_cast<char*>(dyn_lds) + buf * buf_bytes); };
    auto gstat = [&](int buf) {
        return reinterpret_cast<float2*>(reinterpret_cast<char*>(dyn_lds) + buf * buf_bytes + (size_t)kCG * NB * 4 * R * 16);
    };
    // the bias of a strip's columns, staged with the strip's first chunk; two buffers by strip
    // parity (a strip's outputs are stored before the barrier that ends it)
    auto bias_lds = [&](int par) {
        return reinterpret_cast<float*>(reinterpret_cast<char*>(dyn_lds) + 2 * buf_bytes) + par * (kMaxStripBlocks * kCols);
    };
    // sums of parts 1 .. S-1 at a strip's end: [part - 1][block][row][column]
    auto part_lds = [&]() { return bias_lds(2); };

    // ---- staging cursor: the chunk being staged (task si, chunk sch) ----
    struct Stage {
        int si, sch, ngroups;
        const void* x;
        const float* bias;       // the task's bias, or any valid float pointer when it has none
        int K, xdt, ct, nblk, has_bias;
    };
    auto stage_open = [&](Stage& st, int ti) {
        const StripTask t = ld_table(a.tasks + ti);
        const SeqLinear* L = a.lin + t.linear;
        st.si = ti;
        st.sch = 0;
        st.x = uni_ptr(ld_table(&L->x));
        const float* b = ld_table(&L->bias);
        st.has_bias = b != nullptr;
        st.bias = uni_ptr(b ? b : static_cast<const float*>(st.x));
        st.K = ld_table(&L->K);
        st.xdt = ld_table(&L->x_dtype);
        st.ngroups = st.K / GK;
        st.ct = t.ct;
        st.nblk = t.nblk;
    };
    u32x4 xr[H][2];                          // raw activation bits: f32 (both) or f16 ([0])
    constexpr int BV = kMaxStripBlocks * kCols / kThreads;   // bias values staged per thread
    static_assert(BV * kThreads == kMaxStripBlocks * kCols, "threads divide a strip's columns");
    float bv[BV];
    // step 1: unconditional loads (threads past the chunk's items re-read its last item); the
    // raw bits are converted only in step 4, so nothing waits for them here
    auto stage_issue = [&](const Stage& st) {
        const int g0 = st.sch * kCG;
        const int cgc = min(kCG, st.ngroups - g0);
        const int items = cgc * M * CPG;
#pragma unroll
        for (int h = 0; h < H; h++) {
            const int idx = min((int)threadIdx.x + kThreads * h, items - 1);
            const int item = idx / CPG, c = idx - item * CPG;
            const int gg = item / M, m = item - gg * M;
            const size_t e = (size_t)m * st.K + (size_t)(g0 + gg) * GK + (size_t)c * 8;
            if (st.xdt == 0) {
                const u32x4* q = reinterpret_cast<const u32x4*>(static_cast<const float*>(st.x) + e);
                xr[h][0] = ld_global(q);
                xr[h][1] = ld_global(q + 1);
            } else {
                // the same number of loads on both paths keeps the step-4 wait exact
                const u32x4* q = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(st.x) + e);
                uint64_t q2 = reinterpret_cast<uint64_t>(q);
                asm volatile("" : "+v"(q2));        // a second load, not merged with the first
                xr[h][0] = ld_global(q);
                xr[h][1] = ld_global(reinterpret_cast<const u32x4*>(q2));
            }
        }
#pragma unroll
        for (int v = 0; v < BV; v++) {
            const int bi = min((int)threadIdx.x + kThreads * v, st.nblk * kCols - 1);
            bv[v] = ld_global(st.has_bias ? st.bias + st.ct * kCols + bi : st.bias);
        }
    };
    // step 4: digits of the staged chunk into buffer `buf`
    auto stage_finish = [&](const Stage& st, int buf) {
        const int g0 = st.sch * kCG;
        const int cgc = min(kCG, st.ngroups - g0);
        const int items = cgc * M * CPG;
        uint4* xd = digits(buf);
        float2* gst = gstat(buf);
#pragma unroll
        for (int h = 0; h < H; h++) {
            const int idx = (int)threadIdx.x + kThreads * h;
            if (idx < items) {                    // whole CPG-lane groups: CPG divides 64
                const int item = idx / CPG, c = idx - item * CPG;
                const int gg = item / M, m = item - gg * M;
                const int blk = gg * NB + (c >> 3);
                float v[8];
                if (st.xdt == 0) {
                    const f32x4 lo = __builtin_bit_cast(f32x4, xr[h][0]), hi = __builtin_bit_cast(f32x4, xr[h][1]);
                    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
                    v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
                } else {
                    const f16x8 hv = __builtin_bit_cast(f16x8, xr[h][0]);
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = (float)hv[e];
                }
                uint2* rows = reinterpret_cast<uint2*>(&xd[(blk * 4 + ((c & 7) >> 1)) * R + 4 * m]) + (c & 1);
                const float2 s2 = prep_chunk<CPG>(v, rows, 2);
                if (c == 0) gst[gg * M + m] = s2;
            }
        }
        if (st.sch == 0) {
#pragma unroll
            for (int v = 0; v < BV; v++) {
                const int bi = (int)threadIdx.x + kThreads * v;
                if (bi < st.nblk * kCols) bias_lds((st.si - tb) & 1)[bi] = st.has_bias ? bv[v] : 0.f;
            }
        }
    };
    auto stage_next = [&](Stage& st) {    // false past the last chunk of the last task
        if ((st.sch + 1) * kCG < st.ngroups) {
            st.sch++;
            return true;
        }
        if (st.si + 1 >= te) return false;
        stage_open(st, st.si + 1);
        return true;
    };

    // ---- job stream: kCG positions per chunk of every task ----
    uint4 wb[P][BPW][2 * NB];
    uint32_t zb[P][BPW];
    uint2 sb[P][BPW];
    struct Cur {
        int ti, ch, nch, pos, g, nbw, ngroups;
        const char* qw;
        const char* qz;
        const char* sc;
        uint32_t Gq, Gz, Gs;        // bytes from one group to the next
        uint32_t cq, cz, cs;        // byte offsets of the wave's first block
        uint32_t Rq;                // bytes of one packed row (N words)
        // the lane's byte offsets: of each packed row it loads, or (kLean) of the first only
        uint32_t lq[kLean ? 1 : 2 * NB], lz, ls;
    };
    auto blocks_of = [&](const StripTask& t) { return max(0, min(BPW, t.nblk - bw * BPW)); };
    auto open = [&](Cur& c, int ti) {
        // every task has kCG positions per chunk for every wave; a wave without blocks in it
        // fetches the task's last block as padding
        if (ti >= te) return false;
        const StripTask t = ld_table(a.tasks + ti);
        const SeqLinear* L = a.lin + t.linear;
        c.ti = ti;
        c.nbw = uni(blocks_of(t));
        c.qw = reinterpret_cast<const char*>(uni_ptr(ld_table(&L->qweight)));
        c.qz = reinterpret_cast<const char*>(uni_ptr(ld_table(&L->qzeros)));
        c.sc = reinterpret_cast<const char*>(uni_ptr(ld_table(&L->scales)));
        const int N = uni(ld_table(&L->N));
        const int K = uni(ld_table(&L->K));
        c.ngroups = K / GK;
        c.nch = (c.ngroups + kCG - 1) / kCG;
        c.ch = 0;
        c.pos = 0;
        c.g = min(sp, c.ngroups - 1);
        c.Gq = (uint32_t)(NB * 8) * (uint32_t)N * 4u;
        c.Gs = (uint32_t)N * 2u;
        c.Gz = (((uint32_t)N + 7u) >> 3) * 4u;
        const uint32_t blk0 = (uint32_t)(t.ct + min(bw * BPW, t.nblk - 1));
        c.cq = blk0 * (uint32_t)kCols * 4u;
        c.cs = blk0 * (uint32_t)kCols * 2u;
        c.cz = blk0 * (uint32_t)(kCols / 8) * 4u;
        c.Rq = (uint32_t)N * 4u;
#pragma unroll
        for (int r = 0; r < (kLean ? 1 : 2 * NB); r++)
            c.lq[r] = ((uint32_t)(2 * kq + (r >> 1) * 8 + (r & 1)) * (uint32_t)N + 4u * (uint32_t)j) * 4u;
        c.ls = 8u * (uint32_t)j;
        c.lz = (uint32_t)(j >> 1) * 4u;
        return true;
    };
    // positions: QP per chunk, position p on group p * S + sp of the chunk; a position past the
    // linear's groups re-reads a valid one
    auto advance = [&](Cur& c) {
        if (c.pos + 1 < QP) {
            c.pos++;
            c.g = min(c.ch * kCG + c.pos * S + sp, c.ngroups - 1);
        } else if (c.ch + 1 < c.nch) {
            c.ch++;
            c.pos = 0;
            c.g = min(c.ch * kCG + sp, c.ngroups - 1);
        } else {
            Cur n = c;
            if (open(n, c.ti + 1)) c = n;   // else the stream has ended: stay on the last job
        }
    };
    auto fetch = [&](int d, const Cur& c) {
        const uint32_t g = (uint32_t)c.g;
#pragma unroll
        for (int b = 0; b < BPW; b++) {
            const uint32_t bb = (uint32_t)min(b, max(c.nbw, 1) - 1);   // extra blocks re-read the first
            const char* q = c.qw + g * c.Gq + c.cq + bb * (uint32_t)kCols * 4u;
#pragma unroll
            for (int r = 0; r < 2 * NB; r++) {
                // packed row 2 kq + 8 (r / 2) + r % 2 of the group (kLean: a uniform row offset on
                // top of the lane's one)
                const char* qr = kLean ? q + (uint32_t)((r >> 1) * 8 + (r & 1)) * c.Rq + c.lq[0] : q + c.lq[kLean ? 0 : r];
                wb[d][b][r] = __builtin_bit_cast(uint4, NT ? ld_stream(reinterpret_cast<const u32x4*>(qr))
                                                           : ld_global(reinterpret_cast<const u32x4*>(qr)));
            }
            zb[d][b] = ld_global(reinterpret_cast<const uint32_t*>(c.qz + g * c.Gz + c.cz + bb * (uint32_t)(kCols / 8) * 4u + c.lz));
            sb[d][b] = __builtin_bit_cast(uint2, ld_global(reinterpret_cast<const u32x2*>(c.sc + g * c.Gs + c.cs + bb * (uint32_t)kCols * 2u + c.ls)));
        }
    };
    // A padding slot is never consumed; without a use its registers would be free to reuse on
    // that path, and reusing a load's destination waits for every load in flight.
    auto touch_block = [&](int d, int b) {
#pragma unroll
        for (int r = 0; r < 2 * NB; r++) asm volatile("" ::"v"(wb[d][b][r].x), "v"(wb[d][b][r].y), "v"(wb[d][b][r].z), "v"(wb[d][b][r].w));
        asm volatile("" ::"v"(zb[d][b]), "v"(sb[d][b].x), "v"(sb[d][b].y));
    };
    auto touch = [&](int d) {
#pragma unroll
        for (int b = 0; b < BPW; b++) touch_block(d, b);
    };

    float acc[BPW][4][T];
    auto clear = [&]() {
#pragma unroll
        for (int b = 0; b < BPW; b++)
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int t = 0; t < T; t++) acc[b][u][t] = 0.f;
    };

    // one job: local group gg of the chunk in buffer `buf`, the wave's nbw (>= 1) blocks
    auto consume = [&](int d, int buf, int gg, int nbw) {
        const uint4* xd = digits(buf);
        const float2* gst = gstat(buf);
        // Digit rows past the last (R and up) and group statistics of rows past M read the last
        // valid ones instead of zeros: they only feed output rows m >= M, which are never stored,
        // and the loads need no lane masking.
        i32x4 av[NB][T];
#pragma unroll
        for (int bb = 0; bb < NB; bb++)
#pragma unroll
            for (int t = 0; t < T; t++)
                av[bb][t] = __builtin_bit_cast(i32x4, xd[((gg * NB + bb) * 4 + kq) * R + min(16 * t + j, R - 1)]);
        float2 st[T];
#pragma unroll
        for (int t = 0; t < T; t++) {
            st[t] = gst[gg * M + min(4 * t + kq, M - 1)];
            st[t].x *= 0x1p-8f;       // the digit pairs below carry a factor 2^8
        }
#pragma unroll
        for (int b = 0; b < BPW; b++) {
            if (b > 0 && b >= nbw) {
                touch_block(d, b);
                continue;
            }
            const uint32_t zw = zb[d][b] >> (4 * ((4 * j) & 7));
            const uint2 sv = sb[d][b];
            const uint32_t sw[4] = {sv.x & 0xffffu, sv.x >> 16, sv.y & 0xffffu, sv.y >> 16};
            // the weight nibbles of 64-k block bb, column quarter u, as bytes
            auto bq_of = [&](int bb, int u) {
                const uint4 w0 = wb[d][b][2 * bb], w1 = wb[d][b][2 * bb + 1];
                const uint32_t lo[4] = {w0.x, w0.y, w0.z, w0.w};
                const uint32_t hi[4] = {w1.x, w1.y, w1.z, w1.w};
                return i32x4{(int)(lo[u] & 0x0F0F0F0Fu), (int)((lo[u] >> 4) & 0x0F0F0F0Fu),
                             (int)(hi[u] & 0x0F0F0F0Fu), (int)((hi[u] >> 4) & 0x0F0F0F0Fu)};
            };
            // the group epilogue of column quarter u from its T digit sums
            auto quarter = [&](int u, const i32x4* cu) {
                const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)sw[u]);
                const float sz = s * (float)(((zw >> (4 * u)) & 15u) + 1u);
#pragma unroll
                for (int t = 0; t < T; t++) {
                    // digit products (|c| < 2^18, digit 3 most significant) in two exact integer
                    // pairs: 2^8 * sum_d c_d 2^(8d-24) = (c0 + 2^8 c1) 2^-16 + (c2 + 2^8 c3)
                    const int lo2 = cu[t][0] + cu[t][1] * 256;
                    const int hi2 = cu[t][2] + cu[t][3] * 256;
                    const float v = fmaf((float)lo2, 0x1p-16f, (float)hi2);
                    acc[b][u][t] = fmaf(s * st[t].x, v, acc[b][u][t]);
                    acc[b][u][t] = fmaf(-sz, st[t].y, acc[b][u][t]);
                }
            };
            // the first 64-k block starts each sum from an inline zero (no register setup)
            if constexpr (kLean) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    i32x4 c[T];
#pragma unroll
                    for (int bb = 0; bb < NB; bb++) {
                        const i32x4 bq = bq_of(bb, u);
#pragma unroll
                        for (int t = 0; t < T; t++) c[t] = mfma_i8(av[bb][t], bq, bb == 0 ? i32x4{0, 0, 0, 0} : c[t]);
                    }
                    quarter(u, c);
                }
            } else {
                i32x4 c[4][T];
#pragma unroll
                for (int bb = 0; bb < NB; bb++)
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const i32x4 bq = bq_of(bb, u);
#pragma unroll
                        for (int t = 0; t < T; t++) c[u][t] = mfma_i8(av[bb][t], bq, bb == 0 ? i32x4{0, 0, 0, 0} : c[u][t]);
                    }
#pragma unroll
                for (int u = 0; u < 4; u++) quarter(u, c[u]);
            }
        }
    };

    // the first chunk, then the ring's first P positions
    Stage sg;
    stage_open(sg, tb);
    stage_issue(sg);
    stage_finish(sg, 0);
    __syncthreads();
    bool staging = stage_next(sg);
    Cur fc;
    open(fc, tb);
#pragma unroll
    for (int d = 0; d < P; d++) {
        fetch(d, fc);
        advance(fc);
    }
    clear();

    int buf = 0;
    for (int ti = tb; ti < te; ti++) {
        const StripTask t = ld_table(a.tasks + ti);
        const SeqLinear* L = a.lin + t.linear;
        const int groups = ld_table(&L->K) / GK;
        const int nbw = blocks_of(t);
        const int nch = (groups + kCG - 1) / kCG;
        for (int ch = 0; ch < nch; ch++) {
            stage_issue(sg);                 // past the last chunk: repeats it (never finished)
            const int cgc = min(kCG, groups - ch * kCG);
            const int njobs = nbw > 0 && cgc > sp ? (cgc - sp + S - 1) / S : 0;
#pragma unroll
            for (int k = 0; k < QP; k += P) {
#pragma unroll
                for (int d = 0; d < P; d++) {
                    if (k + d < njobs) consume(d, buf, (k + d) * S + sp, nbw);
                    else touch(d);
                    fetch(d, fc);
                    advance(fc);
                }
            }
            if (S > 1 && ch + 1 == nch) {
                // parts 1 .. S-1 hand their sums to part 0 through LDS (one barrier, uniform:
                // every wave walks the same strips and chunks), which adds them in part order
                float* pl = part_lds();
                if (sp > 0 && nbw > 0) {
#pragma unroll
                    for (int tt = 0; tt < T; tt++) {
                        const int m = 4 * tt + kq;
                        if (m < M)
                            *reinterpret_cast<f32x4*>(pl + (((sp - 1) * WB + bw) * M + m) * kCols + 4 * j) =
                                f32x4{acc[0][0][tt], acc[0][1][tt], acc[0][2][tt], acc[0][3][tt]};
                    }
                }
                __syncthreads();
                if (sp == 0 && nbw > 0) {
#pragma unroll
                    for (int q = 1; q < S; q++)
#pragma unroll
                        for (int tt = 0; tt < T; tt++) {
                            const int m = 4 * tt + kq;
                            if (m < M) {
                                const f32x4 v = *reinterpret_cast<const f32x4*>(pl + (((q - 1) * WB + bw) * M + m) * kCols + 4 * j);
                                acc[0][0][tt] += v.x;
                                acc[0][1][tt] += v.y;
                                acc[0][2][tt] += v.z;
                                acc[0][3][tt] += v.w;
                            }
                        }
                }
            }
            if (ch + 1 == nch && nbw > 0 && sp == 0) {
                // the strip's outputs (bias from LDS: no global load on this path)
                const int N = ld_table(&L->N);
                float* y = ld_table(&L->y);
                const float* bl = bias_lds((ti - tb) & 1);
#pragma unroll
                for (int b = 0; b < BPW; b++) {
                    if (b > 0 && b >= nbw) break;
                    const int bc = (bw * BPW + b) * kCols + 4 * j;         // column within the strip
                    const int col = t.ct * kCols + bc;
                    const f32x4 bvv = *reinterpret_cast<const f32x4*>(bl + bc);
#pragma unroll
                    for (int tt = 0; tt < T; tt++) {
                        const int m = 4 * tt + kq;
                        if (m < M)
                            st_global(reinterpret_cast<f32x4*>(y + (size_t)m * N + col),
                                      f32x4{acc[b][0][tt] + bvv.x, acc[b][1][tt] + bvv.y, acc[b][2][tt] + bvv.z,
                                            acc[b][3][tt] + bvv.w});
                    }
                }
            }
            if (ch + 1 == nch) clear();
            if (staging) stage_finish(sg, buf ^ 1);
            __syncthreads();
            buf ^= 1;
            if (staging) staging = stage_next(sg);
        }
    }
}

struct StripKernel {
    const void* fn;
    int threads;
};

// Tunables (compile-time): jobs in flight per wave for M <= 4, <= 8 and <= 16, and the waves of
// the M 9..16 instance (8: one block each, two waves per SIMD; 4: two blocks each, a SIMD each).
#ifndef QL_STRIP_P1
#define QL_STRIP_P1 2
#endif
#ifndef QL_STRIP_P2
#define QL_STRIP_P2 2
#endif
#ifndef QL_STRIP_P4
#define QL_STRIP_P4 2
#endif
#ifndef QL_STRIP_W4
#define QL_STRIP_W4 8
#endif
// The planner starts each CU's second workgroup (the second half of a two-per-CU grid) this many
// block-groups behind: its waves issue after the first workgroup's and stream at about half its
// rate until that one's first strip ends. Measured on the 0.5B step (grid 512): 33.1 us per step
// at 48 or 80 against 34.6 at 0 and 36.3 or more at 112 and up.
#ifndef QL_STRIP_SECOND_OFFSET
#define QL_STRIP_SECOND_OFFSET 64
#endif

// Eight waves of one block each (two waves per SIMD, so one wave's MFMAs overlap the other's
// epilogue); M 9..16 as QL_STRIP_W4 says (four waves of two blocks measured 20% slower). With
// split 2, two waves share each block of a 4-block strip.
// jobs in flight: as asked when they fill a chunk's positions (kCG / S) in whole rounds, else 2
constexpr int ring_depth(int p, int S) { return (kCG / S) % p == 0 ? p : 2; }

template <int NB, int S, bool NT>
StripKernel strip_kernel_for_ns(int M)
{
    constexpr int P1 = ring_depth(QL_STRIP_P1, S), P2 = ring_depth(QL_STRIP_P2, S), P4 = ring_depth(QL_STRIP_P4, S);
    if (M <= 4) return {reinterpret_cast<const void*>(&strip_kernel<1, NB, 8, 1, P1, S, NT>), 64 * 8};
    if (M <= 8) return {reinterpret_cast<const void*>(&strip_kernel<2, NB, 8, 1, P2, S, NT>), 64 * 8};
    if (S > 1) return {reinterpret_cast<const void*>(&strip_kernel<4, NB, 8, 1, P4, S, NT>), 64 * 8};
    return {reinterpret_cast<const void*>(&strip_kernel<4, NB, QL_STRIP_W4, 8 / QL_STRIP_W4, P4, 1, NT>),
            64 * QL_STRIP_W4};
}

template <bool NT>
StripKernel strip_kernel_for_nt(int M, int group, int split)
{
    if (group == 64) return split == 2 ? strip_kernel_for_ns<1, 2, NT>(M) : strip_kernel_for_ns<1, 1, NT>(M);
    if (group == 128) return split == 2 ? strip_kernel_for_ns<2, 2, NT>(M) : strip_kernel_for_ns<2, 1, NT>(M);
    return {nullptr, 0};
}

// Packed weights that the MALL cannot keep until the next step are read with streaming
// (nontemporal) loads: the 7B step at M = 1 takes 503 us against 561 us with ordinary loads.
// Weights that it keeps (the 0.5B step) are read with ordinary loads, so that the next step
// finds them there (34.8 us against 38.6 us). Zeros and scales always use ordinary loads
// (streaming them too measured 2% slower on the 7B step).
StripKernel strip_kernel_for(int M, int group, int split, bool stream)
{
    return stream ? strip_kernel_for_nt<true>(M, group, split) : strip_kernel_for_nt<false>(M, group, split);
}

}  // namespace

// Two workgroups per CU when the weights stay in the 256 MB MALL (the 0.5B step: 39.9 against
// 41.6 us per step), one when they stream from HBM (the 7B step: 557 against 566 us).
// A CU holds two workgroups of the M <= 8 instances only (the M 9..16 instance takes 215 VGPRs,
// two waves per SIMD), so MALL-resident plans for M 9..16 use one workgroup per CU (the 0.5B step
// at M=16: 81.2 against 83.8 us with a second workgroup that waits for the first).
#ifndef QL_STRIP_MALL2_MAX_M
#define QL_STRIP_MALL2_MAX_M 8
#endif
int strip_grid(int cu_count, const std::vector<SeqSpec>& lin, int M)
{
    uint64_t bytes = 0;
    for (const SeqSpec& s : lin) bytes += s.weight_bytes;
    return cu_count * (bytes <= kStripMallBytes && M <= QL_STRIP_MALL2_MAX_M ? 2 : 1);
}

bool strip_eligible(const std::vector<SeqSpec>& lin, int M)
{
    if (M < kStripMinM || M > kGemvMaxM || lin.empty()) return false;
    uint64_t bytes = 0;
    for (const SeqSpec& s : lin) {
        if (s.src >= 0 || s.N % kCols != 0 || (s.group != 64 && s.group != 128) || s.group != lin[0].group ||
            s.K % s.group != 0)
            return false;
        bytes += s.weight_bytes;
    }
    return bytes >= kStripMinBytesPerCU * (uint64_t)kPlanCUs;
}

size_t strip_lds(int M, int group, int split)
{
    // two chunk buffers, two bias buffers, and the part sums of a split strip
    const size_t parts = (size_t)(split - 1) * (kMaxStripBlocks / split) * M * kCols * sizeof(float);
    return 2 * strip_buf_bytes(M, group / 64) + 2 * kMaxStripBlocks * kCols * sizeof(float) + parts;
}

namespace {

// force_stream: 1 plans the launch as streamed from HBM whatever its own bytes (one pass of a
// model whose weights do not stay in the MALL), -1 decides by the launch's bytes
void plan_strips_split(const std::vector<SeqSpec>& lin, int M, int grid, int split, int force_stream, StripPlan* out)
{
    StripPlan& p = *out;
    p = StripPlan{};
    p.grid = grid;
    p.split = split;
    const int SB = kMaxStripBlocks / split;   // blocks per strip
    struct Item {
        StripTask t;
        uint64_t cost;
    };
    std::vector<Item> items;
    for (int i = 0; i < (int)lin.size(); i++) {
        const int ct = lin[i].N / kCols;
        const int groups = lin[i].K / lin[i].group;
        const int chunks = (groups + kCG - 1) / kCG;
        for (int c = 0; c < ct; c += SB) {
            const int nb = std::min(SB, ct - c);
            // weight bytes in block-groups, plus a chunk of a full strip for the pipeline's start
            items.push_back(Item{StripTask{i, c, nb, chunks}, (uint64_t)nb * groups + (uint64_t)kCG * SB});
            p.total_units += (uint64_t)nb * groups;
        }
    }
    // longest first onto the least loaded workgroup
    std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) { return a.cost > b.cost; });
    std::vector<std::vector<StripTask>> per(grid);
    std::vector<uint64_t> load(grid, 0), units(grid, 0);
    typedef std::pair<uint64_t, int> Slot;
    std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>> q;
    // a CU's second workgroup starts behind its first (the first one's waves issue first). The
    // dispatcher fills the CUs with workgroups 0 .. CUs-1 first, so with two per CU (strip_grid's
    // rule: weights the MALL keeps, M <= QL_STRIP_MALL2_MAX_M) the second ones are grid/2 and up.
    uint64_t bytes = 0;
    for (const SeqSpec& s : lin) bytes += s.weight_bytes;
    const bool mall = force_stream >= 0 ? force_stream == 0 : bytes <= kStripMallBytes;
    const int second = mall && M <= QL_STRIP_MALL2_MAX_M ? grid / 2 : grid;
    for (int w = 0; w < grid; w++) {
        load[w] = w >= second ? (uint64_t)QL_STRIP_SECOND_OFFSET : 0;
        q.push({load[w], w});
    }
    for (const Item& it : items) {
        const Slot s = q.top();
        q.pop();
        per[s.second].push_back(it.t);
        load[s.second] = s.first + it.cost;
        units[s.second] += (uint64_t)it.t.nblk * (lin[it.t.linear].K / lin[it.t.linear].group);
        q.push({load[s.second], s.second});
    }
    p.task_begin.assign(grid + 1, 0);
    for (int w = 0; w < grid; w++) {
        p.task_begin[w] = (int32_t)p.tasks.size();
        p.tasks.insert(p.tasks.end(), per[w].begin(), per[w].end());
        p.busiest_units = std::max(p.busiest_units, units[w]);
    }
    p.task_begin[grid] = (int32_t)p.tasks.size();
    p.strips = (int)items.size();
    p.lds_bytes = lin.empty() ? 0 : strip_lds(M, lin[0].group, split);
}

}  // namespace

// Strips of 8 blocks, or of 4 with two waves per block when that balances the workgroups
// better (a strip of 8 blocks of a long-K linear can outweigh a workgroup's mean share).
static void plan_strips_base(const std::vector<SeqSpec>& lin, int M, int grid, int force_stream, StripPlan* out)
{
    uint64_t bytes = 0;
    for (const SeqSpec& s : lin) bytes += s.weight_bytes;
    plan_strips_split(lin, M, grid, 1, force_stream, out);
    out->stream = force_stream >= 0 ? force_stream != 0 : bytes > kStripMallBytes;
    if (out->total_units == 0) return;
    const double mean = (double)out->total_units / grid;
    if (out->busiest_units <= mean * kStripSplitBalance) return;
    StripPlan two;
    plan_strips_split(lin, M, grid, 2, force_stream, &two);
    two.stream = out->stream;
    if (two.busiest_units < out->busiest_units) *out = two;
}

// jobs in flight per wave of the no-padding kernel over whole-K strips (2 or 4)
#ifndef QL_WIDE_RING
#define QL_WIDE_RING 2
#endif

// The plan, then the no-padding kernel where it applies (QL_STRIP_WIDE=0 in the environment
// keeps strip_kernel, for comparisons).
static void plan_strips_final(const std::vector<SeqSpec>& lin, int M, int grid, int force_stream, StripPlan* out)
{
    plan_strips_base(lin, M, grid, force_stream, out);
    const char* env = getenv("QL_STRIP_WIDE");
    if ((!env || atoi(env) != 0) && strip_wide_eligible(lin, M, *out)) {
        // the M 5..8 instance runs two workgroups per CU: plan for that many, with strips of 8
        // blocks (the kernel's one block per wave) whatever the balance
        const int per_cu = strip_wide_per_cu(M);
        if (per_cu > 1 && grid <= kPlanCUs) {
            StripPlan two;
            plan_strips_split(lin, M, grid * per_cu, 1, force_stream, &two);
            two.stream = out->stream;
            *out = two;
        }
        // every strip must be 8 whole blocks: the kernel has no path for a shorter one
        bool whole = out->split == 1;
        for (const StripTask& t : out->tasks) whole = whole && t.nblk == kMaxStripBlocks;
        if (whole) {
            out->wide = true;
            out->ring = QL_WIDE_RING;
            out->lds_bytes = strip_wide_lds(M);
        } else {
            plan_strips_base(lin, M, grid, force_stream, out);
        }
    }
}

void plan_strips(const std::vector<SeqSpec>& lin, int M, int grid, StripPlan* out, int force_stream)
{
    plan_strips_final(lin, M, grid, force_stream, out);
}

void plan_strips_kparts(const std::vector<SeqSpec>& lin, int M, int grid, StripPlan* out)
{
    StripPlan& p = *out;
    p = StripPlan{};
    p.split = 1;
    p.stream = true;
    if (!strip_wide_eligible(lin, M, p, kPassMinM)) return;
    // the M <= 8 instance runs two workgroups per CU
    if (grid <= kPlanCUs) grid *= strip_wide_per_cu(M);
    p.grid = grid;
    int nstrips = 0;
    for (const SeqSpec& s : lin) nstrips += s.N / (kMaxStripBlocks * kCols);
    // at least two parts (every output goes through the part sums), and no more tasks than
    // workgroups: a task's time is mostly its fixed latency (first loads, digits, stores), so a
    // workgroup that runs two takes twice as long whatever their length
    const int target = std::max(2, grid / std::max(1, nstrips));
    struct Item {
        StripTask t;
        uint64_t cost;
    };
    std::vector<Item> items;
    for (int i = 0; i < (int)lin.size(); i++) {
        const int groups = lin[i].K / lin[i].group;
        const int chunks = groups / kCG;
        const int parts = std::min(chunks, target);
        for (int c = 0; c < lin[i].N / kCols; c += kMaxStripBlocks) {
            int c0 = 0;
            for (int q = 0; q < parts; q++) {
                const int nc = chunks / parts + (q < chunks % parts ? 1 : 0);
                items.push_back(Item{StripTask{i, c, kMaxStripBlocks, nc, c0, q, parts},
                                     (uint64_t)kMaxStripBlocks * nc * kCG + (uint64_t)kCG * kMaxStripBlocks});
                c0 += nc;
            }
            p.total_units += (uint64_t)kMaxStripBlocks * groups;
        }
    }
    std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) { return a.cost > b.cost; });
    std::vector<std::vector<StripTask>> per(grid);
    std::vector<uint64_t> units(grid, 0);
    typedef std::pair<uint64_t, int> Slot;
    std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>> q;
    for (int w = 0; w < grid; w++) q.push({0, w});
    for (const Item& it : items) {
        const Slot s = q.top();
        q.pop();
        per[s.second].push_back(it.t);
        units[s.second] += (uint64_t)it.t.nblk * it.t.chunks * kCG;
        q.push({s.first + it.cost, s.second});
    }
    p.task_begin.assign(grid + 1, 0);
    for (int w = 0; w < grid; w++) {
        p.task_begin[w] = (int32_t)p.tasks.size();
        p.tasks.insert(p.tasks.end(), per[w].begin(), per[w].end());
        p.busiest_units = std::max(p.busiest_units, units[w]);
    }
    p.task_begin[grid] = (int32_t)p.tasks.size();
    p.strips = nstrips;
    p.wide = true;
    p.ring = 4;
    p.staged = true;
    p.lds_bytes = strip_wide_lds(M);
}

hipError_t launch_strips(const StripArgs& a, size_t lds, hipStream_t stream)
{
    if (a.wide) return launch_strips_wide(a, lds, stream);
    const StripKernel k = strip_kernel_for(a.M, a.group, a.split, a.stream != 0);
    if (!k.fn) return hipErrorInvalidValue;
    void* args[] = {const_cast<StripArgs*>(&a)};
    return hipLaunchKernel(k.fn, dim3(a.G), dim3(k.threads), args, lds, stream);
}

}  // namespace ql
