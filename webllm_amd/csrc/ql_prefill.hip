// Prefill GEMM over many GPTQ int4 linears in one persistent launch, M > 16:
// y[M,N] = f16(x)[M,K] * f16(W)[N,K]^T (+ bias), fp32 accumulation, x fp16 or fp32 (rounded to
// fp16 as it is staged, as gemm_nt_f16_from_f32.wgsl:60 does in its tile load). The arithmetic of
// the reference's M > 1 path (gemm_nt_f16_from_f32.wgsl: fp16 operands, fp32 sums), with W
// dequantized from the packed int4 words inside the kernel, bit-identical to the load-time fp16
// arena (dequant_word_perm, ql_device.h).
//
// Work: tasks of one 128-row x 256-column output tile of one linear over all of K, so nothing is
// split along K and nothing is reduced. A workgroup (4 waves, one per SIMD) runs a list of tasks
// back to back; each wave owns 64 of the tile's columns for all 128 rows (8 x 4 accumulator tiles
// of v_mfma_f32_16x16x32_f16), so every dequantized weight fragment feeds 8 MFMAs.
// * K is walked in chunks of 128 (one quantization group for group 128). Per chunk the
//   activations (128 rows x 128 k, fp16, permuted into the k order dequant_word_perm emits) go to
//   LDS once behind one barrier (double-buffered), and each lane dequantizes the 16-byte packed
//   words of its 4 columns per 32-k block straight into its B fragments (no LDS for weights).
// * Within a chunk the four 32-k blocks are software-pipelined one block deep: the MFMAs of block
//   kb issue interleaved with the LDS reads and dequantization of block kb + 1, each block in a
//   scheduling region of its own (sched_barrier) with the interleave fixed by
//   sched_group_barrier. Left to itself the compiler reads each pair of A fragments into the
//   same registers right before their MFMAs and dequantizes between blocks, so an LDS round trip
//   stalls every 8 MFMAs (measured: 38 cycles per MFMA in the loop against 16 at peak).
// * Every load runs one chunk ahead, across task boundaries: the chunk after the last one of a
//   task is the next task's first, so the pipeline never drains between tasks. Register slots
//   are refilled as soon as they are consumed (the activations when written to LDS, a block's
//   packed words when dequantized, the scales and zeros when expanded).
// * The bias of a task is staged in LDS with the activations of its first chunk (a register
//   would carry a load across the whole task) and read at its end; two bias buffers alternate by
//   task parity, because the barrier between a task's end and the next-but-one task's start is the
//   only one that orders them.
// * Tasks come from a host plan (longest first onto the least-loaded workgroup, ties on one XCD)
//   or, for a batch of up to 8 linears, from the tile numbering itself (workgroup w takes tiles
//   w, w + G, ...).
#include "ql_device.h"
#include "ql_digits.h"
#include "ql_internal.h"

#include <algorithm>
#include <queue>

namespace ql {

namespace {

constexpr int kBM = kPrefillRows;      // rows per tile
constexpr int kBN = kPrefillCols;      // columns per tile, 64 per wave
constexpr int kMT = kBM / 16;          // 16-row MFMA tiles per wave
constexpr int kAC = kBM * 16 / 256;    // 16-byte activation pieces per thread per chunk

// qzeros word of a linear without qzeros: every stored zero 7 (true zero 8)
__device__ const uint32_t kPrefillSymZeros = 0x77777777u;
// bias of a linear without one
__device__ const float kPrefillZeros[4] = {0.f, 0.f, 0.f, 0.f};

template <typename T>
__device__ __forceinline__ T ld_tab(const T* p)
{
#if defined(__HIP_DEVICE_COMPILE__)
    // tables are written before any launch: constant address space, scalar loads
    return *(const __attribute__((address_space(4))) T*)(reinterpret_cast<uintptr_t>(p));
#else
    return *p;
#endif
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// 8 activations (natural k order, fp16) in the order dequant_word_perm emits {0,4,1,5,2,6,3,7}
__device__ __forceinline__ u32x4 perm_k8(u32x4 nat)
{
    u32x4 r;
    r.x = __builtin_amdgcn_perm(nat.z, nat.x, 0x05040100u);   // k0 | k4
    r.y = __builtin_amdgcn_perm(nat.z, nat.x, 0x07060302u);   // k1 | k5
    r.z = __builtin_amdgcn_perm(nat.w, nat.y, 0x05040100u);   // k2 | k6
    r.w = __builtin_amdgcn_perm(nat.w, nat.y, 0x07060302u);   // k3 | k7
    return r;
}

// 8 activations (natural k order) as fp16 bits: fp16 as loaded, or fp32 rounded to nearest even
template <bool XF32>
__device__ __forceinline__ u32x4 to_f16x8(const u32x4* x)
{
    if constexpr (!XF32) {
        return x[0];
    } else {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        const f32x4 lo = __builtin_bit_cast(f32x4, x[0]), hi = __builtin_bit_cast(f32x4, x[1]);
        u32x4 r;
        r.x = as_u32(__builtin_convertvector(f32x2{lo.x, lo.y}, f16x2));
        r.y = as_u32(__builtin_convertvector(f32x2{lo.z, lo.w}, f16x2));
        r.z = as_u32(__builtin_convertvector(f32x2{hi.x, hi.y}, f16x2));
        r.w = as_u32(__builtin_convertvector(f32x2{hi.z, hi.w}, f16x2));
        return r;
    }
}

// One task's coordinates (uniform across the workgroup).
struct Pos {
    int q;       // task ordinal in this workgroup's list
    int c;       // chunk within the task
    int nch;     // chunks of the task
    int li, m0, n0;
};

template <bool TABLE>
__device__ __forceinline__ void task_at(const PrefillArgs& a, int w, int q, Pos& p)
{
    int li, mt, nt;
    if (TABLE) {
        const PrefillTask t = ld_tab(a.tasks + ld_tab(a.task_begin + w) + q);
        li = t.linear;
        mt = t.mt;
        nt = t.nt;
    } else {
        const int i = w + q * a.G;
        li = 0;
#pragma unroll
        for (int k = 1; k < kMaxBatch; k++)
            if (k < a.count && i >= a.L[k].tile_begin) li = k;
        const int local = i - a.L[li].tile_begin;
        mt = local % a.L[li].tiles_m;
        nt = local / a.L[li].tiles_m;
    }
    p.li = uniform(li);
    p.m0 = uniform(mt * kBM);
    p.n0 = uniform(nt * kBN);
    p.nch = uniform((TABLE ? ld_tab(a.lin + p.li).K : a.L[p.li].K) / 128);
}

template <bool TABLE>
__device__ __forceinline__ PrefillLinear lin_at(const PrefillArgs& a, int li)
{
    return TABLE ? ld_tab(a.lin + li) : a.L[li];
}

// XF32: fp32 activations, loaded as 32 bytes per 8-k piece and rounded to fp16 (round to
// nearest even, v_cvt_pk_f16_f32) when the piece is written to LDS
template <bool TABLE, bool XF32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void prefill_kernel(const PrefillArgs a)
{
    // [buffer][k block][k quarter][row ^ (4 k block + k quarter)]: 8 fp16 in dequant order. The
    // xor spreads both the staging writes (16 lanes: one row, 16 planes) and the fragment reads
    // (16 lanes: 16 rows, one plane) over distinct banks: SQ_LDS_BANK_CONFLICT reads 0 (a spare row
    // per plane instead left 40 % of the LDS cycles in conflicts)
    __shared__ u32x4 As[2][4][4][kBM];
    __shared__ f32x4 Bs[2][kBN / 4];      // bias of the current task, alternating by task parity

    const int w = blockIdx.x;
    const int ntasks = TABLE ? ld_tab(a.task_begin + w + 1) - ld_tab(a.task_begin + w)
                             : (w < a.total_tiles ? (a.total_tiles - w + a.G - 1) / a.G : 0);
    if (ntasks == 0) return;
    const int M = a.M;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kq = lane >> 4;
    // dequantization constants held in registers (see magic_pair_r)
    uint32_t kmask = 0x000F000Fu, kmagic = 0x64006400u;
    asm volatile("" : "+s"(kmask));
    asm volatile("" : "+v"(kmagic));

    // activation piece e = threadIdx.x + 256 a: row e / 16, 8-k piece e % 16 of the chunk
    int arow[kAC], apc[kAC];
#pragma unroll
    for (int e = 0; e < kAC; e++) {
        const int idx = threadIdx.x + 256 * e;
        arow[e] = idx >> 4;
        apc[e] = idx & 15;
    }

    // ---- the load side: the chunk after the one being computed
    Pos nx;
    nx.q = 0;
    nx.c = 0;
    task_at<TABLE>(a, w, 0, nx);
    constexpr int XS = XF32 ? 2 : 1;      // 16-byte loads per 8-k activation piece
    constexpr uint32_t XE = XF32 ? 4 : 2;  // bytes per activation
    u32x4 xa[kAC][XS];
    u32x4 wq[4];
    u32x2 sv;
    uint32_t zv;
    f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};
    // lane-side pointers of the load position (recomputed when it enters a new task)
    const char* xp[kAC];
    const uint32_t* qwp;
    const uint16_t* scp;
    const uint32_t* qzp;
    const float* bp;
    int nN, nzstride, ngroup;
    auto enter = [&](const Pos& p) {
        const PrefillLinear L = lin_at<TABLE>(a, p.li);
        const int ncol = p.n0 + wave * 64 + 4 * j;
        const int nc = ncol < L.N ? ncol : 0;
#pragma unroll
        for (int e = 0; e < kAC; e++)
            xp[e] = static_cast<const char*>(L.x) + ((size_t)min(p.m0 + arow[e], M - 1) * L.K + 8 * apc[e]) * XE;
        qwp = L.qweight + nc + (size_t)kq * L.N;
        scp = L.scales + nc;
        qzp = L.qzeros ? L.qzeros + (nc >> 3) : &kPrefillSymZeros;
        nzstride = L.qzeros ? (L.N + 7) >> 3 : 0;
        nN = L.N;
        ngroup = L.group;
        // bias of the task, columns n0 + 4 (tid % 64) .. + 3 (the first 64 threads stage them);
        // zeros past N or without bias
        const int bcol = p.n0 + 4 * (threadIdx.x & 63);
        bp = L.bias && bcol < L.N ? L.bias + bcol : kPrefillZeros;
    };
    // every chunk loads the bias of its task with its activations (unconditionally, so the wait
    // for them is one and the same), though only a task's first chunk stages it
    auto load_x = [&](int c) {
#pragma unroll
        for (int e = 0; e < kAC; e++)
#pragma unroll
            for (int h = 0; h < XS; h++)
                xa[e][h] = ld_global(reinterpret_cast<const u32x4*>(xp[e] + (size_t)c * 128 * XE) + h);
        bv = ld_global(reinterpret_cast<const f32x4*>(bp));
    };
    auto load_sz = [&](int c) {
        const int g = c * 128 / ngroup;
        sv = ld_global(reinterpret_cast<const u32x2*>(scp + (size_t)g * nN));
        zv = ld_global(qzp + (size_t)g * nzstride);
    };
    auto load_w = [&](int c, int kb) {
        wq[kb] = ld_global(reinterpret_cast<const u32x4*>(qwp + (size_t)(c * 16 + 4 * kb) * nN));
    };
    // moves the load position one chunk on (past the last task it stays on the last chunk, whose
    // loads are repeated and never consumed)
    auto advance = [&]() {
        if (nx.c + 1 < nx.nch) {
            nx.c++;
        } else if (nx.q + 1 < ntasks) {
            nx.q++;
            nx.c = 0;
            task_at<TABLE>(a, w, nx.q, nx);
            enter(nx);
        }
    };

    enter(nx);
    load_x(0);
    load_sz(0);
#pragma unroll
    for (int kb = 0; kb < 4; kb++) load_w(0, kb);

    // ---- the compute side: the tasks in order, each over its chunks, then its outputs
    int slot = 0;
    for (int q = 0; q < ntasks; q++) {
        Pos cu;
        cu.q = q;
        task_at<TABLE>(a, w, q, cu);
        f32x4 acc[kMT][4];
#pragma unroll
        for (int tm = 0; tm < kMT; tm++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc[tm][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int zsh = 4 * ((cu.n0 + wave * 64 + 4 * j) & 7);
        auto chunk = [&](int c) {
            // 1. this chunk's activations (and, at the task's first chunk, its bias) into LDS
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < kAC; e++) As[slot][apc[e] >> 2][apc[e] & 3][arow[e] ^ apc[e]] = perm_k8(to_f16x8<XF32>(xa[e]));
            if (c == 0 && threadIdx.x < 64) Bs[q & 1][threadIdx.x] = bv;
            uint32_t zz[4], ss[4];
            {
                const uint32_t zw = zv >> zsh;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    zz[t] = zero_pair(((zw >> (4 * t)) & 15u) + 1u);
                    ss[t] = (((t < 2 ? sv.x : sv.y) >> (16 * (t & 1))) & 0xFFFFu) * 0x10001u;
                }
            }
            // 2. the next chunk's activations, bias, scales and zeros
            advance();
            load_x(nx.c);
            load_sz(nx.c);
            __syncthreads();

            // 3. four 32-k blocks, software-pipelined one block deep: while the 32 MFMAs of block
            //    kb issue, the A fragments of block kb + 1 come from LDS, its B fragments are
            //    dequantized from the packed words, and those words' slot is refilled for the
            //    next chunk
            u32x4 af[2][kMT];
            f16x8 bf[2][4];
#pragma unroll
            for (int tm = 0; tm < kMT; tm++) af[0][tm] = As[slot][0][kq][(16 * tm + j) ^ kq];
#pragma unroll
            for (int t = 0; t < 4; t++) bf[0][t] = dequant_word_perm_r(wq[0][t], zz[t], ss[t], kmask, kmagic);
            load_w(nx.c, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                if (kb < 3) {
#pragma unroll
                    for (int tm = 0; tm < kMT; tm++) af[(kb + 1) & 1][tm] = As[slot][kb + 1][kq][(16 * tm + j) ^ (4 * (kb + 1) + kq)];
#pragma unroll
                    for (int t = 0; t < 4; t++) bf[(kb + 1) & 1][t] = dequant_word_perm_r(wq[kb + 1][t], zz[t], ss[t], kmask, kmagic);
                    load_w(nx.c, kb + 1);
                }
#pragma unroll
                for (int tm = 0; tm < kMT; tm++)
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        acc[tm][t] = mfma_16x16x32_f16(__builtin_bit_cast(f16x8, af[kb & 1][tm]), bf[kb & 1][t], acc[tm][t]);
                // one region per block: its MFMAs interleaved with the next block's LDS reads and
                // dequantization; no MFMA of the next block moves into it
                if (kb < 3) {
#pragma unroll
                    for (int r = 0; r < 8; r++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            slot ^= 1;
        };
        // the first chunk apart: it alone follows the previous task's stores, so the waits of
        // the loop over the others see the same loads in flight on every path
        chunk(0);
        for (int c = 1; c < cu.nch; c++) chunk(c);

        // 4. the tile's outputs, bias (and a residual) added: lane (j, kq) holds rows
        //    16 tm + 4 kq + r of its 4 adjacent columns; streaming stores (the outputs are not
        //    read back by the launch)
        const PrefillLinear cl = lin_at<TABLE>(a, cu.li);
        const int ncol = cu.n0 + wave * 64 + 4 * j;
        if (ncol < cl.N && cl.res) {
            // y = W.x + bias + res, rows past M skipped (the residual is read only where stored)
            const f32x4 bias = Bs[q & 1][wave * 16 + j];
            const size_t o0 = (size_t)(cu.m0 + 4 * kq) * cl.N + ncol;
#pragma unroll
            for (int tm = 0; tm < kMT; tm++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (cu.m0 + 16 * tm + 4 * kq + r < M) {
                        const size_t o = o0 + (size_t)(16 * tm + r) * cl.N;
                        const f32x4 rv = *reinterpret_cast<const f32x4*>(cl.res + o);
                        __builtin_nontemporal_store(
                            f32x4{acc[tm][0][r] + bias.x + rv.x, acc[tm][1][r] + bias.y + rv.y,
                                  acc[tm][2][r] + bias.z + rv.z, acc[tm][3][r] + bias.w + rv.w},
                            reinterpret_cast<f32x4*>(cl.y + o));
                    }
        } else if (ncol < cl.N) {
            const f32x4 bias = Bs[q & 1][wave * 16 + j];
            float* yb = cl.y + (size_t)(cu.m0 + 4 * kq) * cl.N + ncol;
            if (cu.m0 + kBM <= M) {
#pragma unroll
                for (int tm = 0; tm < kMT; tm++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        __builtin_nontemporal_store(f32x4{acc[tm][0][r] + bias.x, acc[tm][1][r] + bias.y, acc[tm][2][r] + bias.z,
                                        acc[tm][3][r] + bias.w}, reinterpret_cast<f32x4*>(yb + (size_t)(16 * tm + r) * cl.N));
            } else {
#pragma unroll
                for (int tm = 0; tm < kMT; tm++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (cu.m0 + 16 * tm + 4 * kq + r < M)
                            __builtin_nontemporal_store(
                                      f32x4{acc[tm][0][r] + bias.x, acc[tm][1][r] + bias.y,
                                            acc[tm][2][r] + bias.z, acc[tm][3][r] + bias.w},
                                      reinterpret_cast<f32x4*>(yb + (size_t)(16 * tm + r) * cl.N));
            }
        }
    }
}

}  // namespace

bool prefill_ok(int M, int N, int K, int group, int x_dtype)
{
    // every buffer offset of the launch (activations, outputs, packed weights) stays below 2^31
    const int64_t lim = INT64_C(1) << 31;
    return M > kGemvMaxM && (x_dtype == 0 || x_dtype == 1) && N > 0 && N % 4 == 0 && group > 0 &&
           group % 128 == 0 && K > 0 && K % group == 0 && (int64_t)M * N * 4 < lim &&
           (int64_t)M * K * (x_dtype == 0 ? 4 : 2) < lim && (int64_t)K * N / 2 < lim;
}

int prefill_tiles(int M, int N) { return ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN); }

// Longest first onto the least-loaded workgroup; among equally loaded ones the workgroups of
// one XCD come in a row (the hardware deals workgroup w to XCD w % 8), so consecutive tiles -
// the row tiles of one column strip, then the next strip - meet their weights and activations
// in one L2.
void plan_prefill(const std::vector<PrefillSpec>& lin, int M, int grid, PrefillPlan* out)
{
    PrefillPlan& p = *out;
    p = PrefillPlan{};
    p.grid = grid;
    struct Item {
        PrefillTask t;
        uint64_t cost;
    };
    std::vector<Item> items;
    const int tm = (M + kBM - 1) / kBM;
    for (int i = 0; i < (int)lin.size(); i++) {
        const int tn = (lin[i].N + kBN - 1) / kBN;
        for (int nt = 0; nt < tn; nt++)
            for (int mt = 0; mt < tm; mt++) {
                // chunks, plus one for the task's epilogue
                items.push_back(Item{PrefillTask{i, mt, nt, 0}, (uint64_t)lin[i].K / 128 + 1});
                p.total_units += (uint64_t)lin[i].K / 128;
            }
    }
    std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) { return x.cost > y.cost; });
    auto order = [grid](int w) { return grid % 8 == 0 ? (w % 8) * (grid / 8) + w / 8 : w; };
    std::vector<int> by_order(grid);
    for (int w = 0; w < grid; w++) by_order[order(w)] = w;
    std::vector<std::vector<PrefillTask>> per(grid);
    std::vector<uint64_t> units(grid, 0);
    typedef std::pair<uint64_t, int> Slot;      // (load, XCD-major order)
    std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>> q;
    for (int o = 0; o < grid; o++) q.push({0, o});
    for (const Item& it : items) {
        const Slot s = q.top();
        q.pop();
        const int wg = by_order[s.second];
        per[wg].push_back(it.t);
        units[wg] += it.cost - 1;
        q.push({s.first + it.cost, s.second});
    }
    p.task_begin.assign(grid + 1, 0);
    for (int w = 0; w < grid; w++) {
        p.task_begin[w] = (int32_t)p.tasks.size();
        p.tasks.insert(p.tasks.end(), per[w].begin(), per[w].end());
        p.busiest_units = std::max(p.busiest_units, units[w]);
    }
    p.task_begin[grid] = (int32_t)p.tasks.size();
}

hipError_t launch_prefill(const PrefillArgs& a, bool table, hipStream_t stream)
{
    if (a.G < 1) return hipErrorInvalidValue;
    if (table) {
        if (a.x_f32) hipLaunchKernelGGL((prefill_kernel<true, true>), dim3(a.G), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((prefill_kernel<true, false>), dim3(a.G), dim3(256), 0, stream, a);
    } else {
        if (a.x_f32) hipLaunchKernelGGL((prefill_kernel<false, true>), dim3(a.G), dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((prefill_kernel<false, false>), dim3(a.G), dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace ql
