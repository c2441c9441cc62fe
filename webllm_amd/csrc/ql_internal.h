// Host-side interface between the C ABI (ql_api.hip) and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

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
hipError_t launch_gemm_simple(const GemmArgs& a, hipStream_t stream);

// GEMM on MFMA: workgroups of BM rows x kGemmTileCols columns x one K segment; several linears
// (same M and x dtype) can share a launch.
constexpr int kGemmTileCols = 256;
constexpr int kPlanCUs = 256;          // CU count plans assume (MI355X), so plans are device-free
struct GemmLinear {
    const uint32_t* qweight;   // [K/8, N]
    const uint32_t* qzeros;    // [K/group, ceil(N/8)] or nullptr (zero 8)
    const uint16_t* scales;    // [K/group, N] fp16 bits
    const float* bias;         // [N] or nullptr
    const void* x;             // [M, K] f32 or f16
    float* y;                  // [M, N]
    float* partial;            // [split, M, N] (split > 1)
    uint32_t* counters;        // per-tile arrival counters (split > 1), zero between launches
    const float* res;          // [M, N] added at the store, or nullptr
    int N, K, group, split, tiles_n, tiles_m, wg_begin;
    int defer;                 // split > 1: store the partial sums only (a part-sum launch adds them)
};
struct GemmBatch {
    GemmLinear L[kMaxBatch];
    int count, M, x_dtype, bm, wg_total;
};
struct GemmShape {
    int bm, tiles_n, tiles_m, split;
};
bool gemm_fast_ok(int M, int N, int K, int group);
GemmShape gemm_shape(int M, int N, int K, int group, int cu_count);
uint64_t gemm_partial_bytes(int M, int N, int split);
hipError_t launch_gemm_batch(const GemmBatch& b, hipStream_t stream);

// Prefill GEMM over many linears in one persistent launch (M > 16, fp16 x, groups a multiple of
// 128): tasks of one 128 x 256 output tile over all of K, from a host plan (table) or from the
// tile numbering of a batch of up to kMaxBatch linears.
constexpr int kPrefillRows = 128;
constexpr int kPrefillCols = 256;
#ifndef QL_PREFILL_MIN_TILES
#define QL_PREFILL_MIN_TILES 128
#endif
constexpr int kPrefillMinTiles = QL_PREFILL_MIN_TILES;   // fewest tiles a ql_linear(_batch) launch takes it for
struct PrefillLinear {
    const uint32_t* qweight;   // [K/8, N]
    const uint32_t* qzeros;    // [K/group, ceil(N/8)] or nullptr (zero 8)
    const uint16_t* scales;    // [K/group, N] fp16 bits
    const float* bias;         // [N] or nullptr
    const void* x;             // [M, K] fp16, or fp32 (PrefillArgs::x_f32)
    float* y;                  // [M, N]
    const float* res;          // [M, N] added at the store, or nullptr
    int32_t N, K, group;
    int32_t tiles_m;           // batch mode: row tiles, and the linear's first tile number
    int32_t tile_begin;
    int32_t pad;
};
struct PrefillTask {
    int32_t linear, mt, nt, pad;
};
struct PrefillArgs {
    const PrefillLinear* lin;  // table mode: linears, tasks, and each workgroup's first task [G + 1]
    const PrefillTask* tasks;
    const int32_t* task_begin;
    PrefillLinear L[kMaxBatch];// batch mode: the linears; workgroup w takes tiles w, w + G, ...
    int32_t count, total_tiles;
    int32_t M, G;
    int32_t x_f32;             // 1: x is fp32, rounded to fp16 (RNE) as it is staged
};
struct PrefillSpec {
    int N, K;
};
struct PrefillPlan {
    int grid = 0;
    uint64_t total_units = 0, busiest_units = 0;   // 128-k chunks: all, most on one workgroup
    std::vector<PrefillTask> tasks;
    std::vector<int32_t> task_begin;
};
bool prefill_ok(int M, int N, int K, int group, int x_dtype);
int prefill_tiles(int M, int N);
void plan_prefill(const std::vector<PrefillSpec>& lin, int M, int grid, PrefillPlan* out);
hipError_t launch_prefill(const PrefillArgs& a, bool table, hipStream_t stream);

// load-time unpack to fp16 [N, K]
struct UnpackArgs {
    const uint32_t* qweight;
    const uint32_t* qzeros;
    const uint16_t* scales;
    void* out;                 // fp16 [N,K] (launch_unpack) or fp32 [N,K] (launch_unpack_f32)
    int N, K, group;
    const float* scales_f32;   // launch_unpack_f32 only: f32 scales [K/group, N] used instead of
                               // `scales` when set
};
hipError_t launch_unpack(const UnpackArgs& a, bool fast, hipStream_t stream);
// Batched fp16 unpack: up to kUnpackBatch tensors (each meeting the tile path's conditions: N % 4 == 0,
// K % 8 == 0, 16-byte aligned qweight and output, 8-byte aligned scales) in one launch.
constexpr int kUnpackBatch = 32;
struct UnpackItem {
    const uint32_t* qweight;
    const uint32_t* qzeros;    // or nullptr (zero 8)
    const uint16_t* scales;
    uint16_t* out;             // fp16 [N, K]
    int N, K, group;
    int tile_begin;            // the tensor's first tile in the batch numbering
};
struct UnpackBatch {
    UnpackItem it[kUnpackBatch];
    int count, tiles;
};
int unpack_tiles(int N, int K);    // 16-packed-row x 64-column tiles of one tensor
hipError_t launch_unpack_batch(const UnpackBatch& b, hipStream_t stream);
hipError_t launch_unpack_f32(const UnpackArgs& a, hipStream_t stream);

// fp16-weight GEMV (tied lm_head / embedding): y[M,N] = x[M,K] . W[N,K]^T (+ bias), fp32 x/y.
struct F16wArgs {
    const uint16_t* w;         // fp16 [N, K] row-major
    const float* bias;         // [N] or nullptr
    const float* x;            // [M, K]
    float* y;                  // [M, N]
    int M, N, K;
};
bool gemv_f16w_fast_ok(int M, int N, int K);
size_t gemv_f16w_lds(int M, int K);
hipError_t launch_gemv_f16w(const F16wArgs& a, bool fast, int cu_count, hipStream_t stream);

// The embedding lookup over the fp16 table: out[r, :] = f32(w[tokens[r], :]).
struct EmbedArgs {
    const uint16_t* w;         // fp16 [vocab, D]
    const uint32_t* tokens;    // [rows]
    float* out;                // [rows, D]
    int vocab, D, rows;
    int vec;                   // D % 8 == 0 and w, out 16-byte aligned: 8 values per lane
};
hipError_t launch_embed_rows(const EmbedArgs& a, hipStream_t stream);

// Decode attention over an fp32 KV cache [max_t, KV * D] and the cache store.
constexpr int kAttnMaxT = 8192;        // visible keys per query row
constexpr int kAttnMaxD = 256;
constexpr size_t kAttnWsBytes = 4u << 20;   // context workspace for key-split partials
struct AttnArgs {
    const float* q;            // [M, H, D]
    const float* k;            // cache [max_t, KV * D]
    const float* v;
    float* out;                // [M, H, D]
    float* ws;                 // key-split partials: [M, H, nsplit, D] sums, then [.., 2] max/sum
    int M, H, KV, G, D, past;
    float scale;               // fp32(log2(e) / sqrt(D)): scores in base-2 units for exp2
    // plan_attention fills these
    int gm, nj;                // kernel variant: heads per run (template), 64-float pieces of D
    int heads_per_run, runs_per_group, nsplit, chunk_cap;
};
int plan_attention(AttnArgs* a);

// Residual add + RMSNorm, SiLU-mul.
struct ElemArgs {
    const float* x;            // [M, C]
    const float* d;            // [M, C] added to x, or nullptr
    const float* w;            // [C] norm weight
    float* s;                  // x + d stored here (nullptr: not stored)
    float* y;                  // [M, C]
    int M, C;
    float eps;
    int vec;                   // C % 4 == 0 and every pointer 16-byte aligned: f32x4 path
};
hipError_t launch_add_rmsnorm(const ElemArgs& a, hipStream_t stream);
hipError_t launch_silu_mul(const float* gate, const float* up, float* y, long long n, hipStream_t stream);
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);
hipError_t launch_kv_store(const float* src, float* dst, int rows, int row_len, int pos0, hipStream_t stream);

// ----------------------------------------------------------------------------------------------
// Linear sequences: many decode linears (M <= 16) in one persistent launch. Linear i may read the
// output of an earlier linear; the kernel orders them on the device.

constexpr int kSeqMaxLinears = 4096;
constexpr int kSeqMaxRows = 65536;     // rows of a sequence (above kGemvMaxM: prefill GEMM)
constexpr int kSeqTileCols = 64;       // output columns per sequence tile (one wave's width)
constexpr int kSeqMaxSplit = 4096;     // parts (K pieces) of one 64-column block, at most
constexpr int kSeqTickets = 32;        // per-run ticket sub-counters (epoch), 64 B apart
constexpr int kSeqTile = 0;
constexpr int kSeqReduce = 1;
constexpr uint32_t kSeqErrTimeout = 1;
constexpr int kSeqBiasBlocks = 64;    // most (block, row) pairs whose bias (+ residual) a tile stages in LDS

// Device table entry per linear (read-only in the kernel).
// Elementwise work folded into a sequence linear (SeqLinear::fuse bits).
constexpr int kFuseNorm = 1;   // x -> rmsnorm(x) * norm_w at staging
constexpr int kFuseGlu = 2;    // x -> silu(x) * x2 at staging
constexpr int kFuseRes = 4;    // y -> y + res in the epilogue
constexpr int kFuseSsq = 8;    // (tasks only) a consumer normalizes this output: emit its sums of squares

struct SeqLinear {
    const uint32_t* qweight;
    const uint32_t* qzeros;    // never null: symmetric linears point at stored-7 words
    const uint16_t* scales;
    const float* bias;
    const void* x;             // external input [M, K] (src < 0)
    float* y;                  // output [M, N] for the caller
    uint64_t* y_ll;            // output again as (value bits | epoch << 32) for consumers
    int32_t src;               // producer linear (its y is this linear's x), or -1
    int32_t N, K, x_dtype;
};

// A fused sequence linear's elementwise work, in a table of its own beside SeqLinear (read only
// by the fused kernel instance, where it is needed).
struct SeqFuseLin {
    const float* norm_w;       // RMSNorm weight [K] (kFuseNorm)
    const float* x2;           // external second GLU operand [M, K], f32 (kFuseGlu, src2 < 0)
    const float* res;          // external residual [M, N], f32 (kFuseRes, res_src < 0)
    uint64_t* ssq;             // [M][ceil(N/64)] epoch words: sums of squares of the output's
                               // rows by 64-column block, for a consumer that normalizes it
    int32_t src2, res_src;     // producer linears of x2 and res, or -1
    int32_t fuse;              // kFuse* bits
    float norm_eps;
};

// One unit of work, run by one workgroup in list order.
//  tile:   blocks ct .. ct+nblk-1 (64 columns each) over groups [g0, g1) of K. slot < 0: the
//          blocks are whole (all of K) and the tile writes the outputs; otherwise block ct+b
//          writes its partial sums to pool slot (slot + b*stride).
//  reduce: blocks ct .. ct+nblk-1, each the sum of `parts` partial slots (slot + b*stride + p,
//          p = 0..parts-1, in ascending K order), plus bias; writes the outputs.
struct SeqTask {
    int32_t linear, kind, ct, nblk;
    int32_t g0, g1, slot, stride;
    int32_t parts;
    int32_t next_tile;         // index of the same workgroup's next tile task, or -1
    int32_t fuse;              // the linear's kFuse* bits (| kFuseSsq), read with the task
    int32_t pad;
};

struct SeqArgs {
    const SeqLinear* lin;
    const SeqTask* tasks;
    const int32_t* task_begin;      // [G + 1]
    const int32_t* first_tile;      // [G], -1 when a workgroup has no tile task
    unsigned long long* tickets;    // [kSeqTickets * 8]
    uint32_t* abort;
    uint32_t* err;
    uint64_t* part;                 // partial-sum pool: slot s holds [M][64] epoch-tagged words
    int32_t M, G, group;
    uint32_t spin_limit;
    int32_t block_mode;             // some tile runs in block mode: launch the instance with it
    int32_t fused;                  // some linear has fused elementwise work: the instance with it
    const SeqFuseLin* fl;           // [n] when fused
};

// Host description of one linear of a sequence, for planning.
struct SeqSpec {
    int N, K, group, src;
    bool has_qzeros, has_bias;
    uint64_t weight_bytes;
    int src2 = -1, res_src = -1;    // producers of the GLU operand and the residual, or -1
    int fuse = 0;                   // kFuse* bits
};

struct SeqPlanOut {
    int grid = 0, passes = 0, tiles = 0, reduces = 0, max_split = 1, max_gseg = 0;
    uint64_t slots = 0;             // partial-sum pool slots
    uint64_t total_units = 0, busiest_units = 0;   // block-groups: all, most on one workgroup
    bool block_mode = false;        // some tile runs in block mode
    uint64_t lds_bytes = 0;
    std::vector<int> pass_of;
    std::vector<SeqTask> tasks;
    std::vector<int32_t> task_begin, first_tile;
};

// Pure planning (no device calls): passes from the dependencies, a split per linear, tiles and
// reductions dealt to `grid` workgroups.
void plan_seq(const std::vector<SeqSpec>& lin, int M, int grid, SeqPlanOut* out);
// Checks a plan against its linears: every (linear, column block, group) computed by exactly one
// tile; a block split into parts reduced exactly once, over slots in ascending K order that its
// tiles write; passes in order within each workgroup's list, and a pass's reductions after all
// of that workgroup's tiles of the pass. Returns an empty string or the first violation.
std::string verify_seq_plan(const std::vector<SeqSpec>& lin, int M, const SeqPlanOut& p);
size_t seq_lds_budget(int M, int group);   // dynamic LDS a sequence may use per workgroup
// Workgroups of the sequence kernel that fit on one CU at once.
hipError_t seq_blocks_per_cu(int M, int group, bool fused, int* blocks);
int seq_wg_per_cu();
hipError_t launch_seq(const SeqArgs& a, size_t lds, hipStream_t stream);

// ----------------------------------------------------------------------------------------------
// Column strips: a sequence of independent linears (no linear reads another's output) as one
// persistent launch, each workgroup owning strips of 8 whole 64-column blocks (or 4, two waves per
// block) over all of K (no K splits across workgroups). Groups of 64 or 128, N % 64 == 0. Measured
// against the dependency-ordered tiles: equal on the 0.5B step at M = 1, faster at every M > 1 and
// on the 7B step (QL_STRIP_MIN_KB_PER_CU can restrict strips to weights streamed from HBM).
constexpr int kStripMinM = 1;           // fewest rows the strip path serves
#ifndef QL_STRIP_MIN_KB_PER_CU
#define QL_STRIP_MIN_KB_PER_CU 0
#endif
constexpr uint64_t kStripMinBytesPerCU = (uint64_t)QL_STRIP_MIN_KB_PER_CU << 10;   // weight bytes per CU from which it does
#ifndef QL_STRIP_CG
#define QL_STRIP_CG 4
#endif
constexpr int kStripChunkGroups = QL_STRIP_CG;   // quantization groups staged per chunk
// a plan of 8-block strips more than this far off balance is re-planned with 4-block strips
constexpr double kStripSplitBalance = 1.06;

struct StripTask {
    int32_t linear, ct, nblk;  // blocks ct .. ct+nblk-1 of the linear
    int32_t chunks;            // chunks of kStripChunkGroups groups: all of K (ch0 = 0), or
    int32_t ch0;               // (strip_wide_kernel only) chunks ch0 .. ch0+chunks-1 of
    int32_t part, parts;       // K part `part` of `parts` > 1, whose sums (no bias) go to
                               // partial + poff[linear] + part * M * N, row stride N
};

struct StripArgs {
    const SeqLinear* lin;      // y_ll unused
    const StripTask* tasks;
    const int32_t* task_begin; // [G + 1]
    int32_t M, G, group;
    int32_t split;             // waves per block: 1 (strips of 8 blocks) or 2 (strips of 4)
    int32_t stream;            // 1: packed weights by streaming (nontemporal) loads
    int32_t wide;              // 1: strip_wide_kernel (no padding, M 5..16, streamed weights)
    int32_t ring;              // strip_wide_kernel: jobs in flight per wave, 2 or 4
    // strip_wide_kernel: each linear's activation digits, precomputed by wide_digits_kernel (one
    // workgroup per chunk, launched first) as images of the kernel's LDS chunk buffer: linear i's
    // chunk c at dimg + (dimg_base[i] + c) * strip_wide_image_bytes(M); dimg_lin[j] is the linear
    // of image j, dimg_count the images
    char* dimg;
    const int32_t* dimg_base;
    const int32_t* dimg_lin;
    int32_t dimg_count;
    // K parts (tasks with parts > 1): partial sums [part][M][N] of linear i at partial + poff[i]
    float* partial;
    const int64_t* poff;
    // strip_wide_kernel, K-part plans: non-null to stage each linear's activations from its fp32
    // x through in[i] (no digit images)
    const struct StripIn* in;
    // strip_wide_kernel with staged activations: workgroup w runs task flat[w] alone (G tasks),
    // whose record carries its linear's table entry, so no table read waits on another
    const struct StripFlat* flat;
};

// How a pass-by-pass linear's activations are formed while its strips stage them (x is the
// linear's fp32 SeqLinear::x, [M][K]): kind 0 x as is; 1 x * x2[k] (an RMSNorm's weight; the
// row's 1 / rms is applied by the part sums); 2 SiLU-mul, silu(x) * x2[m][k].
struct StripIn {
    const float* x2;           // kind 1: [K]; kind 2: [M][K]
    int32_t kind;
};
struct StripFlat {
    StripTask t;
    SeqLinear L;               // the task's linear
    StripIn in;
    int64_t poff;              // the linear's partial sums at StripArgs::partial + poff
};

// Sums the K parts of strip tasks in a fixed order, with bias and an optional residual, into y:
// one entry per linear.
// y[m][n] = rstd[m] * sum_p part_p[m][n] + bias[n] + res[m][n], rstd[m] = 1 / sqrt(sum_b
// in_ssq[m][b] / K + eps) when the linear's input is an RMSNorm (else 1).
struct PartSum {
    const float* part0;        // parts x [M][N], part p at part0 + p * M * N
    const float* bias;         // [N] or null
    const float* res;          // [M][N] or null
    float* y;                  // [M][N]
    float* ssq;                // null, or [M][N / 256]: sums of squares of y's rows by 256 columns
    const float* in_ssq;       // null, or the input's [M][K / 256] (its producer's ssq)
    float eps;
    int32_t parts, N, K;       // N % 256 == 0 when ssq is set, K % 256 == 0 when in_ssq is
    // SiLU-mul of two linears of one pass (gate: this entry, up: the b fields, same N and
    // parts), instead of a launch of its own: yb gets the up sums, yglu = silu(y) * yb (no ssq,
    // no in_ssq)
    const float* part0b;
    const float* bias_b;
    float* yb;
    float* yglu;               // null: an ordinary entry (set in every entry of a glu launch)
};
hipError_t launch_part_sums(const PartSum* entries_dev, int count, int M, int max_n, bool glu, hipStream_t stream);
struct PartSumArgs {
    PartSum e[kMaxBatch];
    int count, M;
};
hipError_t launch_part_sums_args(const PartSumArgs& a, int max_n, hipStream_t stream);

struct StripPlan {
    int grid = 0, strips = 0, split = 1;
    bool stream = false;       // the weights exceed what the MALL keeps between steps
    bool wide = false;         // strip_wide_kernel: streamed, split 1, M 5..16, no padding
    int ring = 2;              // strip_wide_kernel's jobs in flight per wave (4: K-part tasks)
    bool staged = false;       // K-part plans: activations staged through StripIn, no digit images
    uint64_t lds_bytes = 0;
    uint64_t total_units = 0, busiest_units = 0;   // block-groups: all, most on one workgroup
    std::vector<StripTask> tasks;
    std::vector<int32_t> task_begin;
};

bool strip_eligible(const std::vector<SeqSpec>& lin, int M);
int strip_grid(int cu_count, const std::vector<SeqSpec>& lin, int M);   // workgroups of a strip launch
constexpr uint64_t kStripMallBytes = 192ull << 20;   // weights that stay resident in the MALL
size_t strip_lds(int M, int group, int split);
// force_stream 1: plan as streamed from HBM whatever the launch's own bytes (a pass of a model
// whose weights do not stay in the MALL); -1: by the launch's bytes
void plan_strips(const std::vector<SeqSpec>& lin, int M, int grid, StripPlan* out, int force_stream = -1);
// The wide strips with every strip cut into K parts, for one pass of a pass-by-pass sequence:
// strips of 8 blocks, each cut into about grid / strips parts of whole 512-k chunks, dealt
// longest first. Empty when the linears are not wide-eligible at M.
void plan_strips_kparts(const std::vector<SeqSpec>& lin, int M, int grid, StripPlan* out);
hipError_t launch_strips(const StripArgs& a, size_t lds, hipStream_t stream);
// The strip launch without padding (ql_strip_wide.hip): every linear group 128, K a multiple of
// 4 groups, N a multiple of 512, weights streamed, strips of 8 blocks, M min_m..16 (the kernel
// runs any M from 1; below 5 the padded strip kernel is faster over all of K).
bool strip_wide_eligible(const std::vector<SeqSpec>& lin, int M, const StripPlan& p, int min_m = 5);
constexpr int kPassMinM = 2;   // pass-by-pass sequences: the K-part strips from this M
size_t strip_wide_lds(int M);
int strip_wide_per_cu(int M);          // workgroups per CU of the wide kernel at M rows
size_t strip_wide_image_bytes(int M);   // one chunk's digit image
hipError_t launch_strips_wide(const StripArgs& a, size_t lds, hipStream_t stream);

}  // namespace ql
