// C ABI of libqlinear.so (declared in include/qlinear.h): context, arenas, GPTQ descriptor
// validation, dispatch planning and kernel dispatch. No exceptions cross the ABI; every entry
// point returns a status and records a message for ql_last_error().
#include "../../include/qlinear.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "ql_internal.h"

struct ql_ctx {
    int device;
    hipStream_t stream;
    uint32_t* counters;   // split-K arrival counters; every launch leaves them at zero
    float* attn_ws;       // attention key-split partials (ql::kAttnWsBytes), used in stream order
    float* noalloc_scratch;  // this device's address of `scratch` (ql_linear_noalloc)
    hipEvent_t ev_start, ev_stop;
    bool capturing;
    int cu_count;
    uint64_t hbm_bytes;
    char name[256];
};

struct ql_arena {
    ql_ctx* ctx;          // owner; copies use its stream
    int device;           // release needs only this, so it stays valid after ql_destroy
    char* base;
    uint64_t size;
};

struct ql_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

// One launch of a pass-by-pass sequence: an RMSNorm into a buffer (e), a SiLU-mul into a buffer
// (o = silu(g) * u over n values), a pass's strips (s, lds), a pass's part sums (sums), or a
// pass's prefill GEMM (p) or chunked GEMM (gb).
struct SeqStep {
    enum Kind { kNorm, kGlu, kStrips, kPartSums, kPrefill, kGemm } kind;
    const ql::PartSum* sums = nullptr;   // kPartSums: the device table, count entries
    int count = 0, M = 0, max_n = 0;
    bool glu = false;                    // kPartSums: SiLU-mul entries (part_sum_glu_kernel)
    ql::ElemArgs e{};
    const float* g = nullptr;
    const float* u = nullptr;
    float* o = nullptr;
    long long n = 0;
    ql::StripArgs s{};
    uint64_t lds = 0;
    ql::PrefillArgs p{};
    ql::GemmBatch gb{};
};

struct ql_seq {
    int device;
    char* dev;              // one allocation: tables, exchange buffers, tickets, abort/error words
    ql::SeqArgs args;
    uint64_t lds;
    ql_seq_info info;
    bool strips;            // independent linears at M >= 2: the column-strip kernel (sargs)
    ql::StripArgs sargs;
    bool prefill;           // independent linears at M > 16: the prefill GEMM (pargs)
    ql::PrefillArgs pargs;
    bool passes = false;    // chained, streamed weights, M >= 2: one strip launch per pass (steps)
    std::vector<SeqStep> steps;
    std::vector<char*> bufs;   // the steps' device allocations (dev holds the input buffers)
};

// Split-K partial sums of ql_linear_noalloc. One copy per GPU, loaded with the code object, so
// that entry point allocates nothing. Host code never passes this name to a kernel: it is a
// host-side stand-in there; the device address comes from hipGetSymbolAddress (scratch_address).
static __device__ __align__(256) char scratch[QL_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(QL_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define QL_HIP(call)                                   \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

bool in_range(uint64_t off, uint64_t bytes, uint64_t size)
{
    return off <= size && bytes <= size - off;
}

uint64_t align256(uint64_t v) { return (v + 255) & ~(uint64_t)255; }

// Device address of `scratch` on `device` (which must be current), looked up once per device.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_addr[kMaxDevices];

hipError_t scratch_address(int device, float** out)
{
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_addr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_addr[device] = p;
    }
    *out = static_cast<float*>(g_scratch_addr[device]);
    return hipSuccess;
}

// planGemvSplit of the reference (src/model/qwen.ts:42-44, :61-74), reported in ql_plan.ref_split.
int ref_plan_gemv_split(int wg_n, int K)
{
    if (wg_n >= 256) return 1;
    const int cands[4] = {8, 16, 32, 64};
    int s = 1;
    for (int c : cands) {
        if (K % c == 0 && (K / c) % 2 == 0) {
            s = c;
            if (wg_n * c >= 256) break;
        }
    }
    return s;
}

int plan_impl(int M, int N, int K, int group, ql_plan* p)
{
    memset(p, 0, sizeof *p);
    if (group <= 0) return fail(QL_E_GROUP, "group must be positive (got %d)", group);
    if (M <= 0 || N <= 0 || K <= 0) return fail(QL_E_DIMS, "M, N, K must be positive (M=%d N=%d K=%d)", M, N, K);
    p->ref_split = ref_plan_gemv_split((N + 255) / 256, K);
    if (M <= ql::kGemvMaxM) {
        if (ql::gemv_fast_ok(M, N, K, group)) {
            const ql::GemvShape s = ql::gemv_shape(M, N, K, group);
            p->kind = QL_KIND_GEMV_MFMA;
            p->split = s.split;
            p->waves = s.waves;
            p->grid_x = s.strips * s.split;
            p->grid_y = 1;
            p->block = 256;
            p->scratch_bytes = ql::gemv_partial_bytes(M, N, s.split);
        } else {
            p->kind = QL_KIND_GEMV_SIMPLE;
            p->split = 1;
            p->waves = 4;
            p->grid_x = (N + 255) / 256;
            p->grid_y = (M + 7) / 8;
            p->block = 256;
        }
    } else if (ql::gemm_fast_ok(M, N, K, group)) {
        const ql::GemmShape s = ql::gemm_shape(M, N, K, group, ql::kPlanCUs);
        p->kind = QL_KIND_GEMM_MFMA;
        p->split = s.split;
        p->waves = 4;
        p->grid_x = s.tiles_n * s.tiles_m * s.split;
        p->grid_y = 1;
        p->block = 256;
        p->scratch_bytes = ql::gemm_partial_bytes(M, N, s.split);
    } else {
        p->kind = QL_KIND_GEMM_SIMPLE;
        p->split = 1;
        p->waves = 4;
        p->grid_x = (N + 255) / 256;
        p->grid_y = (M + 7) / 8;
        p->block = 256;
    }
    return QL_OK;
}

// validate_desc with scales of `scale_bytes` bytes per value (2: fp16 as stored, 4: f32)
int validate_desc_scales(const ql_gptq_desc* d, uint64_t arena_bytes, int scale_bytes)
{
    if (!d) return fail(QL_E_INVALID, "null descriptor");
    if (d->bits != 4) return fail(QL_E_BITS, "GPTQ: only 4-bit is supported, got bits=%d", d->bits);
    if (d->group <= 0) return fail(QL_E_GROUP, "GPTQ: group size must be positive");
    if (d->K <= 0 || d->N <= 0) return fail(QL_E_DIMS, "GPTQ: in/out features must be positive");
    uint64_t qw, qz, sc;
    ql_gptq_sizes(d->K, d->N, d->group, &qw, &qz, &sc);
    sc = sc / 2 * (uint64_t)scale_bytes;
    if (!in_range(d->qweight_off, qw, arena_bytes))
        return fail(QL_E_QWEIGHT_SHORT, "GPTQ: qweight needs %llu bytes at offset %llu, arena has %llu",
                    (unsigned long long)qw, (unsigned long long)d->qweight_off,
                    (unsigned long long)arena_bytes);
    if (!in_range(d->scales_off, sc, arena_bytes))
        return fail(QL_E_SCALES_SHORT, "GPTQ: scales need %llu bytes at offset %llu, arena has %llu",
                    (unsigned long long)sc, (unsigned long long)d->scales_off,
                    (unsigned long long)arena_bytes);
    if (d->qzeros_off != QL_NONE && !in_range(d->qzeros_off, qz, arena_bytes))
        return fail(QL_E_QZEROS_SHORT, "GPTQ: qzeros need %llu bytes at offset %llu, arena has %llu",
                    (unsigned long long)qz, (unsigned long long)d->qzeros_off,
                    (unsigned long long)arena_bytes);
    if (d->group % 8 != 0)
        return fail(QL_E_GROUP_PACK, "GPTQ: group size %d must be a multiple of 8", d->group);
    if (d->bias_off != QL_NONE && !in_range(d->bias_off, (uint64_t)d->N * 4, arena_bytes))
        return fail(QL_E_RANGE, "bias [N] f32 outside the weight arena");
    if (d->qweight_off % 4 || (d->qzeros_off != QL_NONE && d->qzeros_off % 4) ||
        d->scales_off % (uint64_t)scale_bytes || (d->bias_off != QL_NONE && d->bias_off % 4))
        return fail(QL_E_ALIGN, "misaligned GPTQ tensor offset (int32/f32: 4 B, f16: 2 B)");
    return QL_OK;
}

int validate_desc(const ql_gptq_desc* d, uint64_t arena_bytes) { return validate_desc_scales(d, arena_bytes, 2); }

int check_desc(const ql_gptq_desc* d, const ql_arena* w)
{
    if (!d || !w) return fail(QL_E_INVALID, "null descriptor or weight arena");
    return validate_desc(d, w->size);
}

ql::GemvLinear make_linear(const ql_gptq_desc* d, const ql_arena* w)
{
    ql::GemvLinear L{};
    L.qweight = reinterpret_cast<const uint32_t*>(w->base + d->qweight_off);
    L.qzeros = d->qzeros_off == QL_NONE ? nullptr
                                        : reinterpret_cast<const uint32_t*>(w->base + d->qzeros_off);
    L.scales = reinterpret_cast<const uint16_t*>(w->base + d->scales_off);
    L.bias = d->bias_off == QL_NONE ? nullptr : reinterpret_cast<const float*>(w->base + d->bias_off);
    L.N = d->N;
    L.K = d->K;
    L.group = d->group;
    L.split = 1;
    return L;
}

bool gemv_aligned(const ql_gptq_desc* d, uint64_t x_off, uint64_t y_off)
{
    return d->qweight_off % 16 == 0 && d->scales_off % 8 == 0 && x_off % 16 == 0 && y_off % 16 == 0 &&
           (d->bias_off == QL_NONE || d->bias_off % 16 == 0);
}

int check_io(const ql_gptq_desc* d, const ql_arena* act, uint64_t x_off, int x_dtype, int M,
             uint64_t y_off)
{
    if (x_dtype != QL_DTYPE_F32 && x_dtype != QL_DTYPE_F16)
        return fail(QL_E_INVALID, "x_dtype must be QL_DTYPE_F32 or QL_DTYPE_F16");
    if (M <= 0 || M > (1 << 20)) return fail(QL_E_INVALID, "M out of range (%d)", M);
    const uint64_t es = x_dtype == QL_DTYPE_F32 ? 4 : 2;
    if (!in_range(x_off, (uint64_t)M * d->K * es, act->size))
        return fail(QL_E_RANGE, "x [M,K] outside the activation arena");
    if (!in_range(y_off, (uint64_t)M * d->N * 4, act->size))
        return fail(QL_E_RANGE, "y [M,N] outside the activation arena");
    if (x_off % es || y_off % 4) return fail(QL_E_ALIGN, "misaligned x or y offset");
    return QL_OK;
}

uint64_t gptq_weight_bytes(const ql_gptq_desc* d)
{
    uint64_t qw, qz, sc;
    ql_gptq_sizes(d->K, d->N, d->group, &qw, &qz, &sc);
    return qw + sc + (d->qzeros_off == QL_NONE ? 0 : qz);
}

// Checks a sequence and finds each linear's producer: linear i reads linear j's output when
// x_offs[i] == y_offs[j] (j < i, N_j == K_i). Every other input is external and must not overlap
// any output of the sequence; outputs must not overlap each other.
int seq_resolve(int32_t n, const ql_gptq_desc* descs, int32_t M, const uint64_t* x_offs,
                int32_t x_dtype, const uint64_t* y_offs, uint64_t w_bytes, uint64_t act_bytes,
                std::vector<ql::SeqSpec>* specs, const ql_seq_fuse* fuse = nullptr)
{
    if (!descs || !x_offs || !y_offs) return fail(QL_E_INVALID, "null sequence arrays");
    if (n <= 0 || n > ql::kSeqMaxLinears)
        return fail(QL_E_INVALID, "a sequence holds 1..%d linears, got %d", ql::kSeqMaxLinears, n);
    if (M < 1 || M > ql::kSeqMaxRows) return fail(QL_E_INVALID, "sequences run M = 1..%d rows", ql::kSeqMaxRows);
    if (x_dtype != QL_DTYPE_F32 && x_dtype != QL_DTYPE_F16)
        return fail(QL_E_INVALID, "x_dtype must be QL_DTYPE_F32 or QL_DTYPE_F16");
    const bool prefill = M > ql::kGemvMaxM;
    const uint64_t es = x_dtype == QL_DTYPE_F32 ? 4 : 2;
    std::vector<std::pair<uint64_t, int>> ys(n);
    for (int i = 0; i < n; i++) {
        const ql_gptq_desc* d = &descs[i];
        int rc = validate_desc(d, w_bytes);
        if (rc) return rc;
        if (prefill && !ql::prefill_ok(M, d->N, d->K, d->group, x_dtype))
            return fail(QL_E_INVALID,
                        "linear %d: a prefill sequence (M > %d) needs N %% 4 == 0, groups a multiple of "
                        "128 dividing K, and M*N*4, M*K*(x bytes) and K*N/2 below 2^31 bytes", i,
                        ql::kGemvMaxM);
        if (!prefill && (!ql::gemv_fast_ok(M, d->N, d->K, d->group) || d->group != descs[0].group))
            return fail(QL_E_INVALID,
                        "linear %d: a sequence needs N %% 4 == 0, K %% group == 0 and one group size "
                        "(64, 128 or 256) for all linears", i);
        if (!gemv_aligned(d, x_offs[i], y_offs[i]))
            return fail(QL_E_ALIGN, "linear %d: qweight, x, y and bias offsets must be 16-byte aligned, "
                        "scales 8-byte", i);
        if (!in_range(y_offs[i], (uint64_t)M * d->N * 4, act_bytes))
            return fail(QL_E_RANGE, "linear %d: y [M,N] outside the activation arena", i);
        ys[i] = {y_offs[i], i};
    }
    std::sort(ys.begin(), ys.end());
    for (int k = 1; k < n; k++) {
        const int a = ys[k - 1].second;
        if (ys[k - 1].first + (uint64_t)M * descs[a].N * 4 > ys[k].first)
            return fail(QL_E_INVALID, "outputs of linears %d and %d overlap", a, ys[k].second);
    }
    specs->assign(n, ql::SeqSpec{});
    for (int i = 0; i < n; i++) {
        const ql_gptq_desc* d = &descs[i];
        ql::SeqSpec& s = (*specs)[i];
        s.N = d->N;
        s.K = d->K;
        s.group = d->group;
        s.src = -1;
        s.weight_bytes = gptq_weight_bytes(d);
        s.has_qzeros = d->qzeros_off != QL_NONE;
        s.has_bias = d->bias_off != QL_NONE;
        // producer: an output starting exactly at x
        auto it = std::lower_bound(ys.begin(), ys.end(), std::make_pair(x_offs[i], -1));
        if (it != ys.end() && it->first == x_offs[i]) {
            const int j = it->second;
            if (j >= i) return fail(QL_E_INVALID, "linear %d reads the output of linear %d, which runs later", i, j);
            if (descs[j].N != d->K)
                return fail(QL_E_INVALID, "linear %d reads linear %d's output, but K=%d != N=%d", i, j, d->K,
                            descs[j].N);
            if (prefill && x_dtype != QL_DTYPE_F32)
                return fail(QL_E_INVALID, "linear %d reads linear %d's output: a chained prefill sequence "
                            "(M > %d) takes fp32 x (x_dtype QL_DTYPE_F32)", i, j, ql::kGemvMaxM);
            s.src = j;
            continue;
        }
        const uint64_t xb = (uint64_t)M * d->K * es;
        if (!in_range(x_offs[i], xb, act_bytes))
            return fail(QL_E_RANGE, "linear %d: x [M,K] outside the activation arena", i);
        // an external input must not overlap any output
        if (it != ys.end() && it->first < x_offs[i] + xb)
            return fail(QL_E_INVALID, "linear %d: input overlaps the output of linear %d", i, it->second);
        if (it != ys.begin()) {
            const auto pv = *(it - 1);
            if (pv.first + (uint64_t)M * descs[pv.second].N * 4 > x_offs[i])
                return fail(QL_E_INVALID, "linear %d: input overlaps the output of linear %d", i, pv.second);
        }
    }
    if (!fuse) return QL_OK;
    // Fused operands: a producer when the offset starts another linear's output (earlier in the
    // sequence, of the operand's width), else an external f32 range that overlaps no output.
    auto operand = [&](int i, uint64_t off, int width, const char* what, int* src) -> int {
        auto it = std::lower_bound(ys.begin(), ys.end(), std::make_pair(off, -1));
        if (it != ys.end() && it->first == off) {
            const int j = it->second;
            if (j >= i) return fail(QL_E_INVALID, "linear %d: its %s is the output of linear %d, which runs later", i, what, j);
            if (descs[j].N != width)
                return fail(QL_E_INVALID, "linear %d: its %s is linear %d's output, width %d != %d", i, what, j,
                            descs[j].N, width);
            *src = j;
            return QL_OK;
        }
        const uint64_t b = (uint64_t)M * width * 4;
        if (off % 16) return fail(QL_E_ALIGN, "linear %d: the %s offset must be 16-byte aligned", i, what);
        if (!in_range(off, b, act_bytes)) return fail(QL_E_RANGE, "linear %d: the %s lies outside the activation arena", i, what);
        if (it != ys.end() && it->first < off + b)
            return fail(QL_E_INVALID, "linear %d: the %s overlaps the output of linear %d", i, what, it->second);
        if (it != ys.begin()) {
            const auto pv = *(it - 1);
            if (pv.first + (uint64_t)M * descs[pv.second].N * 4 > off)
                return fail(QL_E_INVALID, "linear %d: the %s overlaps the output of linear %d", i, what, pv.second);
        }
        *src = -1;
        return QL_OK;
    };
    bool any = false;
    for (int i = 0; i < n; i++) {
        const ql_seq_fuse& f = fuse[i];
        ql::SeqSpec& s = (*specs)[i];
        const int K = descs[i].K, N = descs[i].N;
        if (f.norm_w_off != QL_NONE && f.x2_off != QL_NONE)
            return fail(QL_E_INVALID, "linear %d: a fused RMSNorm and a fused SiLU-mul exclude each other", i);
        if (f.norm_w_off != QL_NONE) {
            if (f.norm_w_off % 16) return fail(QL_E_ALIGN, "linear %d: the norm weight offset must be 16-byte aligned", i);
            if (!in_range(f.norm_w_off, (uint64_t)K * 4, w_bytes))
                return fail(QL_E_RANGE, "linear %d: norm weight [K] outside the weight arena", i);
            if (!(f.norm_eps >= 0.f) || f.norm_eps > 1.f)
                return fail(QL_E_INVALID, "linear %d: norm_eps must be in [0, 1]", i);
            s.fuse |= ql::kFuseNorm;
        }
        if (f.x2_off != QL_NONE) {
            int rc = operand(i, f.x2_off, K, "SiLU-mul operand", &s.src2);
            if (rc) return rc;
            s.fuse |= ql::kFuseGlu;
        }
        if (f.res_off != QL_NONE) {
            int rc = operand(i, f.res_off, N, "residual", &s.res_src);
            if (rc) return rc;
            s.fuse |= ql::kFuseRes;
        }
        any = any || s.fuse != 0;
    }
    // the fused staging reads fp32 words (norm weight, x2 and residual products are fp32)
    if (any && x_dtype != QL_DTYPE_F32)
        return fail(QL_E_INVALID, "fused sequences take fp32 x (x_dtype QL_DTYPE_F32)");
    return QL_OK;
}

bool seq_fused(const std::vector<ql::SeqSpec>& specs)
{
    for (const ql::SeqSpec& s : specs)
        if (s.fuse) return true;
    return false;
}

// Device memory of a planned sequence, laid out in one allocation.
struct SeqLayout {
    std::vector<uint64_t> y_ll;
    std::vector<uint64_t> ssq;      // per linear, or UINT64_MAX when no consumer normalizes it
    uint64_t lin, fl, tasks, task_begin, first_tile, tickets, words, sym_zeros, sym_words, part, total;
};

SeqLayout seq_layout(const std::vector<ql::SeqSpec>& specs, const ql::SeqPlanOut& p, int M)
{
    SeqLayout L;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t o = off;
        off = align256(off + bytes);
        return o;
    };
    const int n = (int)specs.size();
    L.lin = take(sizeof(ql::SeqLinear) * n);
    L.fl = seq_fused(specs) ? take(sizeof(ql::SeqFuseLin) * n) : UINT64_MAX;
    L.tasks = take(sizeof(ql::SeqTask) * std::max<size_t>(1, p.tasks.size()));
    L.task_begin = take(sizeof(int32_t) * (p.grid + 1));
    L.first_tile = take(sizeof(int32_t) * p.grid);
    L.tickets = take(64 * ql::kSeqTickets);
    L.words = take(64);
    // stored-7 qzeros words (zero 8) for the largest linear without qzeros
    L.sym_words = 0;
    for (int i = 0; i < n; i++)
        if (!specs[i].has_qzeros)
            L.sym_words = std::max<uint64_t>(L.sym_words, (uint64_t)(specs[i].K / specs[i].group) *
                                                              ((specs[i].N + 7) / 8));
    L.sym_zeros = take(4 * std::max<uint64_t>(1, L.sym_words));
    for (int i = 0; i < n; i++) L.y_ll.push_back(take((uint64_t)M * specs[i].N * 8));
    // block sums of squares of every output that a fused RMSNorm reads
    L.ssq.assign(n, UINT64_MAX);
    for (int c = 0; c < n; c++)
        if ((specs[c].fuse & ql::kFuseNorm) && specs[c].src >= 0 && L.ssq[specs[c].src] == UINT64_MAX) {
            const int i = specs[c].src;
            L.ssq[i] = take((uint64_t)M * ((specs[i].N + ql::kSeqTileCols - 1) / ql::kSeqTileCols) * 8);
        }
    L.part = take(std::max<uint64_t>(1, p.slots) * (uint64_t)M * ql::kSeqTileCols * 8);
    L.total = off;
    return L;
}

// Device tables of a column-strip sequence: linears, strips, per-workgroup strip ranges, and
// stored-7 qzeros words for linears without qzeros.
struct StripLayout {
    uint64_t lin, tasks, task_begin, sym_zeros, sym_words, poff, in, flat;
    uint64_t dimg, dimg_base, dimg_lin;   // the wide kernel's digit images and their tables
    int32_t dimg_count;
    uint64_t total;
};

StripLayout strip_layout(const std::vector<ql::SeqSpec>& specs, const ql::StripPlan& p, int M)
{
    StripLayout L;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t o = off;
        off = align256(off + bytes);
        return o;
    };
    const int n = (int)specs.size();
    L.lin = take(sizeof(ql::SeqLinear) * n);
    L.tasks = take(sizeof(ql::StripTask) * std::max<size_t>(1, p.tasks.size()));
    L.task_begin = take(sizeof(int32_t) * (p.grid + 1));
    L.sym_words = 0;
    for (int i = 0; i < n; i++)
        if (!specs[i].has_qzeros)
            L.sym_words = std::max<uint64_t>(L.sym_words, (uint64_t)(specs[i].K / specs[i].group) *
                                                              ((specs[i].N + 7) / 8));
    L.sym_zeros = take(4 * std::max<uint64_t>(1, L.sym_words));
    L.poff = take(sizeof(int64_t) * std::max(1, n));
    L.in = take(sizeof(ql::StripIn) * std::max(1, n));
    L.flat = take(p.staged ? sizeof(ql::StripFlat) * std::max<size_t>(1, p.tasks.size()) : 16);
    // strip_wide_kernel: one digit image per 512-k chunk of every linear (unless the activations
    // are staged through StripIn)
    const bool images = p.wide && !p.staged;
    L.dimg_count = 0;
    if (images)
        for (int i = 0; i < n; i++) L.dimg_count += specs[i].K / 512;
    L.dimg_base = take(sizeof(int32_t) * std::max(1, n));
    L.dimg_lin = take(sizeof(int32_t) * std::max(1, L.dimg_count));
    L.dimg = take(images ? ql::strip_wide_image_bytes(M) * (uint64_t)L.dimg_count : 16);
    L.total = off;
    return L;
}

void fill_strip_info(const ql::StripPlan& p, int n, uint64_t scratch, ql_seq_info* info)
{
    info->linears = n;
    info->passes = 1;
    info->tiles = p.strips;
    info->reduces = 0;
    info->grid = p.grid;
    info->max_split = 1;
    info->lds_bytes = p.lds_bytes;
    info->device_bytes = scratch;
    info->total_units = p.total_units;
    info->busiest_units = p.busiest_units;
    info->kernel = QL_SEQ_STRIPS;
    info->split = p.split;
    info->stream = p.stream ? 1 : 0;
    info->variant = p.wide ? 1 : 0;
    info->launches = p.wide ? 2 : 1;     // the wide strips' digits launch first
}

void fill_seq_info(const ql::SeqPlanOut& p, int n, uint64_t scratch, ql_seq_info* info)
{
    info->linears = n;
    info->passes = p.passes;
    info->tiles = p.tiles;
    info->reduces = p.reduces;
    info->grid = p.grid;
    info->max_split = p.max_split;
    info->lds_bytes = p.lds_bytes;
    info->device_bytes = scratch;
    info->total_units = p.total_units;
    info->busiest_units = p.busiest_units;
    info->kernel = QL_SEQ_TILES;
    info->split = 1;
    info->stream = 0;
    info->variant = 0;
    info->launches = 1;
}

int set_device(ql_ctx* ctx)
{
    QL_HIP(hipSetDevice(ctx->device));
    return QL_OK;
}

// One strip launch's device tables over `lin` (x, y and weight pointers filled in, except the
// symmetric zeros of linears without qzeros, which point into the new allocation), planned on
// `grid` workgroups (force_stream as plan_strips). The caller owns *dev.
struct StripBuild {
    char* dev = nullptr;
    ql::StripArgs a{};
    ql::StripPlan plan;
    uint64_t lds = 0, bytes = 0;
};

int strip_build(const std::vector<ql::SeqSpec>& specs, std::vector<ql::SeqLinear> lin, int M, int group,
                const ql::StripPlan& plan, const std::vector<int64_t>* poff, float* partial,
                const std::vector<ql::StripIn>* ins, StripBuild* out)
{
    out->plan = plan;
    const ql::StripPlan& sp = out->plan;
    const StripLayout lay = strip_layout(specs, sp, M);
    const int n = (int)specs.size();
    char* dev = nullptr;
    QL_HIP(hipMalloc(&dev, lay.total));
    for (int i = 0; i < n; i++)
        if (!lin[i].qzeros) lin[i].qzeros = reinterpret_cast<const uint32_t*>(dev + lay.sym_zeros);
    hipError_t e = hipMemset(dev, 0, lay.total);
    if (e == hipSuccess && lay.sym_words)
        e = hipMemsetD32(reinterpret_cast<hipDeviceptr_t>(dev + lay.sym_zeros), 0x77777777, lay.sym_words);
    if (e == hipSuccess) e = hipMemcpy(dev + lay.lin, lin.data(), sizeof(ql::SeqLinear) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess && !sp.tasks.empty())
        e = hipMemcpy(dev + lay.tasks, sp.tasks.data(), sizeof(ql::StripTask) * sp.tasks.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(dev + lay.task_begin, sp.task_begin.data(), sizeof(int32_t) * sp.task_begin.size(),
                      hipMemcpyHostToDevice);
    if (e == hipSuccess && poff)
        e = hipMemcpy(dev + lay.poff, poff->data(), sizeof(int64_t) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess && sp.staged)
        e = ins ? hipMemcpy(dev + lay.in, ins->data(), sizeof(ql::StripIn) * n, hipMemcpyHostToDevice)
                : hipErrorInvalidValue;
    if (e == hipSuccess && sp.staged) {
        // one record per task, workgroup k running task k
        std::vector<ql::StripFlat> flat(sp.tasks.size());
        for (size_t k = 0; k < flat.size(); k++) {
            const int i = sp.tasks[k].linear;
            flat[k].t = sp.tasks[k];
            flat[k].L = lin[i];
            flat[k].in = (*ins)[i];
            flat[k].poff = poff ? (*poff)[i] : 0;
        }
        e = hipMemcpy(dev + lay.flat, flat.data(), sizeof(ql::StripFlat) * flat.size(), hipMemcpyHostToDevice);
    }
    if (e == hipSuccess && sp.wide && !sp.staged) {
        std::vector<int32_t> base(n), owner;
        for (int i = 0; i < n; i++) {
            base[i] = (int32_t)owner.size();
            owner.insert(owner.end(), specs[i].K / 512, i);
        }
        e = hipMemcpy(dev + lay.dimg_base, base.data(), sizeof(int32_t) * n, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy(dev + lay.dimg_lin, owner.data(), sizeof(int32_t) * owner.size(), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "ql_seq_create upload");
    }
    ql::StripArgs& a = out->a;
    a.lin = reinterpret_cast<const ql::SeqLinear*>(dev + lay.lin);
    a.tasks = reinterpret_cast<const ql::StripTask*>(dev + lay.tasks);
    a.task_begin = reinterpret_cast<const int32_t*>(dev + lay.task_begin);
    a.M = M;
    a.G = sp.grid;
    a.group = group;
    a.split = sp.split;
    a.stream = sp.stream ? 1 : 0;
    a.wide = sp.wide ? 1 : 0;
    a.ring = sp.ring;
    a.dimg = sp.wide && !sp.staged ? dev + lay.dimg : nullptr;
    a.in = sp.staged ? reinterpret_cast<const ql::StripIn*>(dev + lay.in) : nullptr;
    a.flat = sp.staged ? reinterpret_cast<const ql::StripFlat*>(dev + lay.flat) : nullptr;
    if (sp.staged) a.G = (int32_t)sp.tasks.size();
    a.dimg_base = reinterpret_cast<const int32_t*>(dev + lay.dimg_base);
    a.dimg_lin = reinterpret_cast<const int32_t*>(dev + lay.dimg_lin);
    a.dimg_count = lay.dimg_count;
    a.partial = partial;
    a.poff = reinterpret_cast<const int64_t*>(dev + lay.poff);
    out->dev = dev;
    out->lds = sp.lds_bytes;
    out->bytes = lay.total;
    return QL_OK;
}

// A linear's table entry with its weights bound (qzeros null when it has none).
ql::SeqLinear seq_linear_of(const ql_gptq_desc* d, const ql_arena* weights, const void* x, int32_t x_dtype, float* y)
{
    ql::SeqLinear L{};
    const ql::GemvLinear g = make_linear(d, weights);
    L.qweight = g.qweight;
    L.qzeros = g.qzeros;
    L.scales = g.scales;
    L.bias = g.bias;
    L.x = x;
    L.y = y;
    L.y_ll = nullptr;
    L.src = -1;
    L.N = d->N;
    L.K = d->K;
    L.x_dtype = x_dtype;
    return L;
}

// ql_seq_create for independent linears at M >= 2: one workgroup per CU walking its strips.
int strip_create(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights, ql_arena* act,
                 const uint64_t* x_offs, int32_t x_dtype, int32_t M, const uint64_t* y_offs,
                 const std::vector<ql::SeqSpec>& specs, ql_seq** out)
{
    std::vector<ql::SeqLinear> lin(n);
    for (int i = 0; i < n; i++)
        lin[i] = seq_linear_of(&descs[i], weights, act->base + x_offs[i], x_dtype,
                               reinterpret_cast<float*>(act->base + y_offs[i]));
    ql::StripPlan plan;
    ql::plan_strips(specs, M, ql::strip_grid(ctx->cu_count, specs, M), &plan);
    StripBuild b;
    int rc = strip_build(specs, lin, M, descs[0].group, plan, nullptr, nullptr, nullptr, &b);
    if (rc) return rc;
    ql_seq* q = new ql_seq();
    q->device = ctx->device;
    q->dev = b.dev;
    q->lds = b.lds;
    q->strips = true;
    q->sargs = b.a;
    fill_strip_info(b.plan, n, b.bytes, &q->info);
    *out = q;
    return QL_OK;
}

// ---- chained sequences of streamed weights at M = 2..16: one strip launch per pass ----
//
// The dependency-ordered tiles at M > 1 cut K into short segments (the digits of a tile's whole
// segment sit in LDS) and reduce them across workgroups. For a model whose weights stream from
// HBM anyway, each pass (the linears whose producers all ran in earlier passes) runs instead as
// the no-padding strip launch with every strip cut into K parts of whole 512-k chunks (about one
// task per workgroup), then one launch that adds each linear's parts in a fixed order with its
// bias and residual. The strips form each linear's activations as they stage them (an RMSNorm's
// weight, or SiLU-mul of two producers); an RMSNorm's 1/rms scales the summed parts, from row
// sums of squares that the producer's part sums write. Only an external input that is RMSNorm'd
// has a launch of its own, into a buffer of the sequence. Stream order replaces the device-side
// waits.
int seq_pass_of(const std::vector<ql::SeqSpec>& specs, std::vector<int>* pass)
{
    const int n = (int)specs.size();
    pass->assign(n, 0);
    int depth = 0;
    for (int i = 0; i < n; i++) {
        int p = 0;
        for (int j : {specs[i].src, specs[i].src2, specs[i].res_src})
            if (j >= 0) p = std::max(p, (*pass)[j] + 1);
        (*pass)[i] = p;
        depth = std::max(depth, p + 1);
    }
    return depth;
}

bool passes_ok(const std::vector<ql::SeqSpec>& specs, int M, int32_t x_dtype)
{
    const char* env = getenv("QL_SEQ_PASSES");
    if (env && atoi(env) == 0) return false;
    if (M < ql::kPassMinM || M > ql::kGemvMaxM || x_dtype != QL_DTYPE_F32) return false;
    uint64_t bytes = 0;
    bool chained = false;
    for (const ql::SeqSpec& s : specs) {
        bytes += s.weight_bytes;
        chained = chained || s.src >= 0 || s.src2 >= 0 || s.res_src >= 0;
        // the no-padding strips, at least two K parts per strip
        if (s.group != 128 || s.K % 512 || s.K < 1024 || s.N % 512) return false;
    }
    return chained && bytes > ql::kStripMallBytes;
}

// The pass-by-pass form's plan: per pass the linears and their strip plan; the external inputs
// that are RMSNorm'd (one launch each, into a buffer of the sequence); the producers whose output
// a consumer RMSNorms (their part sums also write its row sums of squares).
struct PassInput {
    uint64_t x_off, w_off;       // external x in the activation arena, norm weight in the weights'
    float eps;
    int K;
    uint64_t buf_off;            // in the sequence's buffers
};
struct PassesPlan {
    std::vector<int> pass;       // per linear
    int depth = 0;
    std::vector<PassInput> inputs;
    std::vector<int> input_of;   // per linear: index into inputs, or -1
    std::vector<int64_t> ssq_off;  // per linear: its output's row sums of squares (bytes), or -1
    std::vector<std::vector<int>> members;      // per pass: its linears
    std::vector<std::vector<ql::SeqSpec>> specs; // per pass: the strip launch's specs
    std::vector<ql::StripPlan> plans;
    std::vector<std::vector<int64_t>> poff;      // per pass: partial-sum offsets (floats) per member
    std::vector<std::vector<int>> parts;         // per pass: K parts per member
    // the sequence's buffers: normed inputs, then sums of squares, then the partial sums (which
    // serve every pass in turn)
    uint64_t input_bytes = 0, ssq_bytes = 0, partial_bytes = 0;
    uint64_t buffer_bytes() const { return input_bytes + ssq_bytes + partial_bytes; }
};

void plan_passes(const std::vector<ql::SeqSpec>& specs, const ql_seq_fuse* fuse, const uint64_t* x_offs,
                 int M, int grid, PassesPlan* P)
{
    const int n = (int)specs.size();
    P->depth = seq_pass_of(specs, &P->pass);
    P->input_of.assign(n, -1);
    P->ssq_off.assign(n, -1);
    for (int i = 0; i < n; i++) {
        const ql::SeqSpec& sp = specs[i];
        if (!(sp.fuse & ql::kFuseNorm)) continue;
        if (sp.src >= 0) {
            // the producer's part sums give the row sums of squares; the strips stage x * w
            int64_t& o = P->ssq_off[sp.src];
            if (o < 0) {
                o = (int64_t)P->ssq_bytes;
                P->ssq_bytes += align256((uint64_t)M * (sp.K / 256) * 4);
            }
            continue;
        }
        PassInput in{};
        in.x_off = x_offs[i];
        in.w_off = fuse[i].norm_w_off;
        in.eps = fuse[i].norm_eps;
        in.K = sp.K;
        int k = -1;
        for (int q = 0; q < (int)P->inputs.size() && k < 0; q++) {
            const PassInput& o = P->inputs[q];
            if (o.x_off == in.x_off && o.w_off == in.w_off && o.eps == in.eps && o.K == in.K) k = q;
        }
        if (k < 0) {
            in.buf_off = P->input_bytes;
            P->input_bytes += align256((uint64_t)M * in.K * 4);
            k = (int)P->inputs.size();
            P->inputs.push_back(in);
        }
        P->input_of[i] = k;
    }
    P->members.assign(P->depth, {});
    for (int i = 0; i < n; i++) P->members[P->pass[i]].push_back(i);
    P->specs.assign(P->depth, {});
    P->plans.assign(P->depth, ql::StripPlan{});
    P->poff.assign(P->depth, {});
    P->parts.assign(P->depth, {});
    for (int p = 0; p < P->depth; p++) {
        for (int i : P->members[p]) {
            ql::SeqSpec s = specs[i];
            s.src = s.src2 = s.res_src = -1;
            s.fuse = 0;
            P->specs[p].push_back(s);
        }
        ql::plan_strips_kparts(P->specs[p], M, grid, &P->plans[p]);
        if (!P->plans[p].wide) {
            P->depth = 0;  // a shape the K-part strips cannot run: the caller keeps the tiles
            return;
        }
        std::vector<int>& parts = P->parts[p];
        parts.assign(P->members[p].size(), 1);
        for (const ql::StripTask& t : P->plans[p].tasks) parts[t.linear] = std::max(parts[t.linear], t.parts);
        int64_t off = 0;
        for (size_t k = 0; k < parts.size(); k++) {
            P->poff[p].push_back(off);
            off += (int64_t)parts[k] * M * P->specs[p][k].N;
            off = (off + 63) & ~(int64_t)63;
        }
        P->partial_bytes = std::max<uint64_t>(P->partial_bytes, (uint64_t)off * 4);
    }
}

void fill_passes_info(const PassesPlan& P, int n, uint64_t bytes, int grid, ql_seq_info* info)
{
    *info = ql_seq_info{};
    info->linears = n;
    info->passes = P.depth;
    info->grid = grid;
    for (const ql::StripPlan& sp : P.plans) info->grid = std::max(info->grid, sp.grid);
    info->max_split = 1;
    info->device_bytes = bytes;
    info->kernel = QL_SEQ_STRIP_PASSES;
    info->split = 1;
    info->stream = 1;
    info->launches = 2 * P.depth + (int32_t)P.inputs.size();   // strips and part sums; external norms
    for (const ql::StripPlan& sp : P.plans) {
        info->tiles += sp.strips;
        info->lds_bytes = std::max<uint64_t>(info->lds_bytes, sp.lds_bytes);
        info->total_units += sp.total_units;
        info->busiest_units += sp.busiest_units;
        info->split = std::max(info->split, sp.split);
        info->variant = info->variant || sp.wide ? 1 : 0;
    }
}

int passes_create(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights, ql_arena* act,
                  const uint64_t* x_offs, int32_t x_dtype, int32_t M, const uint64_t* y_offs,
                  const ql_seq_fuse* fuse, const std::vector<ql::SeqSpec>& specs, ql_seq** out)
{
    PassesPlan P;
    const int grid = ctx->cu_count;
    plan_passes(specs, fuse, x_offs, M, grid, &P);
    if (P.depth < 1) return fail(QL_E_INVALID, "sequence shapes do not fit the K-part strips");
    ql_seq* q = new ql_seq();
    q->device = ctx->device;
    q->passes = true;
    auto cleanup = [&](int rc) {
        for (char* b : q->bufs) (void)hipFree(b);
        (void)hipFree(q->dev);
        delete q;
        return rc;
    };
    {
        hipError_t e = hipMalloc(&q->dev, P.buffer_bytes());
        if (e != hipSuccess) return cleanup(hip_fail(e, "ql_seq_create pass buffers"));
    }
    float* const ssq = reinterpret_cast<float*>(q->dev + P.input_bytes);
    float* const partial = reinterpret_cast<float*>(q->dev + P.input_bytes + P.ssq_bytes);
    auto ssq_of = [&](int j) {
        return P.ssq_off[j] < 0 ? nullptr : ssq + P.ssq_off[j] / 4;
    };
    auto y_ptr = [&](int j) { return reinterpret_cast<float*>(act->base + y_offs[j]); };
    auto ext_ptr = [&](int src, uint64_t off) -> const float* {
        return src >= 0 ? y_ptr(src) : reinterpret_cast<const float*>(act->base + off);
    };
    std::vector<bool> made(P.inputs.size(), false);
    uint64_t bytes = P.buffer_bytes();
    for (int p = 0; p < P.depth; p++) {
        // the pass's RMSNorm'd external inputs
        for (int i : P.members[p]) {
            const int k = P.input_of[i];
            if (k < 0 || made[k]) continue;
            made[k] = true;
            const PassInput& in = P.inputs[k];
            SeqStep st{};
            st.kind = SeqStep::kNorm;
            st.e.x = ext_ptr(-1, in.x_off);
            st.e.d = nullptr;
            st.e.w = reinterpret_cast<const float*>(weights->base + in.w_off);
            st.e.s = nullptr;
            st.e.y = reinterpret_cast<float*>(q->dev + in.buf_off);
            st.e.M = M;
            st.e.C = in.K;
            st.e.eps = in.eps;
            st.e.vec = in.K % 4 == 0 && reinterpret_cast<uintptr_t>(st.e.x) % 16 == 0 && in.w_off % 16 == 0;
            q->steps.push_back(st);
        }
        // the pass's strips (each linear's activations formed as they are staged)
        std::vector<ql::SeqLinear> lin;
        std::vector<ql::StripIn> ins;
        for (int i : P.members[p]) {
            const int k = P.input_of[i];
            const uint32_t fz = specs[i].fuse;
            ql::StripIn in{};
            const float* x;
            if (k >= 0) {
                x = reinterpret_cast<const float*>(q->dev + P.inputs[k].buf_off);
            } else if (fz & ql::kFuseGlu) {
                x = ext_ptr(specs[i].src, x_offs[i]);
                in.kind = 2;
                in.x2 = ext_ptr(specs[i].src2, fuse[i].x2_off);
            } else if (fz & ql::kFuseNorm) {
                x = y_ptr(specs[i].src);
                in.kind = 1;
                in.x2 = reinterpret_cast<const float*>(weights->base + fuse[i].norm_w_off);
            } else {
                x = ext_ptr(specs[i].src, x_offs[i]);
            }
            lin.push_back(seq_linear_of(&descs[i], weights, x, QL_DTYPE_F32, y_ptr(i)));
            ins.push_back(in);
        }
        StripBuild b;
        int rc = strip_build(P.specs[p], lin, M, descs[0].group, P.plans[p], &P.poff[p], partial, &ins, &b);
        if (rc) return cleanup(rc);
        q->bufs.push_back(b.dev);
        bytes += b.bytes;
        SeqStep st{};
        st.kind = SeqStep::kStrips;
        st.s = b.a;
        st.lds = b.lds;
        q->steps.push_back(st);
        // then its part sums: the row scale of an RMSNorm'd input, bias, residual, and the row
        // sums of squares of outputs that a consumer RMSNorms
        std::vector<ql::PartSum> sums;
        int max_n = 0;
        for (size_t k = 0; k < P.members[p].size(); k++) {
            const int i = P.members[p][k];
            ql::PartSum e{};
            e.part0 = partial + P.poff[p][k];
            e.bias = lin[k].bias;
            e.res = specs[i].fuse & ql::kFuseRes ? ext_ptr(specs[i].res_src, fuse[i].res_off) : nullptr;
            e.y = y_ptr(i);
            e.ssq = ssq_of(i);
            if (ins[k].kind == 1) {
                e.in_ssq = ssq_of(specs[i].src);
                e.eps = fuse[i].norm_eps;
            }
            e.parts = P.parts[p][k];
            e.N = descs[i].N;
            e.K = descs[i].K;
            max_n = std::max(max_n, e.N);
            sums.push_back(e);
        }
        char* tab = nullptr;
        hipError_t e = hipMalloc(&tab, sizeof(ql::PartSum) * sums.size());
        if (e == hipSuccess) q->bufs.push_back(tab);
        if (e == hipSuccess) e = hipMemcpy(tab, sums.data(), sizeof(ql::PartSum) * sums.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) return cleanup(hip_fail(e, "ql_seq_create part sums"));
        bytes += sizeof(ql::PartSum) * sums.size();
        SeqStep ps{};
        ps.kind = SeqStep::kPartSums;
        ps.sums = reinterpret_cast<const ql::PartSum*>(tab);
        ps.count = (int)sums.size();
        ps.M = M;
        ps.max_n = max_n;
        q->steps.push_back(ps);
    }
    fill_passes_info(P, n, bytes, grid, &q->info);
    *out = q;
    return QL_OK;
}

struct PrefillLayout {
    uint64_t lin, tasks, task_begin, total;
};

PrefillLayout prefill_layout(int n, const ql::PrefillPlan& p)
{
    PrefillLayout L;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t o = off;
        off = align256(off + bytes);
        return o;
    };
    L.lin = take(sizeof(ql::PrefillLinear) * n);
    L.tasks = take(sizeof(ql::PrefillTask) * std::max<size_t>(1, p.tasks.size()));
    L.task_begin = take(sizeof(int32_t) * (p.grid + 1));
    L.total = off;
    return L;
}

std::vector<ql::PrefillSpec> prefill_specs(const std::vector<ql::SeqSpec>& specs)
{
    std::vector<ql::PrefillSpec> v(specs.size());
    for (size_t i = 0; i < specs.size(); i++) v[i] = ql::PrefillSpec{specs[i].N, specs[i].K};
    return v;
}

void fill_prefill_info(const ql::PrefillPlan& p, int n, int M, const std::vector<ql::SeqSpec>& specs,
                       uint64_t bytes, ql_seq_info* info)
{
    memset(info, 0, sizeof *info);
    info->linears = n;
    info->passes = 1;
    info->tiles = (int32_t)p.tasks.size();
    info->grid = p.grid;
    info->max_split = 1;
    info->device_bytes = bytes;
    info->total_units = p.total_units;
    info->busiest_units = p.busiest_units;
    info->kernel = QL_SEQ_PREFILL;
    info->split = 1;
    info->launches = 1;
    (void)M;
    (void)specs;
}

// Independent linears at M > 16: one prefill GEMM launch over a planned task table.
int prefill_create(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights, ql_arena* act,
                   const uint64_t* x_offs, int32_t x_dtype, int32_t M, const uint64_t* y_offs,
                   const std::vector<ql::SeqSpec>& specs, ql_seq** out)
{
    ql::PrefillPlan pp;
    ql::plan_prefill(prefill_specs(specs), M, ctx->cu_count, &pp);
    const PrefillLayout lay = prefill_layout(n, pp);
    char* dev = nullptr;
    QL_HIP(hipMalloc(&dev, lay.total));
    std::vector<ql::PrefillLinear> lin(n);
    for (int i = 0; i < n; i++) {
        const ql_gptq_desc* d = &descs[i];
        const ql::GemvLinear g = make_linear(d, weights);
        ql::PrefillLinear& L = lin[i];
        L = ql::PrefillLinear{};
        L.qweight = g.qweight;
        L.qzeros = g.qzeros;
        L.scales = g.scales;
        L.bias = g.bias;
        L.x = act->base + x_offs[i];
        L.y = reinterpret_cast<float*>(act->base + y_offs[i]);
        L.N = d->N;
        L.K = d->K;
        L.group = d->group;
    }
    hipError_t e = hipMemcpy(dev + lay.lin, lin.data(), sizeof(ql::PrefillLinear) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess && !pp.tasks.empty())
        e = hipMemcpy(dev + lay.tasks, pp.tasks.data(), sizeof(ql::PrefillTask) * pp.tasks.size(),
                      hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(dev + lay.task_begin, pp.task_begin.data(), sizeof(int32_t) * pp.task_begin.size(),
                      hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "ql_seq_create upload");
    }
    ql_seq* q = new ql_seq();
    q->device = ctx->device;
    q->dev = dev;
    q->prefill = true;
    q->pargs = ql::PrefillArgs{};
    q->pargs.lin = reinterpret_cast<const ql::PrefillLinear*>(dev + lay.lin);
    q->pargs.tasks = reinterpret_cast<const ql::PrefillTask*>(dev + lay.tasks);
    q->pargs.task_begin = reinterpret_cast<const int32_t*>(dev + lay.task_begin);
    q->pargs.M = M;
    q->pargs.G = pp.grid;
    q->pargs.x_f32 = x_dtype == QL_DTYPE_F32 ? 1 : 0;
    fill_prefill_info(pp, n, M, specs, lay.total, &q->info);
    *out = q;
    return QL_OK;
}

int gemm_entry(const ql_gptq_desc* d, const ql_arena* weights, ql_arena* act, uint64_t x_off, int M,
               uint64_t y_off, float* partial, uint32_t* counters, int counter_base, int wg_begin,
               ql::GemmLinear* out, bool no_split);

// ---- chained prefill (M > 16): one GEMM launch per pass ----

// K segments from which a chained prefill pass's linear leaves its sums to a part-sum launch
#ifndef QL_GEMM_DEFER_SPLIT
#define QL_GEMM_DEFER_SPLIT 2
#endif
//
// The model's dependency order at M > 16 (runForward(M = T) calls each layer's linears in turn):
// each pass (the linears whose producers all ran in earlier passes) is one GEMM launch over the
// pass's linears, reading fp32 x (a producer's output or an external input) rounded to fp16 as it
// is staged, with a residual added at the store. A pass whose output tiles fill the device runs
// the prefill kernel; a smaller one the chunked GEMM with K split across workgroups (the choice
// ql_linear_batch makes), its partial sums and arrival counters in buffers of the sequence. A
// fused RMSNorm or SiLU-mul input runs first, one launch per distinct input, into a buffer of the
// sequence (fp32), as the reference runs its elementwise kernels between the GEMMs. Stream order
// orders the passes.
struct PrefillPasses {
    std::vector<int> pass;
    int depth = 0;
    struct Input {
        bool glu;
        int x_src, x2_src;
        uint64_t x_off, x2_off, w_off;
        float eps;
        int K;
        uint64_t buf_off;
    };
    std::vector<Input> inputs;
    std::vector<int> input_of;                   // per linear: index into inputs, or -1
    std::vector<std::vector<int>> members;       // per pass: its linears
    std::vector<ql::PrefillPlan> plans;
    std::vector<char> chunked;                   // per pass: the chunked split-K GEMM
    std::vector<int> chunk_tiles;                // per chunked pass: its output tiles
    std::vector<char> deferred;                  // per chunked pass: a part-sum launch follows it
    std::vector<char> folded;                    // per input: a SiLU-mul that its gate and up
                                                 // linears' part-sum launch writes
    uint64_t input_bytes = 0;
    uint64_t partial_bytes = 0;                  // the chunked passes' partial sums, reused in turn
    int counters = 0;                            // their arrival counters (self-clearing)
};

bool seq_chained(const std::vector<ql::SeqSpec>& specs)
{
    for (const ql::SeqSpec& s : specs)
        if (s.src >= 0 || s.src2 >= 0 || s.res_src >= 0 || s.fuse) return true;
    return false;
}

void plan_prefill_passes(const std::vector<ql::SeqSpec>& specs, const ql_seq_fuse* fuse, const uint64_t* x_offs,
                         int M, int grid, PrefillPasses* P)
{
    const int n = (int)specs.size();
    P->depth = seq_pass_of(specs, &P->pass);
    P->input_of.assign(n, -1);
    for (int i = 0; i < n; i++) {
        const ql::SeqSpec& sp = specs[i];
        if (!(sp.fuse & (ql::kFuseNorm | ql::kFuseGlu))) continue;
        PrefillPasses::Input in{};
        in.glu = (sp.fuse & ql::kFuseGlu) != 0;
        in.x_src = sp.src;
        in.x_off = sp.src >= 0 ? 0 : x_offs[i];
        in.x2_src = in.glu ? sp.src2 : -1;
        in.x2_off = in.glu && sp.src2 < 0 ? fuse[i].x2_off : 0;
        in.w_off = in.glu ? 0 : fuse[i].norm_w_off;
        in.eps = in.glu ? 0.f : fuse[i].norm_eps;
        in.K = sp.K;
        int k = -1;
        for (int q = 0; q < (int)P->inputs.size() && k < 0; q++) {
            const PrefillPasses::Input& o = P->inputs[q];
            if (o.glu == in.glu && o.x_src == in.x_src && o.x_off == in.x_off && o.x2_src == in.x2_src &&
                o.x2_off == in.x2_off && o.w_off == in.w_off && o.eps == in.eps && o.K == in.K)
                k = q;
        }
        if (k < 0) {
            in.buf_off = P->input_bytes;
            P->input_bytes += align256((uint64_t)M * in.K * 4);
            k = (int)P->inputs.size();
            P->inputs.push_back(in);
        }
        P->input_of[i] = k;
    }
    P->members.assign(P->depth, {});
    for (int i = 0; i < n; i++) P->members[P->pass[i]].push_back(i);
    P->plans.assign(P->depth, ql::PrefillPlan{});
    P->chunked.assign(P->depth, 0);
    P->chunk_tiles.assign(P->depth, 0);
    P->deferred.assign(P->depth, 0);
    for (int p = 0; p < P->depth; p++) {
        std::vector<ql::SeqSpec> sub;
        for (int i : P->members[p]) sub.push_back(specs[i]);
        // the chunked GEMM when the pass's prefill tiles fill less than the device and every
        // linear has the chunked form with one tile height (as ql_linear_batch chooses)
        int tiles = 0, bm = 0;
        bool chunk = (int)sub.size() <= ql::kMaxBatch;
        for (const ql::SeqSpec& sp : sub) {
            tiles += ql::prefill_tiles(M, sp.N);
            ql_plan pl;
            plan_impl(M, sp.N, sp.K, sp.group, &pl);
            const int b = ql::gemm_shape(M, sp.N, sp.K, sp.group, ql::kPlanCUs).bm;
            chunk = chunk && pl.kind == QL_KIND_GEMM_MFMA && (bm == 0 || b == bm);
            bm = b;
        }
        if (chunk && tiles < ql::kPrefillMinTiles) {
            P->chunked[p] = 1;
            uint64_t part = 0;
            int ctr = 0;
            for (const ql::SeqSpec& sp : sub) {
                const ql::GemmShape g = ql::gemm_shape(M, sp.N, sp.K, sp.group, ql::kPlanCUs);
                part += align256(ql::gemm_partial_bytes(M, sp.N, g.split));
                if (g.split > 1) ctr += g.tiles_n * g.tiles_m;
                P->chunk_tiles[p] += g.tiles_n * g.tiles_m;
            }
            P->partial_bytes = std::max(P->partial_bytes, part);
            P->counters = std::max(P->counters, ctr);
            // the split the pass's launch uses (none when its tiles alone fill the device)
            if (P->chunk_tiles[p] * 2 < ql::kPlanCUs)
                for (const ql::SeqSpec& sp : sub)
                    if (ql::gemm_shape(M, sp.N, sp.K, sp.group, ql::kPlanCUs).split >= QL_GEMM_DEFER_SPLIT) P->deferred[p] = 1;
        } else {
            ql::plan_prefill(prefill_specs(sub), M, grid, &P->plans[p]);
        }
    }
    // a SiLU-mul of a gate and an up linear whose sums one part-sum launch adds (one pass, both
    // split as many ways, one width, no residual on up) is written by that launch
    P->folded.assign(P->inputs.size(), 0);
    for (size_t k = 0; k < P->inputs.size(); k++) {
        const PrefillPasses::Input& in = P->inputs[k];
        const int g = in.x_src, u = in.x2_src;
        if (!in.glu || g < 0 || u < 0 || P->pass[g] != P->pass[u] || !P->deferred[P->pass[g]]) continue;
        const ql::SeqSpec& sg = specs[g];
        const ql::SeqSpec& su = specs[u];
        if (sg.N != in.K || su.N != in.K || (su.fuse & ql::kFuseRes)) continue;
        const int split = ql::gemm_shape(M, sg.N, sg.K, sg.group, ql::kPlanCUs).split;
        if (split < QL_GEMM_DEFER_SPLIT || ql::gemm_shape(M, su.N, su.K, su.group, ql::kPlanCUs).split != split)
            continue;
        P->folded[k] = 1;
    }
    // a part-sum launch adds SiLU-mul entries only or none: a pass with another linear that
    // leaves its sums to the launch keeps its SiLU-muls as launches
    for (int p = 0; p < P->depth; p++) {
        std::vector<char> in_fold(n, 0);
        for (size_t k = 0; k < P->inputs.size(); k++)
            if (P->folded[k] && P->pass[P->inputs[k].x_src] == p) in_fold[P->inputs[k].x_src] = in_fold[P->inputs[k].x2_src] = 1;
        bool all = true;
        for (int i : P->members[p])
            if (!in_fold[i] && ql::gemm_shape(M, specs[i].N, specs[i].K, specs[i].group, ql::kPlanCUs).split >= QL_GEMM_DEFER_SPLIT)
                all = false;
        if (!all)
            for (size_t k = 0; k < P->inputs.size(); k++)
                if (P->folded[k] && P->pass[P->inputs[k].x_src] == p) P->folded[k] = 0;
    }
}

void fill_prefill_passes_info(const PrefillPasses& P, int n, uint64_t bytes, ql_seq_info* info)
{
    memset(info, 0, sizeof *info);
    info->linears = n;
    info->passes = P.depth;
    info->max_split = 1;
    info->device_bytes = bytes;
    info->kernel = QL_SEQ_PREFILL_PASSES;
    info->split = 1;
    info->launches = P.depth + (int32_t)P.inputs.size();
    for (const ql::PrefillPlan& pp : P.plans) {
        info->tiles += (int32_t)pp.tasks.size();
        info->grid = std::max(info->grid, pp.grid);
        info->total_units += pp.total_units;
        info->busiest_units += pp.busiest_units;
    }
    for (int p = 0; p < P.depth; p++) {
        info->variant += P.chunked[p];              // passes on the chunked split-K GEMM
        info->tiles += P.chunk_tiles[p];
        info->launches += P.deferred[p];            // their part-sum launches
    }
    for (char f : P.folded) info->launches -= f;    // SiLU-muls written by those
}

uint64_t prefill_passes_bytes(const PrefillPasses& P)
{
    uint64_t bytes = P.input_bytes + P.partial_bytes + align256(4ull * P.counters);
    for (int p = 0; p < P.depth; p++)
        if (!P.chunked[p]) bytes += prefill_layout((int)P.members[p].size(), P.plans[p]).total;
    return bytes;
}

int prefill_passes_create(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights,
                          ql_arena* act, const uint64_t* x_offs, int32_t M, const uint64_t* y_offs,
                          const ql_seq_fuse* fuse, const std::vector<ql::SeqSpec>& specs, ql_seq** out)
{
    PrefillPasses P;
    plan_prefill_passes(specs, fuse, x_offs, M, ctx->cu_count, &P);
    ql_seq* q = new ql_seq();
    q->device = ctx->device;
    q->passes = true;
    auto cleanup = [&](int rc) {
        for (char* b : q->bufs) (void)hipFree(b);
        (void)hipFree(q->dev);
        delete q;
        return rc;
    };
    const uint64_t buf_bytes = P.input_bytes + P.partial_bytes + align256(4ull * P.counters);
    if (buf_bytes) {
        hipError_t e = hipMalloc(&q->dev, buf_bytes);
        if (e == hipSuccess && P.counters)
            e = hipMemset(q->dev + P.input_bytes + P.partial_bytes, 0, 4ull * P.counters);
        if (e != hipSuccess) return cleanup(hip_fail(e, "ql_seq_create pass buffers"));
    }
    float* const partial = reinterpret_cast<float*>(q->dev + P.input_bytes);
    uint32_t* const counters = reinterpret_cast<uint32_t*>(q->dev + P.input_bytes + P.partial_bytes);
    auto y_ptr = [&](int j) { return reinterpret_cast<float*>(act->base + y_offs[j]); };
    auto ext_ptr = [&](int src, uint64_t off) -> const float* {
        return src >= 0 ? y_ptr(src) : reinterpret_cast<const float*>(act->base + off);
    };
    std::vector<bool> made(P.inputs.size(), false);
    for (int p = 0; p < P.depth; p++) {
        // the pass's RMSNorm and SiLU-mul inputs
        for (int i : P.members[p]) {
            const int k = P.input_of[i];
            if (k < 0 || made[k]) continue;
            made[k] = true;
            const PrefillPasses::Input& in = P.inputs[k];
            float* buf = reinterpret_cast<float*>(q->dev + in.buf_off);
            SeqStep st{};
            if (in.glu) {
                st.kind = SeqStep::kGlu;
                st.g = ext_ptr(in.x_src, in.x_off);
                st.u = ext_ptr(in.x2_src, in.x2_off);
                st.o = buf;
                st.n = (long long)M * in.K;
            } else {
                st.kind = SeqStep::kNorm;
                st.e.x = ext_ptr(in.x_src, in.x_off);
                st.e.w = reinterpret_cast<const float*>(weights->base + in.w_off);
                st.e.y = buf;
                st.e.M = M;
                st.e.C = in.K;
                st.e.eps = in.eps;
                st.e.vec = in.K % 4 == 0 && reinterpret_cast<uintptr_t>(st.e.x) % 16 == 0 && in.w_off % 16 == 0;
            }
            q->steps.push_back(st);
        }
        const std::vector<int>& mem = P.members[p];
        auto x_of = [&](int i) {
            const int b = P.input_of[i];
            return b >= 0 ? static_cast<const void*>(q->dev + P.inputs[b].buf_off)
                          : static_cast<const void*>(ext_ptr(specs[i].src, x_offs[i]));
        };
        auto res_of = [&](int i) {
            return specs[i].fuse & ql::kFuseRes ? ext_ptr(specs[i].res_src, fuse[i].res_off) : nullptr;
        };
        if (P.chunked[p]) {
            // the pass's chunked GEMM: K split where its tiles leave CUs idle
            SeqStep st{};
            st.kind = SeqStep::kGemm;
            ql::GemmBatch& b = st.gb;
            b.count = (int)mem.size();
            b.M = M;
            b.x_dtype = QL_DTYPE_F32;
            long tiles = 0;
            for (int i : mem) {
                const ql::GemmShape g = ql::gemm_shape(M, descs[i].N, descs[i].K, descs[i].group, ql::kPlanCUs);
                tiles += (long)g.tiles_n * g.tiles_m;
                b.bm = g.bm;
            }
            const bool no_split = tiles * 2 >= ql::kPlanCUs;
            uint64_t off = 0;
            int wg = 0, counter_base = 0;
            for (size_t k = 0; k < mem.size(); k++) {
                const int i = mem[k];
                int rc = gemm_entry(&descs[i], weights, act, 0, M, y_offs[i],
                                    reinterpret_cast<float*>(reinterpret_cast<char*>(partial) + off), counters,
                                    counter_base, wg, &b.L[k], no_split);
                if (rc) return cleanup(rc);
                ql::GemmLinear& L = b.L[k];
                L.x = x_of(i);
                L.res = res_of(i);
                if (L.split > 1) counter_base += L.tiles_n * L.tiles_m;
                off += align256(ql::gemm_partial_bytes(M, descs[i].N, L.split));
                wg += L.tiles_n * L.tiles_m * L.split;
            }
            b.wg_total = wg;
            // linears split into many K segments leave their sums to a part-sum launch: one
            // workgroup per tile adding every segment alone takes a round trip per two segments
            std::vector<ql::PartSum> sums;
            std::vector<int> sum_of(n, -1);
            int max_n = 0;
            for (size_t k = 0; k < mem.size(); k++) {
                ql::GemmLinear& L = b.L[k];
                if (L.split < QL_GEMM_DEFER_SPLIT) continue;
                L.defer = 1;
                ql::PartSum e{};
                e.part0 = L.partial;
                e.bias = L.bias;
                e.res = L.res;
                e.y = L.y;
                e.parts = L.split;
                e.N = L.N;
                e.K = L.K;
                max_n = std::max(max_n, e.N);
                sum_of[mem[k]] = (int)sums.size();
                sums.push_back(e);
            }
            // SiLU-muls of this pass's gate and up linears: the gate's entry takes the up's
            std::vector<char> drop(sums.size(), 0);
            for (size_t k = 0; k < P.inputs.size(); k++) {
                if (!P.folded[k] || P.pass[P.inputs[k].x_src] != p) continue;
                const int ig = sum_of[P.inputs[k].x_src], iu = sum_of[P.inputs[k].x2_src];
                if (ig < 0 || iu < 0 || drop[ig] || drop[iu] || sums[ig].yglu || sums[ig].parts != sums[iu].parts ||
                    sums[ig].N != sums[iu].N || sums[iu].res)
                    return cleanup(fail(QL_E_STATE, "chained prefill: SiLU-mul fold plan mismatch"));
                ql::PartSum& e = sums[ig];
                e.part0b = sums[iu].part0;
                e.bias_b = sums[iu].bias;
                e.yb = sums[iu].y;
                e.yglu = reinterpret_cast<float*>(q->dev + P.inputs[k].buf_off);
                drop[iu] = 1;
                made[k] = true;
            }
            for (size_t k = sums.size(); k-- > 0;)
                if (drop[k]) sums.erase(sums.begin() + k);
            // a launch adds SiLU-mul entries only (their kernel) or none
            int glu = 0;
            for (const ql::PartSum& e : sums) glu += e.yglu != nullptr;
            if (glu != 0 && glu != (int)sums.size())
                return cleanup(fail(QL_E_STATE, "chained prefill: SiLU-mul fold plan mismatch"));
            q->steps.push_back(st);
            if (sums.empty() != !P.deferred[p]) return cleanup(fail(QL_E_STATE, "chained prefill: part-sum plan mismatch"));
            if (!sums.empty()) {
                char* tab = nullptr;
                hipError_t e = hipMalloc(&tab, sizeof(ql::PartSum) * sums.size());
                if (e == hipSuccess) q->bufs.push_back(tab);
                if (e == hipSuccess) e = hipMemcpy(tab, sums.data(), sizeof(ql::PartSum) * sums.size(), hipMemcpyHostToDevice);
                if (e != hipSuccess) return cleanup(hip_fail(e, "ql_seq_create part sums"));
                SeqStep ps{};
                ps.kind = SeqStep::kPartSums;
                ps.sums = reinterpret_cast<const ql::PartSum*>(tab);
                ps.count = (int)sums.size();
                ps.M = M;
                ps.max_n = max_n;
                ps.glu = glu != 0;
                q->steps.push_back(ps);
            }
            continue;
        }
        // the pass's prefill launch
        const ql::PrefillPlan& pp = P.plans[p];
        const PrefillLayout lay = prefill_layout((int)mem.size(), pp);
        char* dev = nullptr;
        hipError_t e = hipMalloc(&dev, lay.total);
        if (e != hipSuccess) return cleanup(hip_fail(e, "ql_seq_create prefill tables"));
        q->bufs.push_back(dev);
        std::vector<ql::PrefillLinear> lin(mem.size());
        for (size_t k = 0; k < mem.size(); k++) {
            const int i = mem[k];
            const ql::GemvLinear g = make_linear(&descs[i], weights);
            ql::PrefillLinear& L = lin[k];
            L = ql::PrefillLinear{};
            L.qweight = g.qweight;
            L.qzeros = g.qzeros;
            L.scales = g.scales;
            L.bias = g.bias;
            L.x = x_of(i);
            L.y = y_ptr(i);
            L.res = res_of(i);
            L.N = descs[i].N;
            L.K = descs[i].K;
            L.group = descs[i].group;
        }
        e = hipMemcpy(dev + lay.lin, lin.data(), sizeof(ql::PrefillLinear) * lin.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess && !pp.tasks.empty())
            e = hipMemcpy(dev + lay.tasks, pp.tasks.data(), sizeof(ql::PrefillTask) * pp.tasks.size(),
                          hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy(dev + lay.task_begin, pp.task_begin.data(), sizeof(int32_t) * pp.task_begin.size(),
                          hipMemcpyHostToDevice);
        if (e != hipSuccess) return cleanup(hip_fail(e, "ql_seq_create upload"));
        SeqStep st{};
        st.kind = SeqStep::kPrefill;
        st.p.lin = reinterpret_cast<const ql::PrefillLinear*>(dev + lay.lin);
        st.p.tasks = reinterpret_cast<const ql::PrefillTask*>(dev + lay.tasks);
        st.p.task_begin = reinterpret_cast<const int32_t*>(dev + lay.task_begin);
        st.p.M = M;
        st.p.G = pp.grid;
        st.p.x_f32 = 1;
        q->steps.push_back(st);
    }
    fill_prefill_passes_info(P, n, prefill_passes_bytes(P), &q->info);
    *out = q;
    return QL_OK;
}

}  // namespace

extern "C" {

const char* ql_last_error(void) { return g_err; }

int ql_create(int device, ql_ctx** out)
{
    if (!out) return fail(QL_E_INVALID, "null output pointer");
    *out = nullptr;
    int n = 0;
    QL_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(QL_E_INVALID, "device %d not present (%d devices)", device, n);
    QL_HIP(hipSetDevice(device));
    ql_ctx* c = new ql_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) { delete c; return hip_fail(e, "hipGetDeviceProperties"); }
    c->cu_count = prop.multiProcessorCount;
    c->hbm_bytes = prop.totalGlobalMem;
    snprintf(c->name, sizeof c->name, "%s (%s)", prop.name, prop.gcnArchName);
    if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete c;
        return hip_fail(e, "hipStreamCreateWithFlags");
    }
    if ((e = hipMalloc(&c->counters, sizeof(uint32_t) * ql::kCounterCapacity)) != hipSuccess ||
        (e = hipMemset(c->counters, 0, sizeof(uint32_t) * ql::kCounterCapacity)) != hipSuccess ||
        (e = hipMalloc(&c->attn_ws, ql::kAttnWsBytes)) != hipSuccess ||
        (e = scratch_address(device, &c->noalloc_scratch)) != hipSuccess ||
        (e = hipEventCreate(&c->ev_start)) != hipSuccess ||
        (e = hipEventCreate(&c->ev_stop)) != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return hip_fail(e, "ql_create");
    }
    *out = c;
    return QL_OK;
}

int ql_destroy(ql_ctx* ctx)
{
    if (!ctx) return fail(QL_E_INVALID, "null context");
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipEventDestroy(ctx->ev_start);
    (void)hipEventDestroy(ctx->ev_stop);
    (void)hipFree(ctx->counters);
    (void)hipFree(ctx->attn_ws);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return QL_OK;
}

int ql_device_info(ql_ctx* ctx, char* name, int name_len, int* cu_count, uint64_t* hbm_bytes)
{
    if (!ctx) return fail(QL_E_INVALID, "null context");
    if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", ctx->name);
    if (cu_count) *cu_count = ctx->cu_count;
    if (hbm_bytes) *hbm_bytes = ctx->hbm_bytes;
    return QL_OK;
}

int ql_arena_reserve(ql_ctx* ctx, uint64_t bytes, ql_arena** out)
{
    if (!ctx || !out) return fail(QL_E_INVALID, "null context or output pointer");
    if (bytes == 0) return fail(QL_E_INVALID, "arena size must be positive");
    if (ctx->capturing) return fail(QL_E_STATE, "cannot allocate during graph capture");
    *out = nullptr;
    int rc = set_device(ctx);
    if (rc) return rc;
    void* p = nullptr;
    QL_HIP(hipMalloc(&p, bytes));
    ql_arena* a = new ql_arena();
    a->ctx = ctx;
    a->device = ctx->device;
    a->base = static_cast<char*>(p);
    a->size = bytes;
    *out = a;
    return QL_OK;
}

int ql_arena_release(ql_arena* arena)
{
    if (!arena) return fail(QL_E_INVALID, "null arena");
    (void)hipSetDevice(arena->device);
    (void)hipFree(arena->base);   // hipFree waits for outstanding work on the device
    delete arena;
    return QL_OK;
}

uint64_t ql_arena_size(const ql_arena* arena) { return arena ? arena->size : 0; }

uint64_t ql_arena_device_ptr(const ql_arena* arena)
{
    return arena ? (uint64_t)(uintptr_t)arena->base : 0;
}

int ql_arena_write(ql_arena* arena, uint64_t off, const void* src, uint64_t bytes)
{
    if (!arena || (!src && bytes)) return fail(QL_E_INVALID, "null arena or source");
    if (arena->ctx->capturing) return fail(QL_E_STATE, "synchronous copy during graph capture");
    if (!in_range(off, bytes, arena->size)) return fail(QL_E_RANGE, "write outside the arena");
    if (!bytes) return QL_OK;
    int rc = set_device(arena->ctx);
    if (rc) return rc;
    QL_HIP(hipStreamSynchronize(arena->ctx->stream));
    QL_HIP(hipMemcpy(arena->base + off, src, bytes, hipMemcpyHostToDevice));
    return QL_OK;
}

int ql_arena_read(ql_arena* arena, uint64_t off, void* dst, uint64_t bytes)
{
    if (!arena || (!dst && bytes)) return fail(QL_E_INVALID, "null arena or destination");
    if (arena->ctx->capturing) return fail(QL_E_STATE, "synchronous copy during graph capture");
    if (!in_range(off, bytes, arena->size)) return fail(QL_E_RANGE, "read outside the arena");
    if (!bytes) return QL_OK;
    int rc = set_device(arena->ctx);
    if (rc) return rc;
    QL_HIP(hipStreamSynchronize(arena->ctx->stream));
    QL_HIP(hipMemcpy(dst, arena->base + off, bytes, hipMemcpyDeviceToHost));
    return QL_OK;
}

int ql_arena_copy(ql_ctx* ctx, ql_arena* dst, uint64_t dst_off, const ql_arena* src,
                  uint64_t src_off, uint64_t bytes)
{
    if (!ctx || !dst || !src) return fail(QL_E_INVALID, "null context or arena");
    if (!in_range(dst_off, bytes, dst->size) || !in_range(src_off, bytes, src->size))
        return fail(QL_E_RANGE, "copy outside an arena");
    if (!bytes) return QL_OK;
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipMemcpyAsync(dst->base + dst_off, src->base + src_off, bytes,
                          hipMemcpyDeviceToDevice, ctx->stream));
    return QL_OK;
}

int ql_gptq_sizes(int32_t K, int32_t N, int32_t group, uint64_t* qweight_bytes,
                  uint64_t* qzeros_bytes, uint64_t* scales_bytes)
{
    if (K <= 0 || N <= 0) return fail(QL_E_DIMS, "GPTQ: in/out features must be positive");
    if (group <= 0) return fail(QL_E_GROUP, "GPTQ: group size must be positive");
    const uint64_t pack_rows = ((uint64_t)K + 7) / 8;
    const uint64_t pack_cols = ((uint64_t)N + 7) / 8;
    const uint64_t groups = ((uint64_t)K + group - 1) / (uint64_t)group;
    if (qweight_bytes) *qweight_bytes = pack_rows * (uint64_t)N * 4;
    if (qzeros_bytes) *qzeros_bytes = groups * pack_cols * 4;
    if (scales_bytes) *scales_bytes = groups * (uint64_t)N * 2;
    return QL_OK;
}

int ql_gptq_validate(const ql_gptq_desc* desc, uint64_t arena_bytes)
{
    return validate_desc(desc, arena_bytes);
}

int ql_gptq_check(const ql_gptq_desc* desc, const ql_arena* weights)
{
    return check_desc(desc, weights);
}

int ql_unpack_f16(ql_ctx* ctx, const ql_gptq_desc* d, const ql_arena* weights, ql_arena* out,
                  uint64_t out_off)
{
    if (!ctx || !out) return fail(QL_E_INVALID, "null context or output arena");
    int rc = check_desc(d, weights);
    if (rc) return rc;
    if (!in_range(out_off, (uint64_t)d->N * d->K * 2, out->size))
        return fail(QL_E_RANGE, "fp16 [N,K] output outside the arena");
    if (out_off % 2) return fail(QL_E_ALIGN, "fp16 output offset must be 2-byte aligned");
    const int P = (d->K + 7) / 8;
    if (P > 65535) return fail(QL_E_INVALID, "K too large (%d)", d->K);
    if ((rc = set_device(ctx))) return rc;
    ql::UnpackArgs a{};
    a.qweight = reinterpret_cast<const uint32_t*>(weights->base + d->qweight_off);
    a.qzeros = d->qzeros_off == QL_NONE ? nullptr
                                        : reinterpret_cast<const uint32_t*>(weights->base + d->qzeros_off);
    a.scales = reinterpret_cast<const uint16_t*>(weights->base + d->scales_off);
    a.out = reinterpret_cast<uint16_t*>(out->base + out_off);
    a.N = d->N;
    a.K = d->K;
    a.group = d->group;
    const bool fast = d->N % 4 == 0 && d->K % 8 == 0 && d->qweight_off % 16 == 0 &&
                      d->scales_off % 8 == 0 && out_off % 16 == 0;
    QL_HIP(ql::launch_unpack(a, fast, ctx->stream));
    return QL_OK;
}

int ql_unpack_f16_batch(ql_ctx* ctx, int32_t count, const ql_gptq_desc* descs, const ql_arena* weights,
                        ql_arena* out, const uint64_t* out_offs)
{
    if (!ctx || !out || (count > 0 && (!descs || !out_offs)))
        return fail(QL_E_INVALID, "null context, output arena, descriptors or offsets");
    if (count < 0) return fail(QL_E_INVALID, "negative tensor count");
    // validate everything before any work is enqueued
    for (int i = 0; i < count; i++) {
        const ql_gptq_desc* d = &descs[i];
        int rc = check_desc(d, weights);
        if (rc) return rc;
        if (!in_range(out_offs[i], (uint64_t)d->N * d->K * 2, out->size))
            return fail(QL_E_RANGE, "tensor %d: fp16 [N,K] output outside the arena", i);
        if (out_offs[i] % 2) return fail(QL_E_ALIGN, "tensor %d: fp16 output offset must be 2-byte aligned", i);
        if ((d->K + 7) / 8 > 65535) return fail(QL_E_INVALID, "tensor %d: K too large (%d)", i, d->K);
    }
    int rc = set_device(ctx);
    if (rc) return rc;
    ql::UnpackBatch b{};
    auto flush = [&]() -> hipError_t {
        hipError_t e = b.count ? ql::launch_unpack_batch(b, ctx->stream) : hipSuccess;
        b.count = 0;
        b.tiles = 0;
        return e;
    };
    for (int i = 0; i < count; i++) {
        const ql_gptq_desc* d = &descs[i];
        const bool fast = d->N % 4 == 0 && d->K % 8 == 0 && d->qweight_off % 16 == 0 &&
                          d->scales_off % 8 == 0 && out_offs[i] % 16 == 0;
        if (!fast) {
            // the generic kernel, in order with the batch launches around it
            if ((rc = ql_unpack_f16(ctx, d, weights, out, out_offs[i]))) return rc;
            continue;
        }
        const int tiles = ql::unpack_tiles(d->N, d->K);
        if (b.count == ql::kUnpackBatch || (int64_t)b.tiles + tiles > INT32_MAX) QL_HIP(flush());
        ql::UnpackItem& it = b.it[b.count++];
        it.qweight = reinterpret_cast<const uint32_t*>(weights->base + d->qweight_off);
        it.qzeros = d->qzeros_off == QL_NONE ? nullptr
                                             : reinterpret_cast<const uint32_t*>(weights->base + d->qzeros_off);
        it.scales = reinterpret_cast<const uint16_t*>(weights->base + d->scales_off);
        it.out = reinterpret_cast<uint16_t*>(out->base + out_offs[i]);
        it.N = d->N;
        it.K = d->K;
        it.group = d->group;
        it.tile_begin = b.tiles;
        b.tiles += tiles;
    }
    QL_HIP(flush());
    return QL_OK;
}

int ql_unpack_f32(ql_ctx* ctx, const ql_gptq_desc* d, const ql_arena* weights, ql_arena* out,
                  uint64_t out_off)
{
    return ql_unpack_f32_ex(ctx, d, weights, QL_DTYPE_F16, out, out_off);
}

int ql_unpack_f32_ex(ql_ctx* ctx, const ql_gptq_desc* d, const ql_arena* weights, int32_t scales_dtype,
                     ql_arena* out, uint64_t out_off)
{
    if (!ctx || !out) return fail(QL_E_INVALID, "null context or output arena");
    if (scales_dtype != QL_DTYPE_F16 && scales_dtype != QL_DTYPE_F32)
        return fail(QL_E_INVALID, "scales dtype must be QL_DTYPE_F16 or QL_DTYPE_F32");
    if (!weights) return fail(QL_E_INVALID, "null descriptor or weight arena");
    int rc = validate_desc_scales(d, weights->size, scales_dtype == QL_DTYPE_F32 ? 4 : 2);
    if (rc) return rc;
    if (!in_range(out_off, (uint64_t)d->N * d->K * 4, out->size))
        return fail(QL_E_RANGE, "fp32 [N,K] output outside the arena");
    if (out_off % 16) return fail(QL_E_ALIGN, "fp32 output offset must be 16-byte aligned");
    if ((d->K + 7) / 8 > 65535) return fail(QL_E_INVALID, "K too large (%d)", d->K);
    if ((rc = set_device(ctx))) return rc;
    ql::UnpackArgs a{};
    a.qweight = reinterpret_cast<const uint32_t*>(weights->base + d->qweight_off);
    a.qzeros = d->qzeros_off == QL_NONE ? nullptr
                                        : reinterpret_cast<const uint32_t*>(weights->base + d->qzeros_off);
    a.scales = reinterpret_cast<const uint16_t*>(weights->base + d->scales_off);
    a.out = out->base + out_off;
    a.N = d->N;
    a.K = d->K;
    a.group = d->group;
    a.scales_f32 = scales_dtype == QL_DTYPE_F32 ? reinterpret_cast<const float*>(weights->base + d->scales_off)
                                                : nullptr;
    QL_HIP(ql::launch_unpack_f32(a, ctx->stream));
    return QL_OK;
}

namespace {

// One GEMM batch entry: pointers, shape, partial sums at scratch_off and arrival counters from
// counter_base (both used only when the linear splits K).
int gemm_entry(const ql_gptq_desc* d, const ql_arena* weights, ql_arena* act, uint64_t x_off, int M,
               uint64_t y_off, float* partial, uint32_t* counters, int counter_base, int wg_begin,
               ql::GemmLinear* out, bool no_split)
{
    ql::GemmShape s = ql::gemm_shape(M, d->N, d->K, d->group, ql::kPlanCUs);
    if (no_split) s.split = 1;
    const ql::GemvLinear g = make_linear(d, weights);
    ql::GemmLinear& L = *out;
    L.defer = 0;
    L.qweight = g.qweight;
    L.qzeros = g.qzeros;
    L.scales = g.scales;
    L.bias = g.bias;
    L.x = act->base + x_off;
    L.y = reinterpret_cast<float*>(act->base + y_off);
    L.partial = partial;
    L.counters = counters + counter_base;
    L.res = nullptr;
    L.N = d->N;
    L.K = d->K;
    L.group = d->group;
    L.split = s.split;
    L.tiles_n = s.tiles_n;
    L.tiles_m = s.tiles_m;
    L.wg_begin = wg_begin;
    if (s.split > 1 && counter_base + s.tiles_n * s.tiles_m > ql::kCounterCapacity)
        return fail(QL_E_INVALID, "too many GEMM tiles for the split-K counters");
    return QL_OK;
}

// The batch's GEMM launch, then, for its linears split along K, one part-sum launch that adds
// their segments (ascending order within each lane, bias, residual) where the last workgroup of
// each tile would add them alone (a round trip per two segments).
hipError_t launch_gemm_parts(ql::GemmBatch& b, hipStream_t stream)
{
    ql::PartSumArgs ps{};
    ps.M = b.M;
    int max_n = 0;
    for (int i = 0; i < b.count; i++) {
        ql::GemmLinear& L = b.L[i];
        if (L.split < QL_GEMM_DEFER_SPLIT) continue;
        L.defer = 1;
        ql::PartSum& e = ps.e[ps.count++];
        e = ql::PartSum{};
        e.part0 = L.partial;
        e.bias = L.bias;
        e.res = L.res;
        e.y = L.y;
        e.parts = L.split;
        e.N = L.N;
        e.K = L.K;
        max_n = std::max(max_n, L.N);
    }
    hipError_t e = ql::launch_gemm_batch(b, stream);
    if (e == hipSuccess) e = ql::launch_part_sums_args(ps, max_n, stream);
    return e;
}

}  // namespace

namespace {

// A batch of linears (x offsets, dtype and alignment already checked) as one prefill GEMM launch,
// when every linear qualifies, all share K (the batch form deals tiles round robin, which balances
// only equal tiles) and the tiles fill at least half the device (fewer tiles run faster split
// along K by the chunked GEMM). Returns false when it does not apply.
bool prefill_batch(ql_ctx* ctx, int count, const ql_gptq_desc* descs, const ql_arena* weights, ql_arena* act,
                   const uint64_t* x_offs, int x_dtype, int M, const uint64_t* y_offs, int* rc)
{
    int tiles = 0;
    for (int i = 0; i < count; i++) {
        if (!ql::prefill_ok(M, descs[i].N, descs[i].K, descs[i].group, x_dtype) ||
            !gemv_aligned(&descs[i], x_offs[i], y_offs[i]) || descs[i].K != descs[0].K)
            return false;
        tiles += ql::prefill_tiles(M, descs[i].N);
    }
    if (tiles < ql::kPrefillMinTiles) return false;
    ql::PrefillArgs a{};
    a.count = count;
    a.M = M;
    int begin = 0;
    for (int i = 0; i < count; i++) {
        const ql::GemvLinear g = make_linear(&descs[i], weights);
        ql::PrefillLinear& L = a.L[i];
        L.qweight = g.qweight;
        L.qzeros = g.qzeros;
        L.scales = g.scales;
        L.bias = g.bias;
        L.x = act->base + x_offs[i];
        L.y = reinterpret_cast<float*>(act->base + y_offs[i]);
        L.N = descs[i].N;
        L.K = descs[i].K;
        L.group = descs[i].group;
        L.tiles_m = (M + ql::kPrefillRows - 1) / ql::kPrefillRows;
        L.tile_begin = begin;
        begin += ql::prefill_tiles(M, descs[i].N);
    }
    a.total_tiles = begin;
    a.G = std::min(begin, ctx->cu_count);
    a.x_f32 = x_dtype == QL_DTYPE_F32 ? 1 : 0;
    if ((*rc = set_device(ctx))) return true;
    const hipError_t e = ql::launch_prefill(a, false, ctx->stream);
    *rc = e == hipSuccess ? QL_OK : hip_fail(e, "launch_prefill");
    return true;
}

}  // namespace

int ql_plan_linear(int32_t M, int32_t N, int32_t K, int32_t group, ql_plan* out)
{
    if (!out) return fail(QL_E_INVALID, "null plan pointer");
    return plan_impl(M, N, K, group, out);
}

namespace {

// ql_linear after its scratch has been resolved: `partial` holds the plan's scratch_bytes (split-K
// partial sums; unused when the plan does not split K).
int linear_impl(ql_ctx* ctx, const ql_gptq_desc* d, const ql_arena* weights, ql_arena* act,
                uint64_t x_off, int32_t x_dtype, int32_t M, uint64_t y_off, const ql_plan& p,
                float* partial)
{
    int rc;
    if ((rc = set_device(ctx))) return rc;
    ql::GemvLinear L = make_linear(d, weights);
    L.x = act->base + x_off;
    L.y = reinterpret_cast<float*>(act->base + y_off);

    if (p.kind == QL_KIND_GEMV_MFMA && gemv_aligned(d, x_off, y_off)) {
        const ql::GemvShape s = ql::gemv_shape(M, d->N, d->K, d->group);
        ql::GemvBatch b{};
        L.split = s.split;
        L.strips = s.strips;
        L.wg_begin = 0;
        L.partial = partial;
        L.counters = ctx->counters;
        if (s.strips > ql::kCounterCapacity) return fail(QL_E_INVALID, "N too large (%d)", d->N);
        b.L[0] = L;
        b.count = 1;
        b.M = M;
        b.x_dtype = x_dtype;
        b.wg_total = s.strips * s.split;
        QL_HIP(ql::launch_gemv_batch(b, ctx->stream));
        return QL_OK;
    }
    if (p.kind == QL_KIND_GEMV_MFMA || p.kind == QL_KIND_GEMV_SIMPLE) {
        QL_HIP(ql::launch_gemv_simple(L, M, x_dtype, ctx->stream));
        return QL_OK;
    }
    if (p.kind == QL_KIND_GEMM_MFMA && gemv_aligned(d, x_off, y_off)) {
        if (prefill_batch(ctx, 1, d, weights, act, &x_off, x_dtype, M, &y_off, &rc)) return rc;
        ql::GemmBatch b{};
        int rc2 = gemm_entry(d, weights, act, x_off, M, y_off, partial, ctx->counters, 0, 0, &b.L[0], false);
        if (rc2) return rc2;
        b.count = 1;
        b.M = M;
        b.x_dtype = x_dtype;
        b.bm = ql::gemm_shape(M, d->N, d->K, d->group, ql::kPlanCUs).bm;
        b.wg_total = b.L[0].tiles_n * b.L[0].tiles_m * b.L[0].split;
        QL_HIP(launch_gemm_parts(b, ctx->stream));
        return QL_OK;
    }
    ql::GemmArgs g;
    g.qweight = L.qweight;
    g.qzeros = L.qzeros;
    g.scales = L.scales;
    g.bias = L.bias;
    g.x = L.x;
    g.y = L.y;
    g.M = M;
    g.N = d->N;
    g.K = d->K;
    g.group = d->group;
    g.x_dtype = x_dtype;
    QL_HIP(ql::launch_gemm_simple(g, ctx->stream));
    return QL_OK;
}

// true when the plan's MFMA path runs and reads split-K scratch
bool uses_scratch(const ql_gptq_desc* d, const ql_plan& p, uint64_t x_off, uint64_t y_off)
{
    return (p.kind == QL_KIND_GEMV_MFMA || p.kind == QL_KIND_GEMM_MFMA) && gemv_aligned(d, x_off, y_off);
}

}  // namespace

int ql_linear(ql_ctx* ctx, const ql_gptq_desc* d, const ql_arena* weights, ql_arena* act,
              uint64_t x_off, int32_t x_dtype, int32_t M, uint64_t y_off, uint64_t scratch_off)
{
    if (!ctx || !act) return fail(QL_E_INVALID, "null context or activation arena");
    int rc = check_desc(d, weights);
    if (rc) return rc;
    if ((rc = check_io(d, act, x_off, x_dtype, M, y_off))) return rc;
    ql_plan p;
    if ((rc = plan_impl(M, d->N, d->K, d->group, &p))) return rc;
    if (uses_scratch(d, p, x_off, y_off)) {
        if (!in_range(scratch_off, p.scratch_bytes, act->size))
            return fail(QL_E_RANGE, "scratch (%llu bytes) outside the activation arena",
                        (unsigned long long)p.scratch_bytes);
        if (scratch_off % 16) return fail(QL_E_ALIGN, "scratch offset must be 16-byte aligned");
    }
    return linear_impl(ctx, d, weights, act, x_off, x_dtype, M, y_off, p,
                       reinterpret_cast<float*>(act->base + scratch_off));
}

int ql_linear_noalloc(ql_ctx* ctx, const ql_gptq_desc* d, const ql_arena* weights, ql_arena* act,
                      uint64_t x_off, int32_t x_dtype, int32_t M, uint64_t y_off)
{
    if (!ctx || !act) return fail(QL_E_INVALID, "null context or activation arena");
    int rc = check_desc(d, weights);
    if (rc) return rc;
    if ((rc = check_io(d, act, x_off, x_dtype, M, y_off))) return rc;
    ql_plan p;
    if ((rc = plan_impl(M, d->N, d->K, d->group, &p))) return rc;
    if (uses_scratch(d, p, x_off, y_off) && p.scratch_bytes > QL_NOALLOC_SCRATCH_BYTES)
        return fail(QL_E_RANGE,
                    "ql_linear_noalloc: this plan needs %llu bytes of split-K scratch, more than the "
                    "%u-byte static scratch (use ql_linear with a scratch offset)",
                    (unsigned long long)p.scratch_bytes, (unsigned)QL_NOALLOC_SCRATCH_BYTES);
    if (!ctx->noalloc_scratch) return fail(QL_E_STATE, "static scratch address not resolved");
    return linear_impl(ctx, d, weights, act, x_off, x_dtype, M, y_off, p, ctx->noalloc_scratch);
}

int ql_gemv_f16w(ql_ctx* ctx, const ql_arena* weights, uint64_t w_off, uint64_t bias_off,
                 ql_arena* act, uint64_t x_off, int32_t M, int32_t N, int32_t K, uint64_t y_off)
{
    if (!ctx || !weights || !act) return fail(QL_E_INVALID, "null context or arena");
    if (M < 1 || M > 65535) return fail(QL_E_INVALID, "M must be 1..65535 (got %d)", M);
    if (N <= 0 || K <= 0) return fail(QL_E_DIMS, "N and K must be positive");
    if (K % 8) return fail(QL_E_INVALID, "K must be a multiple of 8 (got %d)", K);
    if (!in_range(w_off, (uint64_t)N * K * 2, weights->size)) return fail(QL_E_RANGE, "fp16 weights [N,K] outside the arena");
    if (bias_off != QL_NONE && !in_range(bias_off, (uint64_t)N * 4, weights->size))
        return fail(QL_E_RANGE, "bias [N] outside the weight arena");
    if (!in_range(x_off, (uint64_t)M * K * 4, act->size)) return fail(QL_E_RANGE, "x [M,K] outside the activation arena");
    if (!in_range(y_off, (uint64_t)M * N * 4, act->size)) return fail(QL_E_RANGE, "y [M,N] outside the activation arena");
    if (w_off % 16 || x_off % 16 || y_off % 16 || (bias_off != QL_NONE && bias_off % 4))
        return fail(QL_E_ALIGN, "w, x and y offsets must be 16-byte aligned (bias 4-byte)");
    const uint64_t xa = x_off, xb = x_off + (uint64_t)M * K * 4, ya = y_off, yb = y_off + (uint64_t)M * N * 4;
    if (xa < yb && ya < xb) return fail(QL_E_INVALID, "x and y overlap");
    int rc = set_device(ctx);
    if (rc) return rc;
    ql::F16wArgs a;
    a.w = reinterpret_cast<const uint16_t*>(weights->base + w_off);
    a.bias = bias_off == QL_NONE ? nullptr : reinterpret_cast<const float*>(weights->base + bias_off);
    a.x = reinterpret_cast<const float*>(act->base + x_off);
    a.y = reinterpret_cast<float*>(act->base + y_off);
    a.M = M;
    a.N = N;
    a.K = K;
    QL_HIP(ql::launch_gemv_f16w(a, ql::gemv_f16w_fast_ok(M, N, K), ctx->cu_count, ctx->stream));
    return QL_OK;
}

int ql_embed_f16(ql_ctx* ctx, const ql_arena* weights, uint64_t embed_off, int32_t vocab, int32_t D,
                 ql_arena* act, uint64_t tokens_off, int32_t rows, uint64_t out_off)
{
    if (!ctx || !weights || !act) return fail(QL_E_INVALID, "null context or arena");
    if (rows < 1 || rows > 65535) return fail(QL_E_INVALID, "rows must be 1..65535 (got %d)", rows);
    if (vocab < 1 || D < 1 || D > (1 << 24)) return fail(QL_E_DIMS, "vocab and D must be positive (D <= 2^24)");
    if (!in_range(embed_off, (uint64_t)vocab * D * 2, weights->size))
        return fail(QL_E_RANGE, "fp16 embedding [vocab, D] outside the weight arena");
    if (!in_range(tokens_off, (uint64_t)rows * 4, act->size)) return fail(QL_E_RANGE, "tokens [rows] outside the activation arena");
    if (!in_range(out_off, (uint64_t)rows * D * 4, act->size)) return fail(QL_E_RANGE, "out [rows, D] outside the activation arena");
    if (embed_off % 2 || tokens_off % 4 || out_off % 4) return fail(QL_E_ALIGN, "embed 2-byte, tokens and out 4-byte aligned");
    if (tokens_off < out_off + (uint64_t)rows * D * 4 && out_off < tokens_off + (uint64_t)rows * 4)
        return fail(QL_E_INVALID, "tokens and out overlap");
    int rc = set_device(ctx);
    if (rc) return rc;
    ql::EmbedArgs a;
    a.w = reinterpret_cast<const uint16_t*>(weights->base + embed_off);
    a.tokens = reinterpret_cast<const uint32_t*>(act->base + tokens_off);
    a.out = reinterpret_cast<float*>(act->base + out_off);
    a.vocab = vocab;
    a.D = D;
    a.rows = rows;
    a.vec = D % 8 == 0 && embed_off % 16 == 0 && out_off % 16 == 0;
    QL_HIP(ql::launch_embed_rows(a, ctx->stream));
    return QL_OK;
}

int ql_kv_store(ql_ctx* ctx, const ql_arena* act, uint64_t src_off, ql_arena* cache, uint64_t cache_off,
                int32_t max_t, int32_t rows, int32_t row_len, int32_t pos0)
{
    if (!ctx || !act || !cache) return fail(QL_E_INVALID, "null context or arena");
    if (max_t <= 0 || rows <= 0 || row_len <= 0 || pos0 < 0)
        return fail(QL_E_INVALID, "max_t, rows and row_len must be positive, pos0 >= 0");
    if ((int64_t)pos0 + rows > max_t)
        return fail(QL_E_RANGE, "context length %lld exceeds the cache's %d positions", (long long)pos0 + rows, max_t);
    if (row_len % 4) return fail(QL_E_INVALID, "row_len must be a multiple of 4 (got %d)", row_len);
    if ((int64_t)rows * row_len >= (1ll << 31)) return fail(QL_E_INVALID, "rows x row_len too large");
    if (!in_range(src_off, (uint64_t)rows * row_len * 4, act->size)) return fail(QL_E_RANGE, "src [rows, row_len] outside the activation arena");
    if (!in_range(cache_off, (uint64_t)max_t * row_len * 4, cache->size)) return fail(QL_E_RANGE, "cache [max_t, row_len] outside its arena");
    if (src_off % 16 || cache_off % 16) return fail(QL_E_ALIGN, "src and cache offsets must be 16-byte aligned");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(ql::launch_kv_store(reinterpret_cast<const float*>(act->base + src_off),
                               reinterpret_cast<float*>(cache->base + cache_off), rows, row_len, pos0, ctx->stream));
    return QL_OK;
}

namespace {

// The dimension checks shared by ql_attention_decode and ql_plan_attention.
int check_attention_dims(int32_t max_t, int32_t M, int32_t n_head, int32_t n_kv_head, int32_t D, int32_t past_len)
{
    if (M < 1 || M > 65535 || n_head < 1 || n_head > 65535 || n_kv_head < 1 || past_len < 0 || max_t < 1)
        return fail(QL_E_INVALID, "bad attention dimensions");
    if (n_head % n_kv_head) return fail(QL_E_INVALID, "n_head (%d) must be a multiple of n_kv_head (%d)", n_head, n_kv_head);
    if (D < 4 || D > ql::kAttnMaxD || D % 4) return fail(QL_E_INVALID, "head dim must be 4..%d, a multiple of 4 (got %d)", ql::kAttnMaxD, D);
    if ((int64_t)past_len + M > max_t)
        return fail(QL_E_RANGE, "context length %lld exceeds the cache's %d positions", (long long)past_len + M, max_t);
    if ((int64_t)past_len + M > ql::kAttnMaxT)
        return fail(QL_E_INVALID, "context length %lld above the supported %d", (long long)past_len + M, ql::kAttnMaxT);
    return QL_OK;
}

}  // namespace

int ql_plan_attention(int32_t max_t, int32_t M, int32_t n_head, int32_t n_kv_head, int32_t D, int32_t past_len,
                      ql_attn_info* info)
{
    if (!info) return fail(QL_E_INVALID, "null info");
    int rc = check_attention_dims(max_t, M, n_head, n_kv_head, D, past_len);
    if (rc) return rc;
    ql::AttnArgs a{};
    a.M = M;
    a.H = n_head;
    a.KV = n_kv_head;
    a.G = n_head / n_kv_head;
    a.D = D;
    a.past = past_len;
    if (ql::plan_attention(&a)) return fail(QL_E_INVALID, "attention shape does not fit the workspace");
    info->heads_per_run = a.heads_per_run;
    info->nsplit = a.nsplit;
    info->workgroups = a.KV * a.runs_per_group * a.nsplit * a.M;
    info->keys_per_split = a.chunk_cap;
    return QL_OK;
}

int ql_attention_decode(ql_ctx* ctx, ql_arena* act, uint64_t q_off, const ql_arena* cache, uint64_t k_off,
                        uint64_t v_off, int32_t max_t, int32_t M, int32_t n_head, int32_t n_kv_head, int32_t D,
                        int32_t past_len, uint64_t out_off)
{
    if (!ctx || !act || !cache) return fail(QL_E_INVALID, "null context or arena");
    int rc = check_attention_dims(max_t, M, n_head, n_kv_head, D, past_len);
    if (rc) return rc;
    const uint64_t qo = (uint64_t)M * n_head * D * 4, cb = (uint64_t)max_t * n_kv_head * D * 4;
    if (!in_range(q_off, qo, act->size)) return fail(QL_E_RANGE, "q [M, n_head, D] outside the activation arena");
    if (!in_range(out_off, qo, act->size)) return fail(QL_E_RANGE, "out [M, n_head, D] outside the activation arena");
    if (!in_range(k_off, cb, cache->size) || !in_range(v_off, cb, cache->size))
        return fail(QL_E_RANGE, "K/V cache [max_t, n_kv_head * D] outside its arena");
    if (q_off % 16 || out_off % 16 || k_off % 16 || v_off % 16) return fail(QL_E_ALIGN, "offsets must be 16-byte aligned");
    if (q_off < out_off + qo && out_off < q_off + qo) return fail(QL_E_INVALID, "q and out overlap");
    rc = set_device(ctx);
    if (rc) return rc;
    ql::AttnArgs a;
    a.q = reinterpret_cast<const float*>(act->base + q_off);
    a.k = reinterpret_cast<const float*>(cache->base + k_off);
    a.v = reinterpret_cast<const float*>(cache->base + v_off);
    a.out = reinterpret_cast<float*>(act->base + out_off);
    a.ws = ctx->attn_ws;
    a.M = M;
    a.H = n_head;
    a.KV = n_kv_head;
    a.G = n_head / n_kv_head;
    a.D = D;
    a.past = past_len;
    a.scale = (float)(1.4426950408889634 / std::sqrt((double)D));   // log2(e) / sqrt(D): scores in base-2 units
    if (ql::plan_attention(&a)) return fail(QL_E_INVALID, "attention shape does not fit the workspace");
    QL_HIP(ql::launch_attention(a, ctx->stream));
    return QL_OK;
}

int ql_add_rmsnorm(ql_ctx* ctx, ql_arena* act, uint64_t x_off, uint64_t d_off, const ql_arena* weights,
                   uint64_t w_off, float eps, int32_t M, int32_t C, uint64_t sum_off, uint64_t y_off)
{
    if (!ctx || !act || !weights) return fail(QL_E_INVALID, "null context or arena");
    if (M < 1 || M > 65535 || C < 1 || C > (1 << 24)) return fail(QL_E_INVALID, "M must be 1..65535 and C 1..2^24");
    if (!(eps >= 0.f)) return fail(QL_E_INVALID, "eps must be >= 0");
    const uint64_t rb = (uint64_t)M * C * 4;
    if (!in_range(x_off, rb, act->size) || !in_range(y_off, rb, act->size) ||
        (d_off != QL_NONE && !in_range(d_off, rb, act->size)) || (sum_off != QL_NONE && !in_range(sum_off, rb, act->size)))
        return fail(QL_E_RANGE, "x, d, sum or y [M, C] outside the activation arena");
    if (!in_range(w_off, (uint64_t)C * 4, weights->size)) return fail(QL_E_RANGE, "norm weight [C] outside the weight arena");
    if (sum_off != QL_NONE && d_off == QL_NONE) return fail(QL_E_INVALID, "sum_off needs d_off (the sum is x + d)");
    if (x_off % 4 || y_off % 4 || w_off % 4 || (d_off != QL_NONE && d_off % 4) || (sum_off != QL_NONE && sum_off % 4))
        return fail(QL_E_ALIGN, "offsets must be 4-byte aligned");
    const uint64_t ya = y_off, yb = y_off + rb;
    auto overlaps = [&](uint64_t o) { return o != QL_NONE && o < yb && ya < o + rb; };
    if (overlaps(x_off) || overlaps(d_off) || overlaps(sum_off)) return fail(QL_E_INVALID, "y overlaps an input or the sum");
    // the sum may replace x or d in place (same offset), never overlap them partly: other
    // threads' elements would change under their reads
    auto partly = [&](uint64_t o) { return o != QL_NONE && o != sum_off && o < sum_off + rb && sum_off < o + rb; };
    if (sum_off != QL_NONE && (partly(x_off) || partly(d_off)))
        return fail(QL_E_INVALID, "the sum partly overlaps x or d (in place it must start at the same offset)");
    int rc = set_device(ctx);
    if (rc) return rc;
    ql::ElemArgs a{};
    a.x = reinterpret_cast<const float*>(act->base + x_off);
    a.d = d_off == QL_NONE ? nullptr : reinterpret_cast<const float*>(act->base + d_off);
    a.w = reinterpret_cast<const float*>(weights->base + w_off);
    a.s = sum_off == QL_NONE ? nullptr : reinterpret_cast<float*>(act->base + sum_off);
    a.y = reinterpret_cast<float*>(act->base + y_off);
    a.M = M;
    a.C = C;
    a.eps = eps;
    a.vec = C % 4 == 0 && x_off % 16 == 0 && y_off % 16 == 0 && w_off % 16 == 0 &&
            (d_off == QL_NONE || d_off % 16 == 0) && (sum_off == QL_NONE || sum_off % 16 == 0);
    QL_HIP(ql::launch_add_rmsnorm(a, ctx->stream));
    return QL_OK;
}

int ql_silu_mul(ql_ctx* ctx, ql_arena* act, uint64_t gate_off, uint64_t up_off, int64_t n, uint64_t y_off)
{
    if (!ctx || !act) return fail(QL_E_INVALID, "null context or arena");
    if (n < 1 || n > (1ll << 34)) return fail(QL_E_INVALID, "n out of range");
    const uint64_t b = (uint64_t)n * 4;
    if (!in_range(gate_off, b, act->size) || !in_range(up_off, b, act->size) || !in_range(y_off, b, act->size))
        return fail(QL_E_RANGE, "gate, up or y [n] outside the activation arena");
    if (gate_off % 16 || up_off % 16 || y_off % 16) return fail(QL_E_ALIGN, "offsets must be 16-byte aligned");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(ql::launch_silu_mul(reinterpret_cast<const float*>(act->base + gate_off),
                               reinterpret_cast<const float*>(act->base + up_off),
                               reinterpret_cast<float*>(act->base + y_off), n, ctx->stream));
    return QL_OK;
}

int ql_plan_batch(int32_t count, const ql_gptq_desc* descs, int32_t M, uint64_t* scratch_bytes)
{
    if (!descs || !scratch_bytes || count <= 0 || count > ql::kMaxBatch)
        return fail(QL_E_INVALID, "batch needs 1..%d descriptors", ql::kMaxBatch);
    uint64_t total = 0;
    for (int i = 0; i < count; i++) {
        ql_plan p;
        int rc = plan_impl(M, descs[i].N, descs[i].K, descs[i].group, &p);
        if (rc) return rc;
        total += align256(p.scratch_bytes);
    }
    *scratch_bytes = total;
    return QL_OK;
}

int ql_linear_batch(ql_ctx* ctx, int32_t count, const ql_gptq_desc* descs,
                    const ql_arena* weights, ql_arena* act, const uint64_t* x_offs,
                    int32_t x_dtype, int32_t M, const uint64_t* y_offs, uint64_t scratch_off)
{
    if (!ctx || !descs || !act || !x_offs || !y_offs || count <= 0 || count > ql::kMaxBatch)
        return fail(QL_E_INVALID, "batch needs a context, arenas and 1..%d linears", ql::kMaxBatch);
    uint64_t total = 0;
    int rc = ql_plan_batch(count, descs, M, &total);
    if (rc) return rc;
    if (!in_range(scratch_off, total, act->size))
        return fail(QL_E_RANGE, "batch scratch (%llu bytes) outside the activation arena",
                    (unsigned long long)total);
    if (scratch_off % 16) return fail(QL_E_ALIGN, "scratch offset must be 16-byte aligned");
    bool fused = true, gemm = true;
    int bm = 0;
    for (int i = 0; i < count; i++) {
        if ((rc = check_desc(&descs[i], weights))) return rc;
        if ((rc = check_io(&descs[i], act, x_offs[i], x_dtype, M, y_offs[i]))) return rc;
        ql_plan p;
        plan_impl(M, descs[i].N, descs[i].K, descs[i].group, &p);
        const bool aligned = gemv_aligned(&descs[i], x_offs[i], y_offs[i]);
        fused &= p.kind == QL_KIND_GEMV_MFMA && aligned && descs[i].group == descs[0].group;
        gemm &= p.kind == QL_KIND_GEMM_MFMA && aligned;
        if (gemm) {
            const int b = ql::gemm_shape(M, descs[i].N, descs[i].K, descs[i].group, ql::kPlanCUs).bm;
            gemm &= i == 0 || b == bm;
            bm = b;
        }
    }
    if (gemm && prefill_batch(ctx, count, descs, weights, act, x_offs, x_dtype, M, y_offs, &rc)) return rc;
    if (gemm) {
        // one launch; each linear's partial sums at its own offset, as ql_plan_batch sized them
        if ((rc = set_device(ctx))) return rc;
        ql::GemmBatch b{};
        b.count = count;
        b.M = M;
        b.x_dtype = x_dtype;
        b.bm = bm;
        // a K split pays for its partial-sum round trips only when the tiles leave CUs idle; the
        // batch's tiles together may already fill the device (then no linear splits; the scratch
        // ql_plan_batch sized per linear is an upper bound)
        long tiles = 0;
        for (int i = 0; i < count; i++) {
            const ql::GemmShape s = ql::gemm_shape(M, descs[i].N, descs[i].K, descs[i].group, ql::kPlanCUs);
            tiles += (long)s.tiles_n * s.tiles_m;
        }
        const bool no_split = tiles * 2 >= ql::kPlanCUs;
        uint64_t off = scratch_off;
        int wg = 0, counter_base = 0;
        for (int i = 0; i < count; i++) {
            if ((rc = gemm_entry(&descs[i], weights, act, x_offs[i], M, y_offs[i],
                                 reinterpret_cast<float*>(act->base + off), ctx->counters,
                                 counter_base, wg, &b.L[i], no_split)))
                return rc;
            const ql::GemmLinear& L = b.L[i];
            if (L.split > 1) counter_base += L.tiles_n * L.tiles_m;
            off += align256(ql::gemm_partial_bytes(M, descs[i].N, L.split));
            wg += L.tiles_n * L.tiles_m * L.split;
        }
        b.wg_total = wg;
        QL_HIP(launch_gemm_parts(b, ctx->stream));
        return QL_OK;
    }
    if (!fused) {
        uint64_t off = scratch_off;
        for (int i = 0; i < count; i++) {
            ql_plan p;
            plan_impl(M, descs[i].N, descs[i].K, descs[i].group, &p);
            if ((rc = ql_linear(ctx, &descs[i], weights, act, x_offs[i], x_dtype, M, y_offs[i], off)))
                return rc;
            off += align256(p.scratch_bytes);
        }
        return QL_OK;
    }
    if ((rc = set_device(ctx))) return rc;
    ql::GemvBatch b{};
    b.count = count;
    b.M = M;
    b.x_dtype = x_dtype;
    uint64_t off = scratch_off;
    int wg = 0, counter_base = 0;
    for (int i = 0; i < count; i++) {
        const ql_gptq_desc* d = &descs[i];
        const ql::GemvShape s = ql::gemv_shape(M, d->N, d->K, d->group);
        ql::GemvLinear L = make_linear(d, weights);
        L.x = act->base + x_offs[i];
        L.y = reinterpret_cast<float*>(act->base + y_offs[i]);
        L.split = s.split;
        L.strips = s.strips;
        L.wg_begin = wg;
        L.partial = reinterpret_cast<float*>(act->base + off);
        L.counters = ctx->counters + counter_base;
        counter_base += s.strips;
        if (counter_base > ql::kCounterCapacity) return fail(QL_E_INVALID, "batch too wide");
        off += align256(ql::gemv_partial_bytes(M, d->N, s.split));
        wg += s.strips * s.split;
        b.L[i] = L;
    }
    b.wg_total = wg;
    QL_HIP(ql::launch_gemv_batch(b, ctx->stream));
    return QL_OK;
}

namespace {

int plan_seq_impl(int32_t n, const ql_gptq_desc* descs, int32_t M, const uint64_t* x_offs, int32_t x_dtype,
                  const uint64_t* y_offs, const ql_seq_fuse* fuse, int32_t grid, ql_seq_info* info)
{
    if (!info) return fail(QL_E_INVALID, "null info pointer");
    if (grid < 1 || grid > (1 << 16)) return fail(QL_E_INVALID, "grid must be 1..65536");
    std::vector<ql::SeqSpec> specs;
    int rc = seq_resolve(n, descs, M, x_offs, x_dtype, y_offs, UINT64_MAX, UINT64_MAX, &specs, fuse);
    if (rc) return rc;
    if (M > ql::kGemvMaxM && seq_chained(specs)) {
        PrefillPasses P;
        plan_prefill_passes(specs, fuse, x_offs, M, grid, &P);
        fill_prefill_passes_info(P, n, prefill_passes_bytes(P), info);
        return QL_OK;
    }
    if (M > ql::kGemvMaxM) {
        ql::PrefillPlan pp;
        ql::plan_prefill(prefill_specs(specs), M, grid, &pp);
        fill_prefill_info(pp, n, M, specs, prefill_layout(n, pp).total, info);
        return QL_OK;
    }
    if (!seq_fused(specs) && ql::strip_eligible(specs, M)) {
        ql::StripPlan sp;
        ql::plan_strips(specs, M, grid, &sp);
        fill_strip_info(sp, n, strip_layout(specs, sp, M).total, info);
        return QL_OK;
    }
    if (passes_ok(specs, M, x_dtype)) {
        PassesPlan P;
        plan_passes(specs, fuse, x_offs, M, grid, &P);
        if (P.depth < 1) return fail(QL_E_INVALID, "sequence shapes do not fit the K-part strips");
        uint64_t bytes = P.buffer_bytes();
        for (int p = 0; p < P.depth; p++)
            bytes += strip_layout(P.specs[p], P.plans[p], M).total + sizeof(ql::PartSum) * P.members[p].size();
        fill_passes_info(P, n, bytes, grid, info);
        return QL_OK;
    }
    ql::SeqPlanOut p;
    ql::plan_seq(specs, M, grid, &p);
    const std::string bad = ql::verify_seq_plan(specs, M, p);
    if (!bad.empty()) return fail(QL_E_INVALID, "sequence plan check failed: %s", bad.c_str());
    fill_seq_info(p, n, seq_layout(specs, p, M).total, info);
    return QL_OK;
}

}  // namespace

int ql_plan_seq(int32_t n, const ql_gptq_desc* descs, int32_t M, const uint64_t* x_offs,
                int32_t x_dtype, const uint64_t* y_offs, int32_t grid, ql_seq_info* info)
{
    return plan_seq_impl(n, descs, M, x_offs, x_dtype, y_offs, nullptr, grid, info);
}

int ql_plan_seq_fused(int32_t n, const ql_gptq_desc* descs, int32_t M, const uint64_t* x_offs,
                      int32_t x_dtype, const uint64_t* y_offs, const ql_seq_fuse* fuse, int32_t grid,
                      ql_seq_info* info)
{
    return plan_seq_impl(n, descs, M, x_offs, x_dtype, y_offs, fuse, grid, info);
}

namespace {

int seq_create_impl(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights, ql_arena* act,
                    const uint64_t* x_offs, int32_t x_dtype, int32_t M, const uint64_t* y_offs,
                    const ql_seq_fuse* fuse, ql_seq** out)
{
    if (!ctx || !weights || !act || !out) return fail(QL_E_INVALID, "null context, arena or output");
    *out = nullptr;
    if (ctx->capturing) return fail(QL_E_STATE, "ql_seq_create during graph capture");
    if (weights->device != ctx->device || act->device != ctx->device)
        return fail(QL_E_INVALID, "arenas belong to another device");
    std::vector<ql::SeqSpec> specs;
    int rc = seq_resolve(n, descs, M, x_offs, x_dtype, y_offs, weights->size, act->size, &specs, fuse);
    if (rc) return rc;
    if ((rc = set_device(ctx))) return rc;
    const bool fused = seq_fused(specs);
    if (M > ql::kGemvMaxM && seq_chained(specs))
        return prefill_passes_create(ctx, n, descs, weights, act, x_offs, M, y_offs, fuse, specs, out);
    if (M > ql::kGemvMaxM) return prefill_create(ctx, n, descs, weights, act, x_offs, x_dtype, M, y_offs, specs, out);
    if (!fused && ql::strip_eligible(specs, M))
        return strip_create(ctx, n, descs, weights, act, x_offs, x_dtype, M, y_offs, specs, out);
    if (passes_ok(specs, M, x_dtype))
        return passes_create(ctx, n, descs, weights, act, x_offs, x_dtype, M, y_offs, fuse, specs, out);
    int per_cu = 0;
    QL_HIP(ql::seq_blocks_per_cu(M, descs[0].group, fused, &per_cu));
    if (per_cu < 1) return fail(QL_E_INVALID, "sequence kernel does not fit on a CU");
    const int grid = std::min(per_cu, ql::seq_wg_per_cu()) * ctx->cu_count;
    ql::SeqPlanOut p;
    ql::plan_seq(specs, M, grid, &p);
    // a plan that left a group uncomputed or a part unreduced would make the kernel wait forever
    const std::string bad = ql::verify_seq_plan(specs, M, p);
    if (!bad.empty()) return fail(QL_E_INVALID, "sequence plan check failed: %s", bad.c_str());
    if (p.lds_bytes > ql::seq_lds_budget(M, descs[0].group)) return fail(QL_E_INVALID, "sequence plan exceeds LDS");
    const SeqLayout lay = seq_layout(specs, p, M);

    char* dev = nullptr;
    QL_HIP(hipMalloc(&dev, lay.total));
    std::vector<ql::SeqLinear> lin(n);
    std::vector<ql::SeqFuseLin> fl(n);
    for (int i = 0; i < n; i++) {
        const ql_gptq_desc* d = &descs[i];
        ql::SeqLinear& L = lin[i];
        ql::SeqFuseLin& F = fl[i];
        const ql::GemvLinear g = make_linear(d, weights);
        L.qweight = g.qweight;
        L.qzeros = g.qzeros ? g.qzeros : reinterpret_cast<const uint32_t*>(dev + lay.sym_zeros);
        L.scales = g.scales;
        L.bias = g.bias;
        L.x = specs[i].src >= 0 ? nullptr : act->base + x_offs[i];
        L.y = reinterpret_cast<float*>(act->base + y_offs[i]);
        L.y_ll = reinterpret_cast<uint64_t*>(dev + lay.y_ll[i]);
        L.src = specs[i].src;
        L.N = d->N;
        L.K = d->K;
        L.x_dtype = x_dtype;
        F.fuse = specs[i].fuse;
        F.src2 = specs[i].src2;
        F.res_src = specs[i].res_src;
        F.norm_w = nullptr;
        F.x2 = nullptr;
        F.res = nullptr;
        F.norm_eps = 0.f;
        if (F.fuse & ql::kFuseNorm) {
            F.norm_w = reinterpret_cast<const float*>(weights->base + fuse[i].norm_w_off);
            F.norm_eps = fuse[i].norm_eps;
        }
        if ((F.fuse & ql::kFuseGlu) && F.src2 < 0) F.x2 = reinterpret_cast<const float*>(act->base + fuse[i].x2_off);
        if ((F.fuse & ql::kFuseRes) && F.res_src < 0) F.res = reinterpret_cast<const float*>(act->base + fuse[i].res_off);
        F.ssq = lay.ssq[i] == UINT64_MAX ? nullptr : reinterpret_cast<uint64_t*>(dev + lay.ssq[i]);
    }
    hipError_t e = hipMemset(dev, 0, lay.total);
    if (e == hipSuccess && lay.sym_words)
        e = hipMemsetD32(reinterpret_cast<hipDeviceptr_t>(dev + lay.sym_zeros), 0x77777777,
                         lay.sym_words);
    if (e == hipSuccess) e = hipMemcpy(dev + lay.lin, lin.data(), sizeof(ql::SeqLinear) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess && fused)
        e = hipMemcpy(dev + lay.fl, fl.data(), sizeof(ql::SeqFuseLin) * n, hipMemcpyHostToDevice);
    if (e == hipSuccess && !p.tasks.empty())
        e = hipMemcpy(dev + lay.tasks, p.tasks.data(), sizeof(ql::SeqTask) * p.tasks.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(dev + lay.task_begin, p.task_begin.data(), sizeof(int32_t) * p.task_begin.size(),
                      hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(dev + lay.first_tile, p.first_tile.data(), sizeof(int32_t) * p.first_tile.size(),
                      hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(e, "ql_seq_create upload");
    }
    ql_seq* q = new ql_seq();
    q->device = ctx->device;
    q->dev = dev;
    q->lds = p.lds_bytes;
    ql::SeqArgs& a = q->args;
    a.lin = reinterpret_cast<const ql::SeqLinear*>(dev + lay.lin);
    a.tasks = reinterpret_cast<const ql::SeqTask*>(dev + lay.tasks);
    a.task_begin = reinterpret_cast<const int32_t*>(dev + lay.task_begin);
    a.first_tile = reinterpret_cast<const int32_t*>(dev + lay.first_tile);
    a.tickets = reinterpret_cast<unsigned long long*>(dev + lay.tickets);
    a.abort = reinterpret_cast<uint32_t*>(dev + lay.words);
    a.err = reinterpret_cast<uint32_t*>(dev + lay.words + 4);
    a.part = reinterpret_cast<uint64_t*>(dev + lay.part);
    a.M = M;
    a.G = p.grid;
    a.group = descs[0].group;
    a.spin_limit = 1u << 22;
    a.block_mode = p.block_mode ? 1 : 0;
    a.fused = fused ? 1 : 0;
    a.fl = fused ? reinterpret_cast<const ql::SeqFuseLin*>(dev + lay.fl) : nullptr;
    fill_seq_info(p, n, lay.total, &q->info);
    *out = q;
    return QL_OK;
}

}  // namespace

int ql_seq_create(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights,
                  ql_arena* act, const uint64_t* x_offs, int32_t x_dtype, int32_t M,
                  const uint64_t* y_offs, ql_seq** out)
{
    return seq_create_impl(ctx, n, descs, weights, act, x_offs, x_dtype, M, y_offs, nullptr, out);
}

int ql_seq_create_fused(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights,
                        ql_arena* act, const uint64_t* x_offs, int32_t x_dtype, int32_t M,
                        const uint64_t* y_offs, const ql_seq_fuse* fuse, ql_seq** out)
{
    return seq_create_impl(ctx, n, descs, weights, act, x_offs, x_dtype, M, y_offs, fuse, out);
}

int ql_seq_get_info(const ql_seq* seq, ql_seq_info* info)
{
    if (!seq || !info) return fail(QL_E_INVALID, "null sequence or info");
    *info = seq->info;
    return QL_OK;
}

int ql_seq_run(ql_ctx* ctx, ql_seq* seq)
{
    if (!ctx || !seq) return fail(QL_E_INVALID, "null context or sequence");
    if (seq->device != ctx->device) return fail(QL_E_INVALID, "sequence belongs to another device");
    int rc = set_device(ctx);
    if (rc) return rc;
    if (seq->passes) {
        for (const SeqStep& st : seq->steps) {
            switch (st.kind) {
            case SeqStep::kNorm: QL_HIP(ql::launch_add_rmsnorm(st.e, ctx->stream)); break;
            case SeqStep::kGlu: QL_HIP(ql::launch_silu_mul(st.g, st.u, st.o, st.n, ctx->stream)); break;
            case SeqStep::kPrefill: QL_HIP(ql::launch_prefill(st.p, true, ctx->stream)); break;
            case SeqStep::kGemm: QL_HIP(ql::launch_gemm_batch(st.gb, ctx->stream)); break;
            case SeqStep::kStrips: QL_HIP(ql::launch_strips(st.s, st.lds, ctx->stream)); break;
            case SeqStep::kPartSums: QL_HIP(ql::launch_part_sums(st.sums, st.count, st.M, st.max_n, st.glu, ctx->stream)); break;
            }
        }
    } else if (seq->prefill) QL_HIP(ql::launch_prefill(seq->pargs, true, ctx->stream));
    else if (seq->strips) QL_HIP(ql::launch_strips(seq->sargs, seq->lds, ctx->stream));
    else QL_HIP(ql::launch_seq(seq->args, seq->lds, ctx->stream));
    return QL_OK;
}

int ql_seq_status(ql_ctx* ctx, ql_seq* seq)
{
    if (!ctx || !seq) return fail(QL_E_INVALID, "null context or sequence");
    if (ctx->capturing) return fail(QL_E_STATE, "ql_seq_status during graph capture");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipStreamSynchronize(ctx->stream));
    if (seq->strips || seq->prefill || seq->passes) return QL_OK;   // no device-side waits: nothing can abort
    uint32_t words[2] = {0, 0};
    QL_HIP(hipMemcpy(words, seq->args.abort, sizeof words, hipMemcpyDeviceToHost));
    if (words[0] == 0 && words[1] == 0) return QL_OK;
    QL_HIP(hipMemset(seq->args.abort, 0, sizeof words));
    return fail(QL_E_STATE, "sequence run aborted (code %u): a wait exceeded its spin limit; outputs "
                "of that run are invalid", words[1]);
}

int ql_seq_set_spin_limit(ql_seq* seq, uint32_t polls)
{
    if (!seq) return fail(QL_E_INVALID, "null sequence");
    if (polls < 64) return fail(QL_E_INVALID, "spin limit must be at least 64 polls");
    seq->args.spin_limit = polls;
    return QL_OK;
}

int ql_seq_destroy(ql_seq* seq)
{
    if (!seq) return fail(QL_E_INVALID, "null sequence");
    (void)hipSetDevice(seq->device);
    for (char* b : seq->bufs) (void)hipFree(b);
    (void)hipFree(seq->dev);
    delete seq;
    return QL_OK;
}

int ql_sync(ql_ctx* ctx)
{
    if (!ctx) return fail(QL_E_INVALID, "null context");
    if (ctx->capturing) return fail(QL_E_STATE, "ql_sync during graph capture");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipStreamSynchronize(ctx->stream));
    return QL_OK;
}

int ql_timer_start(ql_ctx* ctx)
{
    if (!ctx) return fail(QL_E_INVALID, "null context");
    if (ctx->capturing) return fail(QL_E_STATE, "timer during graph capture");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipEventRecord(ctx->ev_start, ctx->stream));
    return QL_OK;
}

int ql_timer_stop(ql_ctx* ctx, float* elapsed_ms)
{
    if (!ctx || !elapsed_ms) return fail(QL_E_INVALID, "null context or output");
    if (ctx->capturing) return fail(QL_E_STATE, "timer during graph capture");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipEventRecord(ctx->ev_stop, ctx->stream));
    QL_HIP(hipEventSynchronize(ctx->ev_stop));
    QL_HIP(hipEventElapsedTime(elapsed_ms, ctx->ev_start, ctx->ev_stop));
    return QL_OK;
}

int ql_graph_begin(ql_ctx* ctx)
{
    if (!ctx) return fail(QL_E_INVALID, "null context");
    if (ctx->capturing) return fail(QL_E_STATE, "capture already active");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return QL_OK;
}

int ql_graph_end(ql_ctx* ctx, ql_graph** out)
{
    if (!ctx || !out) return fail(QL_E_INVALID, "null context or output");
    if (!ctx->capturing) return fail(QL_E_STATE, "no capture active");
    *out = nullptr;
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    QL_HIP(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_fail(e, "hipGraphInstantiate");
    }
    ql_graph* gr = new ql_graph();
    gr->graph = g;
    gr->exec = exec;
    *out = gr;
    return QL_OK;
}

int ql_graph_launch(ql_ctx* ctx, ql_graph* graph)
{
    if (!ctx || !graph) return fail(QL_E_INVALID, "null context or graph");
    if (ctx->capturing) return fail(QL_E_STATE, "graph launch during capture");
    int rc = set_device(ctx);
    if (rc) return rc;
    QL_HIP(hipGraphLaunch(graph->exec, ctx->stream));
    return QL_OK;
}

int ql_graph_destroy(ql_graph* graph)
{
    if (!graph) return fail(QL_E_INVALID, "null graph");
    (void)hipGraphExecDestroy(graph->exec);
    (void)hipGraphDestroy(graph->graph);
    delete graph;
    return QL_OK;
}

}  // extern "C"
