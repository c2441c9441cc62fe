/*
 * qlinear.h — C ABI of libqlinear.so: GPTQ int4 quantized linears on MI355X (gfx950).
 *
 * Drop-in for the quantized-linear hot path of intplusplus/webllm. Plain pointers, sizes and
 * byte offsets only; every function returns an int status (QL_OK = 0, negative = error class)
 * and ql_last_error() holds the message of the calling thread's last failure. No exceptions
 * cross the ABI. Weights stay GPTQ-packed in device memory; dequantization is fused into the
 * kernels.
 *
 * Reference interfaces each entry point replaces (paths relative to the reference checkout):
 *   ql_create / ql_destroy        src/gpu/device.ts:40-98 initGpu (one device, one queue)
 *   ql_arena_*                    src/gpu/buffer.ts:20-34 createStorageBuffer, :103-120 writeF16 /
 *                                 device.queue.writeBuffer, :123-170 readback; src/gpu/arena.ts:17-59
 *   ql_gptq_desc / ql_gptq_check  src/weights/quant.ts:16-30 GptqInt4Params, :44-79 validation
 *   ql_unpack_f16                 src/weights/qwen-loader.ts:55-67 dequantGptqLinear +
 *                                 src/model/qwen.ts:262-266 uploadF16 (CPU dequant + f16 encode)
 *   ql_unpack_f32, ql_unpack_f32_ex  src/weights/quant.ts:42-118 dequantizeGptqInt4
 *   ql_plan_linear                src/model/qwen.ts:61-74 planGemvSplit + the branch in :568-618
 *   ql_linear                     src/model/qwen.ts:568-618 QwenGpt.gemm (GEMV / split-K / GEMM)
 *   ql_linear_batch               src/model/qwen.ts:411-413, :464-465 (q/k/v and gate/up issued
 *                                 back to back on one input inside one CommandBatch pass)
 *   ql_sync, ql_timer_*           src/gpu/buffer.ts:123-145 mapAsync readback,
 *                                 src/gpu/pipeline.ts:119-161 timestamp-query profiling
 *   ql_graph_*                    src/gpu/pipeline.ts:55-117 CommandBatch (one submit per forward)
 *   ql_plan_seq, ql_seq_*         src/gpu/pipeline.ts:71-116 CommandBatch.dispatch/endPass/submit
 *                                 with src/model/qwen.ts:556-559 passBreak, as runForward uses
 *                                 them (qwen.ts:382-387, :411-473): a forward's linears recorded
 *                                 once, then submitted as one unit per step
 *   ql_seq_fuse, ql_plan_seq_fused, ql_seq_create_fused
 *                                 the same, with the layer's elementwise dispatches around the
 *                                 linears folded in: rmsnorm before q/k/v and gate/up
 *                                 (qwen.ts:403-405, :458-460, src/gpu/kernels/norm/rmsnorm.wgsl),
 *                                 the residual vec_add after o and down (qwen.ts:453-455,
 *                                 :476-478, src/gpu/kernels/misc/vec_add.wgsl) and silu_mul
 *                                 before down (qwen.ts:468-470,
 *                                 src/gpu/kernels/activation/silu_mul.wgsl)
 */
#ifndef QLINEAR_H
#define QLINEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes. -1..-7 are the failure classes of quant.ts:46-79, in its check order. */
#define QL_OK 0
#define QL_E_BITS (-1)          /* bits != 4                                    quant.ts:46 */
#define QL_E_GROUP (-2)         /* group <= 0                                   quant.ts:47 */
#define QL_E_DIMS (-3)          /* K <= 0 or N <= 0                             quant.ts:48 */
#define QL_E_QWEIGHT_SHORT (-4) /* qweight [ceil(K/8), N] int32 outside arena   quant.ts:58 */
#define QL_E_SCALES_SHORT (-5)  /* scales [ceil(K/group), N] outside arena      quant.ts:62 */
#define QL_E_QZEROS_SHORT (-6)  /* qzeros [ceil(K/group), ceil(N/8)] outside    quant.ts:69 */
#define QL_E_GROUP_PACK (-7)    /* group % 8 != 0                               quant.ts:76 */
#define QL_E_INVALID (-10)      /* null handle/pointer, bad M, bad dtype                     */
#define QL_E_RANGE (-11)        /* activation/output/scratch range outside its arena         */
#define QL_E_ALIGN (-12)        /* misaligned offset (int32/f32: 4 B, f16: 2 B)              */
#define QL_E_HIP (-13)          /* HIP runtime failure (message in ql_last_error)            */
#define QL_E_STATE (-14)        /* call not valid in the current state (graph capture)       */

/* Sentinel for optional offsets (no qzeros -> symmetric zero 8, quant.ts:73-74; no bias). */
#define QL_NONE UINT64_MAX

#define QL_DTYPE_F32 0
#define QL_DTYPE_F16 1

/* kernel families returned by ql_plan_linear */
#define QL_KIND_GEMV_MFMA 1   /* M <= 16: packed-int4 GEMV on MFMA, hi/lo split activations */
#define QL_KIND_GEMV_SIMPLE 2 /* any shape: one lane per output column, fp32                */
#define QL_KIND_GEMM_MFMA 3   /* M > 16: LDS-dequant f16 tiles, MFMA f16, fp32 accumulate   */
#define QL_KIND_GEMM_SIMPLE 4 /* any shape: f16 operands, fp32 accumulate, no MFMA          */

typedef struct ql_ctx ql_ctx;
typedef struct ql_arena ql_arena;
typedef struct ql_graph ql_graph;

/* GPTQ int4 linear inside a weight arena (byte offsets). Mirrors GptqInt4Params
 * (quant.ts:16-30) except that scales stay raw fp16 as stored in the checkpoint.
 *   qweight int32 [ceil(K/8), N]   8 nibbles per word, low nibble = smallest input index
 *   qzeros  int32 [ceil(K/group), ceil(N/8)] stored zero - 1, or QL_NONE (zero = 8)
 *   scales  fp16  [ceil(K/group), N]
 *   bias    fp32  [N] or QL_NONE
 * W[n,k] = (q[k,n] - (qz[g,n] + 1)) * s[g,n], g = k / group. */
typedef struct ql_gptq_desc {
    uint64_t qweight_off;
    uint64_t qzeros_off;
    uint64_t scales_off;
    uint64_t bias_off;
    int32_t K;     /* in_features  */
    int32_t N;     /* out_features */
    int32_t group; /* group size (128 for Qwen2.5 GPTQ) */
    int32_t bits;  /* must be 4 */
} ql_gptq_desc;

typedef struct ql_plan {
    int32_t kind;          /* QL_KIND_* */
    int32_t split;         /* K segments; partial sums reduced in fixed ascending order */
    int32_t waves;         /* waves per workgroup splitting each segment */
    int32_t grid_x;        /* workgroups along N */
    int32_t grid_y;        /* workgroups along K (split) or M (GEMM) */
    int32_t block;         /* threads per workgroup */
    uint64_t scratch_bytes;/* bytes the caller must provide at scratch_off (0 if none) */
    int32_t ref_split;     /* planGemvSplit(ceil(N/256), K) of the reference, for comparison */
    int32_t reserved;
} ql_plan;

/* ---- context: one device, one HIP stream (default priority). */
int ql_create(int device, ql_ctx** out);
int ql_destroy(ql_ctx* ctx);
const char* ql_last_error(void);
int ql_device_info(ql_ctx* ctx, char* name, int name_len, int* cu_count, uint64_t* hbm_bytes);

/* ---- arenas: one device allocation addressed by byte offset (256-B aligned base). */
int ql_arena_reserve(ql_ctx* ctx, uint64_t bytes, ql_arena** out);
int ql_arena_release(ql_arena* arena);
uint64_t ql_arena_size(const ql_arena* arena);
/* device address of arena byte 0, for interop (e.g. wrapping as a framework tensor) */
uint64_t ql_arena_device_ptr(const ql_arena* arena);
/* synchronous host<->device copies; the host pointer is borrowed for the call only */
int ql_arena_write(ql_arena* arena, uint64_t off, const void* src, uint64_t bytes);
int ql_arena_read(ql_arena* arena, uint64_t off, void* dst, uint64_t bytes);
/* device-side copy between arenas, enqueued on the context stream */
int ql_arena_copy(ql_ctx* ctx, ql_arena* dst, uint64_t dst_off, const ql_arena* src,
                  uint64_t src_off, uint64_t bytes);

/* ---- GPTQ descriptors (host only, no GPU work). */
/* sizes in bytes of the three packed tensors of a K x N linear */
int ql_gptq_sizes(int32_t K, int32_t N, int32_t group, uint64_t* qweight_bytes,
                  uint64_t* qzeros_bytes, uint64_t* scales_bytes);
/* validates like quant.ts:44-79 (same classes, same order) against a weight arena of
 * arena_bytes bytes, then the bias range (QL_E_RANGE) and alignment (QL_E_ALIGN). Host only. */
int ql_gptq_validate(const ql_gptq_desc* desc, uint64_t arena_bytes);
/* ql_gptq_validate against the arena's size */
int ql_gptq_check(const ql_gptq_desc* desc, const ql_arena* weights);

/* ---- load time: fp16 [N,K] row-major, bit-identical to
 * f32ToF16Bits(dequantizeGptqInt4(...)) (quant.ts:42-118, buffer.ts:57-100). */
int ql_unpack_f16(ql_ctx* ctx, const ql_gptq_desc* desc, const ql_arena* weights,
                  ql_arena* out, uint64_t out_off);
/* many tensors at once (the loader's whole weight set, qwen-loader.ts:146-162 calling
 * dequantGptqLinear + uploadF16 per linear): tensor i into out_offs[i], same bits as
 * ql_unpack_f16. Tensors are batched into few launches (up to 32 tensors each); every descriptor
 * and output range is validated before anything is enqueued. */
int ql_unpack_f16_batch(ql_ctx* ctx, int32_t count, const ql_gptq_desc* descs,
                        const ql_arena* weights, ql_arena* out, const uint64_t* out_offs);
/* fp32 [N,K] row-major, bit-identical to dequantizeGptqInt4(...) itself (quant.ts:42-118) with
 * the scales decoded from fp16 as the loader does (safetensors.ts:180-182, qwen-loader.ts:65).
 * out_off must be 16-byte aligned. */
int ql_unpack_f32(ql_ctx* ctx, const ql_gptq_desc* desc, const ql_arena* weights,
                  ql_arena* out, uint64_t out_off);
/* ql_unpack_f32 with the scales' dtype stated: QL_DTYPE_F16 (as stored in the checkpoint; the same
 * as ql_unpack_f32) or QL_DTYPE_F32, where desc->scales_off holds f32 scales [ceil(K/group), N]
 * (4-byte aligned) — GptqInt4Params.scales as the reference takes it, any Float32Array
 * (quant.ts:22-23, :62 sizes it in values). Each weight is (q - zero) * scale rounded once to f32,
 * bit-identical to dequantizeGptqInt4 for every f32 scale (quant.ts:111-112). */
int ql_unpack_f32_ex(ql_ctx* ctx, const ql_gptq_desc* desc, const ql_arena* weights, int32_t scales_dtype,
                     ql_arena* out, uint64_t out_off);

/* ---- dispatch plan (host only, deterministic, pure). */
int ql_plan_linear(int32_t M, int32_t N, int32_t K, int32_t group, ql_plan* out);

/* ---- y[M,N] (fp32) = x[M,K] * W^T (+ bias), enqueued on the context stream.
 * x_dtype: QL_DTYPE_F32 (decode path) or QL_DTYPE_F16. Offsets are into `act`.
 * scratch_off: plan.scratch_bytes bytes in `act` for split-K partial sums (ignored when 0).
 * The caller orders work by issuing it on this one stream (stream order replaces the
 * reference's passBreak, qwen.ts:556-559). */
int ql_linear(ql_ctx* ctx, const ql_gptq_desc* desc, const ql_arena* weights, ql_arena* act,
              uint64_t x_off, int32_t x_dtype, int32_t M, uint64_t y_off, uint64_t scratch_off);

/* ql_linear with no scratch argument and no allocation. No counterpart in the reference: it is
 * for callers that cannot allocate or carve out a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same kernels, plan and results as ql_linear.
 * Split-K partial sums go to a static device array of QL_NOALLOC_SCRATCH_BYTES per GPU, resolved
 * at ql_create; a plan needing more scratch (ql_plan_linear's scratch_bytes: at most 6.94 MiB for
 * the Qwen2.5-0.5B and -7B decode shapes at M <= 16) fails with QL_E_RANGE before anything is
 * enqueued. Nothing in the array must
 * start at zero (every partial is written before it is read; the arrival counters are the
 * context's and every launch leaves them at zero). Every call on a GPU shares its array and it
 * keeps the last call's contents: calls that overlap on one GPU (several streams, contexts or
 * threads) race. */
#define QL_NOALLOC_SCRATCH_BYTES (8u << 20)
int ql_linear_noalloc(ql_ctx* ctx, const ql_gptq_desc* desc, const ql_arena* weights, ql_arena* act,
                      uint64_t x_off, int32_t x_dtype, int32_t M, uint64_t y_off);

/* y[M,N] (fp32) = x[M,K] (fp32) . W^T (+ bias) for an fp16 weight W [N,K] row-major at w_off in
 * `weights` (bias f32 [N] at bias_off or QL_NONE): the tied lm_head / embedding product,
 * QwenGpt.gemm(lnf, 'embed', logits, null, M, V, C) (qwen.ts:488-489) on gemm_gemv_f16.wgsl's
 * arithmetic (fp32 x, fp16 weights, fp32 accumulation). M = 1..65535, up to 4 rows per pass over
 * the weights (a decode-sized product: prefill rows re-read W once per 4 rows); x, y, w offsets 16-byte aligned, K % 8 == 0. */
int ql_gemv_f16w(ql_ctx* ctx, const ql_arena* weights, uint64_t w_off, uint64_t bias_off,
                 ql_arena* act, uint64_t x_off, int32_t M, int32_t N, int32_t K, uint64_t y_off);

/* ---- decode attention over the KV cache (qwen.ts:424-442).
 * Cache: per layer one fp32 K and one fp32 V region of [max_t, n_kv_head * D], row t holding the
 * vectors of position t (the reference's kCache[i] / vCache[i], qwen.ts:200-205).
 *
 * ql_kv_store: cache[(pos0 + r) * row_len + c] = src[r * row_len + c] for r < rows
 *   (misc/kv_store.wgsl); pos0 + rows > max_t fails with QL_E_RANGE (qwen.ts:352-355 throws).
 *   row_len % 4 == 0, offsets 16-byte aligned. */
int ql_kv_store(ql_ctx* ctx, const ql_arena* act, uint64_t src_off, ql_arena* cache, uint64_t cache_off,
                int32_t max_t, int32_t rows, int32_t row_len, int32_t pos0);

/* ql_attention_decode: out[m, h, :] = softmax_s(q[m, h] . K[s, h / (H / KV)] / sqrt(D)) V[s, ...]
 *   over s = 0 .. past_len + m (causal; attention/attention_gqa_cache.wgsl, CPU form
 *   reference/qwen-ref.ts:65-111 attentionGqaRef). q and out are [M, n_head, D] fp32 in `act`;
 *   D = 4..256 (multiple of 4); past_len + M <= max_t and <= 8192. fp32 throughout. Few rows x heads
 *   (decode) split the keys over workgroups, with partials in a 4 MiB workspace the context owns:
 *   calls on one context run in its stream's order, so they never share it at the same time. */
int ql_attention_decode(ql_ctx* ctx, ql_arena* act, uint64_t q_off, const ql_arena* cache, uint64_t k_off,
                        uint64_t v_off, int32_t max_t, int32_t M, int32_t n_head, int32_t n_kv_head, int32_t D,
                        int32_t past_len, uint64_t out_off);
/* ql_plan_attention (diagnostic, host only): the launch shape ql_attention_decode picks for these
 *   dimensions, with the same checks (no counterpart in the reference, whose attention is one
 *   dispatch per layer, qwen.ts:430-442). heads_per_run query heads share each K/V row read;
 *   nsplit key splits (1 = no merge launch); workgroups of the attention launch. */
typedef struct ql_attn_info {
    int32_t heads_per_run;
    int32_t nsplit;
    int32_t workgroups;
    int32_t keys_per_split;
} ql_attn_info;
int ql_plan_attention(int32_t max_t, int32_t M, int32_t n_head, int32_t n_kv_head, int32_t D, int32_t past_len,
                      ql_attn_info* info);

/* ql_embed_f16: out[r, :] = f32(embed[tokens[r], :]) for r < rows: the embedding lookup that
 *   starts a forward (embedding_f16.wgsl, dispatched at qwen.ts:392), over the fp16 [vocab, D]
 *   table at embed_off in `weights` (the tied table ql_gemv_f16w reads as lm_head), with uint32
 *   token ids [rows] at tokens_off and the fp32 [rows, D] output at out_off in `act`. Exact
 *   (binary16 -> binary32, as f16BitsToF32, safetensors.ts:144-152). A token id >= vocab writes a
 *   row of zeros (the WGSL reads past the table there; WebGPU's robust access makes that read
 *   implementation-defined). rows 1..65535; embed 2-byte, tokens and out 4-byte aligned (D % 8 == 0
 *   with 16-byte embed/out offsets takes the 16-byte path). */
int ql_embed_f16(ql_ctx* ctx, const ql_arena* weights, uint64_t embed_off, int32_t vocab, int32_t D,
                 ql_arena* act, uint64_t tokens_off, int32_t rows, uint64_t out_off);

/* ---- the elementwise work around the linears (qwen.ts:401-405, :447-478).
 * ql_add_rmsnorm: s = x + d (misc/vec_add.wgsl: the residual add after o_proj / down_proj), stored
 *   at sum_off unless QL_NONE, then y = s * rstd * w, rstd = 1 / sqrt(mean(s^2) + eps)
 *   (norm/rmsnorm.wgsl; CPU form reference/qwen-ref.ts:12-28). d_off = QL_NONE: plain RMSNorm of x.
 *   One launch where the reference runs two; fp32; x, d, sum, y [M, C] in `act`, w [C] in
 *   `weights`; offsets 4-byte aligned (16-byte and C % 4 == 0 take the vector path). The sum may
 *   be stored in place over x or d (sum_off == x_off or d_off); any other overlap of the sum with
 *   x or d, or of y with anything, fails with QL_E_INVALID. */
int ql_add_rmsnorm(ql_ctx* ctx, ql_arena* act, uint64_t x_off, uint64_t d_off, const ql_arena* weights,
                   uint64_t w_off, float eps, int32_t M, int32_t C, uint64_t sum_off, uint64_t y_off);
/* ql_silu_mul: y[i] = (g / (1 + exp(-g))) * up[i], g = gate[i] (activation/silu_mul.wgsl;
 *   siluMulRef, qwen-ref.ts:114-121); offsets 16-byte aligned. */
int ql_silu_mul(ql_ctx* ctx, ql_arena* act, uint64_t gate_off, uint64_t up_off, int64_t n, uint64_t y_off);

/* several independent linears in one launch (e.g. q/k/v on one input, gate/up on another);
 * linear i reads x_offs[i] and writes y_offs[i]; scratch for all of them starts at scratch_off
 * (ql_plan_batch gives the size). M and x_dtype are shared; at most 8 linears. */
int ql_plan_batch(int32_t count, const ql_gptq_desc* descs, int32_t M, uint64_t* scratch_bytes);
int ql_linear_batch(ql_ctx* ctx, int32_t count, const ql_gptq_desc* descs,
                    const ql_arena* weights, ql_arena* act, const uint64_t* x_offs,
                    int32_t x_dtype, int32_t M, const uint64_t* y_offs, uint64_t scratch_off);

/* ---- linear sequences: many decode linears (M = 1..16) in ONE persistent launch.
 * Linear i reads x_offs[i] and writes y_offs[i] (fp32 [M, N_i]) in `act`. When x_offs[i] equals
 * y_offs[j] of an earlier linear j (with N_j == K_i), linear i consumes linear j's output and the
 * kernel orders the two on the device (the reference's passBreak); every other input is external
 * (x_dtype) and must not overlap any output; outputs must not overlap each other. All linears
 * share one group size (64, 128 or 256), need N % 4 == 0, and 16-byte aligned qweight, bias, x
 * and y offsets (scales 8-byte).
 * ql_seq_create validates, plans and allocates the sequence's device tables and exchange
 * buffers (the arenas are bound by address and must outlive it). ql_seq_run enqueues its launch
 * (one, except pass-by-pass sequences, below) on the context stream; it allocates nothing and
 * may be captured into a graph and replayed.
 * Runs of one sequence must not overlap (one stream). ql_seq_status waits for the stream and
 * reports whether a run was aborted (a bounded device-side wait ran out: QL_E_STATE).
 * Prefill (M = 17..65536): a sequence of independent linears (no linear reads another's output)
 * with fp16 x, N % 4 == 0 and groups a multiple of 128 runs as ONE persistent prefill GEMM
 * launch (kernel QL_SEQ_PREFILL): tasks of 128 rows x 256 columns over all of K, planned longest
 * first onto one workgroup per CU; y = f16(x) . f16(W)^T in fp32, as ql_linear's MFMA GEMM. */
#define QL_SEQ_TILES 0
#define QL_SEQ_STRIPS 1
#define QL_SEQ_PREFILL 2
#define QL_SEQ_STRIP_PASSES 3
#define QL_SEQ_PREFILL_PASSES 4
typedef struct ql_seq ql_seq;
typedef struct ql_seq_info {
    int32_t linears;
    int32_t passes;       /* dependency depth: linears that must run one after another */
    int32_t tiles;        /* GEMV tiles (64 columns x a K segment) */
    int32_t reduces;      /* split-K reductions (one per column tile of a split linear) */
    int32_t grid;         /* resident workgroups */
    int32_t max_split;    /* most parts (K pieces) of one 64-column block */
    uint64_t lds_bytes;   /* dynamic LDS per workgroup */
    uint64_t device_bytes;/* tables + exchange buffers ql_seq_create allocates */
    uint64_t total_units; /* block-groups (64 columns x one quantization group) of all linears */
    uint64_t busiest_units; /* block-groups of the most loaded workgroup: balance = busiest*grid/total */
    int32_t kernel;       /* QL_SEQ_TILES: dependency-ordered tiles; QL_SEQ_STRIPS: column strips;
                             QL_SEQ_PREFILL: prefill GEMM tiles (units: 128-k chunks);
                             QL_SEQ_STRIP_PASSES: one strip launch per pass (figures summed over
                             the passes) */
    int32_t split;        /* strips: waves per 64-column block (1: strips of 8 blocks, 2: of 4) */
    int32_t stream;       /* strips: 1 when the packed weights are read with streaming loads (the
                             weights exceed what the 256 MB MALL keeps between steps) */
    int32_t variant;      /* strips: 1 when the launch is the no-padding kernel on streamed
                             weights (every linear: group 128, K a multiple of 512, N a multiple
                             of 512; M = 5..16, or 2..16 pass by pass); QL_SEQ_PREFILL_PASSES: the
                             passes that run the chunked split-K GEMM; 0 otherwise */
    int32_t launches;     /* kernel launches one ql_seq_run enqueues */
} ql_seq_info;
/* plan only (host, pure) for a given grid size: validation and the figures above */
int ql_plan_seq(int32_t n, const ql_gptq_desc* descs, int32_t M, const uint64_t* x_offs,
                int32_t x_dtype, const uint64_t* y_offs, int32_t grid, ql_seq_info* info);
int ql_seq_create(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights,
                  ql_arena* act, const uint64_t* x_offs, int32_t x_dtype, int32_t M,
                  const uint64_t* y_offs, ql_seq** out);
int ql_seq_get_info(const ql_seq* seq, ql_seq_info* info);
int ql_seq_run(ql_ctx* ctx, ql_seq* seq);
int ql_seq_status(ql_ctx* ctx, ql_seq* seq);
/* Fused sequences (M = 1..16, fp32 x): per linear, elementwise work folded into the launch.
 *   norm_w_off  QL_NONE, or the weights-arena offset of an fp32 [K] RMSNorm weight: the linear
 *               reads rmsnorm(x) = x * rsqrt(mean(x^2) + norm_eps) * w per row (rmsNormRef)
 *               instead of x;
 *   x2_off      QL_NONE, or the activation-arena offset of an fp32 [M, K] second operand: the
 *               linear reads silu(x) * x2 (siluMulRef) instead of x; like x_offs it is another
 *               linear's output when it equals that linear's y offset, else external;
 *   res_off     QL_NONE, or the activation-arena offset of an fp32 [M, N] residual added to the
 *               linear's output (y = W.x + bias + res); another linear's output when it equals
 *               that linear's y offset, else external.
 * norm and x2 exclude each other. A linear runs after every producer it reads (x, x2 or res).
 * A fused sequence runs as dependency-ordered tiles (QL_SEQ_TILES) in one launch, except as
 * below. ql_plan_seq_fused and ql_seq_create_fused with fuse == NULL behave as ql_plan_seq and
 * ql_seq_create.
 * Chained sequences (fused or not) at M = 2..16 with fp32 x whose weights exceed what the MALL
 * keeps (192 MiB) and whose linears all have groups of 128, K % 512 == 0, K >= 1024 and
 * N % 512 == 0 run pass by pass instead (QL_SEQ_STRIP_PASSES): ql_seq_run enqueues, per pass,
 * the pass's column-strip launch (every strip cut into K parts of whole 512-k chunks, each part's
 * sums stored apart; each linear's activations formed as they are staged: as is, times an
 * RMSNorm weight, or SiLU-mul of two producers) and one launch that adds each linear's parts in a
 * fixed order, times the row's 1/rms for an RMSNorm'd input, with bias and residual (and the row
 * sums of squares of outputs a later linear RMSNorms); an external input that is RMSNorm'd adds
 * one launch before its pass. Stream order replaces the device-side waits (nothing can abort).
 * QL_SEQ_PASSES=0 in the environment keeps the tiles. */
typedef struct ql_seq_fuse {
    uint64_t norm_w_off;
    uint64_t x2_off;
    uint64_t res_off;
    float norm_eps;
    int32_t reserved;
} ql_seq_fuse;
int ql_plan_seq_fused(int32_t n, const ql_gptq_desc* descs, int32_t M, const uint64_t* x_offs,
                      int32_t x_dtype, const uint64_t* y_offs, const ql_seq_fuse* fuse, int32_t grid,
                      ql_seq_info* info);
int ql_seq_create_fused(ql_ctx* ctx, int32_t n, const ql_gptq_desc* descs, const ql_arena* weights,
                        ql_arena* act, const uint64_t* x_offs, int32_t x_dtype, int32_t M,
                        const uint64_t* y_offs, const ql_seq_fuse* fuse, ql_seq** out);
/* diagnostic: polls a device-side wait makes before aborting the run (default 4M, min 64) */
int ql_seq_set_spin_limit(ql_seq* seq, uint32_t polls);
int ql_seq_destroy(ql_seq* seq);

/* ---- ordering and timing on the context stream */
int ql_sync(ql_ctx* ctx);
int ql_timer_start(ql_ctx* ctx);
int ql_timer_stop(ql_ctx* ctx, float* elapsed_ms); /* waits for the stop event */

/* ---- stream capture into a HIP graph (one replayable submit per forward). */
int ql_graph_begin(ql_ctx* ctx);
int ql_graph_end(ql_ctx* ctx, ql_graph** out);
int ql_graph_launch(ql_ctx* ctx, ql_graph* graph);
int ql_graph_destroy(ql_graph* graph);

#ifdef __cplusplus
}
#endif
#endif /* QLINEAR_H */
