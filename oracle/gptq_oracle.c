/*
 * CPU oracle for the GPTQ int4 quantized-linear path — TEST INFRASTRUCTURE ONLY.
 * Restates the reference's CPU path (intplusplus/webllm TypeScript) in plain C.
 * Used by tests/ and by bench.py's cpu_baseline leg as the checker; never by the product.
 * Citations are to files under the reference checkout.
 */
#include "gptq_oracle.h"

#include <immintrin.h>
#include <pthread.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* src/gpu/buffer.ts:57-100 f32ToF16Bits: binary16 round-to-nearest-even with subnormals,
 * overflow to Inf, any NaN -> 0x7e00. Note buffer.ts:71 returns a signed zero for every
 * |value| < 2^-24 (unbiased exponent < -24), so values in (2^-25, 2^-24) become 0 where IEEE
 * RNE gives the smallest subnormal 0x0001. This quirk is reproduced, not corrected. */
uint16_t orc_f32_to_f16_bits(float value)
{
    if (value != value) return 0x7e00;                       /* buffer.ts:61 */
    const uint32_t bits = f32_bits(value);
    const uint32_t sign = (bits & 0x80000000u) >> 16;        /* buffer.ts:66 */
    const uint32_t exp = (bits & 0x7f800000u) >> 23;
    const uint32_t mant = bits & 0x007fffffu;
    if (exp == 0xff) return (uint16_t)(sign | (mant != 0 ? 0x7e00 : 0x7c00)); /* :69 */
    int e = (int)exp - 127;                                  /* :71 */
    if (e > 15) return (uint16_t)(sign | 0x7c00);            /* :72 */
    if (e < -24) return (uint16_t)sign;                      /* :73 */
    if (e < -14) {                                           /* :75-84 subnormal half */
        const uint32_t m = mant | 0x00800000u;
        const int shift = -(e + 1);
        uint32_t half = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half & 1u) != 0)) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = mant >> 13;                              /* :87-99 normal half */
    const uint32_t rem = mant & 0x1fffu;
    const uint32_t halfway = 0x1000u;
    if (rem > halfway || (rem == halfway && (half & 1u) != 0)) {
        half++;
        if (half == 0x400u) {
            half = 0;
            e++;
            if (e > 15) return (uint16_t)(sign | 0x7c00);
        }
    }
    return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | half);
}

/* src/weights/safetensors.ts:144-152 f16BitsToF32: exact decode (subnormal = mant*2^-24). */
float orc_f16_bits_to_f32(uint16_t bits)
{
    const double sign = (bits & 0x8000u) ? -1.0 : 1.0;
    const unsigned exp = (bits >> 10) & 0x1fu;
    const unsigned mant = bits & 0x03ffu;
    if (exp == 0) return (float)(sign * (double)mant * ldexp(1.0, -24));
    if (exp == 31) return mant == 0 ? (float)(sign * INFINITY) : NAN;
    return (float)(sign * (1.0 + (double)mant / 1024.0) * ldexp(1.0, (int)exp - 15));
}

void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n)
{
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16_bits(src[i]);
}

void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n)
{
    for (size_t i = 0; i < n; i++) dst[i] = orc_f16_bits_to_f32(src[i]);
}

/* counts[0]: all mismatches against the F16C conversion (IEEE RNE, imm 0);
 * counts[1]: mismatches inside the (2^-25, 2^-24) flush quirk (exp field 102, mant != 0);
 * counts[2]: mismatches on NaN inputs (payload/sign: the reference always gives 0x7e00);
 * counts[3]: any other mismatch (must be zero). */
__attribute__((target("f16c")))
void orc_f16_exhaustive_check(uint64_t counts[4])
{
    uint64_t c0 = 0, c1 = 0, c2 = 0, c3 = 0;
    uint32_t u = 0;
    do {
        const float f = bits_f32(u);
        const uint16_t ref = orc_f32_to_f16_bits(f);
        const uint16_t hw = (uint16_t)_cvtss_sh(f, 0);
        if (ref != hw) {
            c0++;
            const uint32_t exp = (u >> 23) & 0xffu;
            const uint32_t mant = u & 0x7fffffu;
            if (exp == 102 && mant != 0 && ref == ((u >> 16) & 0x8000u) && hw == (ref | 1u)) c1++;
            else if (f != f) c2++;
            else c3++;
        }
        u++;
    } while (u != 0);
    counts[0] = c0; counts[1] = c1; counts[2] = c2; counts[3] = c3;
}

static uint32_t rd_u32le(const uint8_t* p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Validation of src/weights/quant.ts:44-79, same order and classes. */
static int validate(size_t qweight_bytes, const uint8_t* qzeros, size_t qzeros_bytes,
                    size_t n_scales, int in_f, int out_f, int group, int bits)
{
    if (bits != 4) return ORC_E_BITS;                                   /* :46 */
    if (group <= 0) return ORC_E_GROUP;                                 /* :47 */
    if (in_f <= 0 || out_f <= 0) return ORC_E_DIMS;                     /* :48 */
    const size_t pack_rows = ((size_t)in_f + 7) / 8;                    /* :54 */
    const size_t pack_cols = ((size_t)out_f + 7) / 8;                   /* :55 */
    const size_t groups = ((size_t)in_f + group - 1) / (size_t)group;   /* :56 */
    if (qweight_bytes < pack_rows * (size_t)out_f * 4) return ORC_E_QWEIGHT_SHORT; /* :58 */
    if (n_scales < groups * (size_t)out_f) return ORC_E_SCALES_SHORT;   /* :62 */
    if (qzeros && qzeros_bytes < groups * pack_cols * 4) return ORC_E_QZEROS_SHORT; /* :69 */
    if (group % 8 != 0) return ORC_E_GROUP_PACK;                        /* :76 */
    return ORC_OK;
}

/* src/weights/quant.ts:42-118 dequantizeGptqInt4. Output [out_features, in_features] f32. */
int orc_dequant_gptq_int4(const uint8_t* qweight, size_t qweight_bytes,
                          const uint8_t* qzeros, size_t qzeros_bytes,
                          const float* scales, size_t n_scales,
                          int in_f, int out_f, int group, int bits, float* out)
{
    const int rc = validate(qweight_bytes, qzeros, qzeros_bytes, n_scales, in_f, out_f, group, bits);
    if (rc != ORC_OK) return rc;
    const int pack_rows = (in_f + 7) / 8;
    const int pack_cols = (out_f + 7) / 8;
    const int symmetric_zero = 1 << (bits - 1);                          /* :74 */
    for (int pr = 0; pr < pack_rows; pr++) {                             /* :83 */
        const int row_base = pr * 8;
        const int g = row_base / group;                                  /* :87 */
        for (int o = 0; o < out_f; o++) {                                /* :90 */
            const uint32_t word = rd_u32le(qweight + ((size_t)pr * out_f + o) * 4);
            const float scale = scales[(size_t)g * out_f + o];           /* :93 */
            int zero;
            if (qzeros) {                                                /* :96-100 stored zero + 1 */
                const uint32_t zw = rd_u32le(qzeros + ((size_t)g * pack_cols + o / 8) * 4);
                zero = (int)((zw >> (4 * (o % 8))) & 15u) + 1;
            } else {
                zero = symmetric_zero;
            }
            float* row = out + (size_t)o * in_f;
            for (int k = 0; k < 8; k++) {                                /* :107-113 */
                const int i = row_base + k;
                if (i >= in_f) break;
                const int q = (int)((word >> (4 * k)) & 15u);
                row[i] = (float)((double)(q - zero) * (double)scale);
            }
        }
    }
    return ORC_OK;
}

/* Loader composition: readTensorF32 (F16 scales, safetensors.ts:180-182) -> dequantizeGptqInt4
 * -> writeF16 (buffer.ts:103-120). Evaluated per element, which is the same function. */
int orc_dequant_gptq_int4_f16(const uint8_t* qweight, size_t qweight_bytes,
                              const uint8_t* qzeros, size_t qzeros_bytes,
                              const uint16_t* scales_f16, size_t n_scales,
                              int in_f, int out_f, int group, uint16_t* out)
{
    const int rc = validate(qweight_bytes, qzeros, qzeros_bytes, n_scales, in_f, out_f, group, 4);
    if (rc != ORC_OK) return rc;
    const int pack_rows = (in_f + 7) / 8;
    const int pack_cols = (out_f + 7) / 8;
    for (int pr = 0; pr < pack_rows; pr++) {
        const int g = (pr * 8) / group;
        for (int o = 0; o < out_f; o++) {
            const uint32_t word = rd_u32le(qweight + ((size_t)pr * out_f + o) * 4);
            const float scale = orc_f16_bits_to_f32(scales_f16[(size_t)g * out_f + o]);
            int zero = 8;
            if (qzeros) {
                const uint32_t zw = rd_u32le(qzeros + ((size_t)g * pack_cols + o / 8) * 4);
                zero = (int)((zw >> (4 * (o % 8))) & 15u) + 1;
            }
            uint16_t* row = out + (size_t)o * in_f;
            for (int k = 0; k < 8; k++) {
                const int i = pr * 8 + k;
                if (i >= in_f) break;
                const int q = (int)((word >> (4 * k)) & 15u);
                row[i] = orc_f32_to_f16_bits((float)((double)(q - zero) * (double)scale));
            }
        }
    }
    return ORC_OK;
}

/* src/reference/qwen-ref.ts:126-145 gemmNTRef: C[m,n] = f32(sum_k A[m,k]*W[n,k] (+bias[n])),
 * accumulated in double (JS number) in ascending k. f32*f32 products are exact in double. */
void orc_gemm_nt(const float* A, const float* W, int M, int N, int K, const float* bias, float* C)
{
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            const float* a = A + (size_t)m * K;
            const float* w = W + (size_t)n * K;
            for (int k = 0; k < K; k++) acc += (double)a[k] * (double)w[k];
            C[(size_t)m * N + n] = bias ? (float)(acc + (double)bias[n]) : (float)acc;
        }
    }
}

/* dequantizeGptqInt4 (raw f16 scales decoded as the loader does) followed by gemmNTRef,
 * evaluated for 16 output columns at a time so memory stays O(16*K). */
int orc_gptq_linear(const uint8_t* qweight, const uint8_t* qzeros, const uint16_t* scales_f16,
                    const float* bias, const float* x, int M, int K, int N, int group, float* y)
{
    if (M <= 0 || K <= 0 || N <= 0 || group <= 0 || group % 8 != 0) return ORC_E_DIMS;
    enum { NB = 16 };
    const int pack_cols = (N + 7) / 8;
    float* w = (float*)malloc(sizeof(float) * (size_t)NB * K);
    if (!w) return ORC_E_DIMS;
    for (int n0 = 0; n0 < N; n0 += NB) {
        const int nb = (N - n0) < NB ? (N - n0) : NB;
        for (int i = 0; i < K; i++) {
            const int pr = i / 8, k = i % 8, g = i / group;
            for (int j = 0; j < nb; j++) {
                const int o = n0 + j;
                const uint32_t word = rd_u32le(qweight + ((size_t)pr * N + o) * 4);
                int zero = 8;
                if (qzeros) {
                    const uint32_t zw = rd_u32le(qzeros + ((size_t)g * pack_cols + o / 8) * 4);
                    zero = (int)((zw >> (4 * (o % 8))) & 15u) + 1;
                }
                const float scale = orc_f16_bits_to_f32(scales_f16[(size_t)g * N + o]);
                const int q = (int)((word >> (4 * k)) & 15u);
                w[(size_t)j * K + i] = (float)((double)(q - zero) * (double)scale);
            }
        }
        for (int m = 0; m < M; m++) {
            const float* a = x + (size_t)m * K;
            for (int j = 0; j < nb; j++) {
                const float* wr = w + (size_t)j * K;
                double acc = 0.0;
                for (int i = 0; i < K; i++) acc += (double)a[i] * (double)wr[i];
                const int o = n0 + j;
                y[(size_t)m * N + o] = bias ? (float)(acc + (double)bias[o]) : (float)acc;
            }
        }
    }
    free(w);
    return ORC_OK;
}

/* src/model/qwen.ts:42-44 (GEMV_SPLIT_TARGET_WG=256, GEMV_SPLIT_MAX=64) and :61-74 planGemvSplit. */
int orc_plan_gemv_split(int wg_n, int K)
{
    if (wg_n >= 256) return 1;
    static const int cands[4] = {8, 16, 32, 64};
    int s = 1;
    for (int i = 0; i < 4; i++) {
        const int c = cands[i];
        if (K % c == 0 && (K / c) % 2 == 0) {
            s = c;
            if (wg_n * c >= 256) break;
        }
    }
    return s;
}

/* src/reference/cpu-ref.ts:27-47 checkTolerance: pass iff |g-r| <= atol + rtol*|r| for all i. */
int orc_check_tolerance(const float* got, const float* ref, size_t n, double atol, double rtol,
                        double* max_abs, double* max_rel)
{
    int ok = 1;
    double ma = 0.0, mr = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double diff = fabs((double)got[i] - (double)ref[i]);
        if (diff > atol + rtol * fabs((double)ref[i])) ok = 0;
        if (diff > ma) ma = diff;
        const double den = fabs((double)ref[i]) > 1e-30 ? fabs((double)ref[i]) : 1e-30;
        const double rel = diff / den;
        if (rel > mr) mr = rel;
    }
    if (max_abs) *max_abs = ma;
    if (max_rel) *max_rel = mr;
    return ok;
}

/* src/reference/cpu-ref.ts:57-67 makeRng: xorshift32 (13, 17, 5), seed 0 -> 1, value / 2^32. */
void orc_rng_seed(uint32_t* state, uint32_t seed) { *state = seed ? seed : 1u; }

uint32_t orc_rng_step(uint32_t* state)
{
    uint32_t s = *state;
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    *state = s;
    return s;
}

double orc_rng_next(uint32_t* state) { return (double)orc_rng_step(state) / 4294967296.0; }

/* src/reference/cpu-ref.ts:50-54 randomF32 with makeRng: out[i] = f32(rng() * 2 - 1), the double
 * rng() * 2 - 1 being exact and rounded to f32 by the Float32Array store. */
void orc_random_f32(uint32_t* state, size_t n, float* out)
{
    for (size_t i = 0; i < n; i++) out[i] = (float)(orc_rng_next(state) * 2.0 - 1.0);
}

/* src/model/init.ts:36-52 makeNormal (Box-Muller over makeRng): draws u, v in (0, 1) skipping
 * zeros, returns r*cos(2*pi*v) and keeps r*sin(2*pi*v) as the next value, r = sqrt(-2 ln u).
 * double throughout, as JS numbers; Math.log/sin/cos may differ from libm in the last ulp. */
double orc_normal_next(uint32_t* state, double* spare, int* has_spare)
{
    if (*has_spare) {
        *has_spare = 0;
        return *spare;
    }
    double u = 0.0, v = 0.0;
    while (u == 0.0) u = orc_rng_next(state);
    while (v == 0.0) v = orc_rng_next(state);
    const double r = sqrt(-2.0 * log(u));
    const double angle = 2.0 * 3.141592653589793 * v;     /* Math.PI */
    *spare = r * sin(angle);
    *has_spare = 1;
    return r * cos(angle);
}

/* attentionGqaRef (src/reference/qwen-ref.ts:65-111) with the cache's positions
 * (attention_gqa_cache.wgsl): query row m of q [M, H, D] sits at position past + m and sees keys
 * 0 .. past + m of the caches kc / vc [>= past + M, KV * D]. JS arithmetic kept: the dot product,
 * max, exp and sum in double; scores stored in a Float32Array (rounded at each store);
 * p_s = f32(f32(e_s) / sum); out = f32(sum_s p_s * v_s) accumulated in double. */
int orc_attention_gqa_cache(const float* q, const float* kc, const float* vc, int M, int H, int KV, int D,
                            int past, float* out)
{
    if (M <= 0 || H <= 0 || KV <= 0 || D <= 0 || past < 0 || H % KV) return ORC_E_DIMS;
    const double scale = 1.0 / sqrt((double)D);
    const int group = H / KV, row_len = KV * D;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(past + M));
    if (!scores) return ORC_E_DIMS;
    for (int h = 0; h < H; h++) {
        const int kvh = h / group;
        for (int m = 0; m < M; m++) {
            const int t = past + m;
            const float* qv = q + ((size_t)m * H + h) * D;
            double max_score = -INFINITY;
            for (int s = 0; s <= t; s++) {
                const float* kr = kc + (size_t)s * row_len + (size_t)kvh * D;
                double dot = 0.0;
                for (int d = 0; d < D; d++) dot += (double)qv[d] * (double)kr[d];
                dot *= scale;
                scores[s] = (float)dot;
                if (dot > max_score) max_score = dot;
            }
            double sum = 0.0;
            for (int s = 0; s <= t; s++) {
                const double e = exp((double)scores[s] - max_score);
                scores[s] = (float)e;
                sum += e;
            }
            for (int s = 0; s <= t; s++) scores[s] = (float)((double)scores[s] / sum);
            float* o = out + ((size_t)m * H + h) * D;
            for (int d = 0; d < D; d++) {
                double acc = 0.0;
                for (int s = 0; s <= t; s++)
                    acc += (double)scores[s] * (double)vc[(size_t)s * row_len + (size_t)kvh * D + d];
                o[d] = (float)acc;
            }
        }
    }
    free(scores);
    return 0;
}

/* rmsNormRef (src/reference/qwen-ref.ts:12-28) after the residual add of vec_add.wgsl:
 * s = f32(x + d) (d may be NULL), sum of s^2 in double, rstd = 1 / sqrt(sum / D + eps) in double,
 * out = f32(s * rstd * w) evaluated left to right in double. */
void orc_add_rmsnorm(const float* x, const float* d, const float* w, int rows, int D, double eps, float* s_out,
                     float* out)
{
    for (int r = 0; r < rows; r++) {
        const size_t base = (size_t)r * D;
        double sum = 0.0;
        for (int i = 0; i < D; i++) {
            const float v = d ? x[base + i] + d[base + i] : x[base + i];
            if (s_out) s_out[base + i] = v;
            sum += (double)v * (double)v;
        }
        const double rstd = 1.0 / sqrt(sum / D + eps);
        for (int i = 0; i < D; i++) {
            const float v = d ? x[base + i] + d[base + i] : x[base + i];
            out[base + i] = (float)((double)v * rstd * (double)w[i]);
        }
    }
}

/* siluMulRef (qwen-ref.ts:114-121): out = f32((g / (1 + exp(-g))) * u) in double. */
void orc_silu_mul(const float* gate, const float* up, size_t n, float* out)
{
    for (size_t i = 0; i < n; i++) {
        const double g = gate[i];
        out[i] = (float)((g / (1.0 + exp(-g))) * (double)up[i]);
    }
}

/* orc_gptq_linear over a subset of output columns, on several threads: the same arithmetic as
 * orc_gptq_linear per output (weights dequantized as quant.ts:83-115, dot product accumulated
 * in double in ascending k as qwen-ref.ts:135-141, one rounding to f32), so every output it
 * computes is bit-identical to orc_gptq_linear's. Columns are dealt to threads in chunks of 16;
 * y is [M, ncols], column j holding output cols[j]. */
typedef struct {
    const uint8_t* qweight; const uint8_t* qzeros; const uint16_t* scales; const float* bias;
    const float* x; int M, K, N, group; const int32_t* cols; int ncols; float* y;
    int w_f16;    /* weights rounded to fp16 as the uploaded arena (f32ToF16Bits), the GEMM's operand */
    int next; pthread_mutex_t lock; int rc;
} cols_job;

static void* cols_worker(void* arg)
{
    cols_job* J = (cols_job*)arg;
    enum { NB = 16 };
    const int K = J->K, N = J->N, M = J->M;
    const int pack_cols = (N + 7) / 8;
    float* w = (float*)malloc(sizeof(float) * (size_t)NB * K);
    if (!w) { pthread_mutex_lock(&J->lock); J->rc = ORC_E_DIMS; pthread_mutex_unlock(&J->lock); return NULL; }
    for (;;) {
        pthread_mutex_lock(&J->lock);
        const int c0 = J->next;
        J->next += NB;
        pthread_mutex_unlock(&J->lock);
        if (c0 >= J->ncols) break;
        const int nb = (J->ncols - c0) < NB ? (J->ncols - c0) : NB;
        for (int j = 0; j < nb; j++) {
            const int o = J->cols[c0 + j];
            float* wr = w + (size_t)j * K;
            for (int pr = 0; pr * 8 < K; pr++) {
                const uint32_t word = rd_u32le(J->qweight + ((size_t)pr * N + o) * 4);
                for (int k = 0; k < 8 && pr * 8 + k < K; k++) {
                    const int i = pr * 8 + k, g = i / J->group;
                    int zero = 8;
                    if (J->qzeros) {
                        const uint32_t zw = rd_u32le(J->qzeros + ((size_t)g * pack_cols + o / 8) * 4);
                        zero = (int)((zw >> (4 * (o % 8))) & 15u) + 1;
                    }
                    const float scale = orc_f16_bits_to_f32(J->scales[(size_t)g * N + o]);
                    const int q = (int)((word >> (4 * k)) & 15u);
                    wr[i] = (float)((double)(q - zero) * (double)scale);
                    if (J->w_f16) wr[i] = orc_f16_bits_to_f32(orc_f32_to_f16_bits(wr[i]));
                }
            }
        }
        for (int m = 0; m < M; m++) {
            const float* a = J->x + (size_t)m * K;
            int j = 0;
            for (; j + 4 <= nb; j += 4) {     /* four independent chains, each in ascending k */
                const float *w0 = w + (size_t)j * K, *w1 = w0 + K, *w2 = w1 + K, *w3 = w2 + K;
                double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
                for (int i = 0; i < K; i++) {
                    const double xv = (double)a[i];
                    a0 += xv * (double)w0[i];
                    a1 += xv * (double)w1[i];
                    a2 += xv * (double)w2[i];
                    a3 += xv * (double)w3[i];
                }
                const double acc[4] = {a0, a1, a2, a3};
                for (int t = 0; t < 4; t++) {
                    const int o = J->cols[c0 + j + t];
                    J->y[(size_t)m * J->ncols + c0 + j + t] =
                        J->bias ? (float)(acc[t] + (double)J->bias[o]) : (float)acc[t];
                }
            }
            for (; j < nb; j++) {
                const float* wr = w + (size_t)j * K;
                double acc = 0.0;
                for (int i = 0; i < K; i++) acc += (double)a[i] * (double)wr[i];
                const int o = J->cols[c0 + j];
                J->y[(size_t)m * J->ncols + c0 + j] = J->bias ? (float)(acc + (double)J->bias[o]) : (float)acc;
            }
        }
    }
    free(w);
    return NULL;
}

int orc_gptq_linear_cols(const uint8_t* qweight, const uint8_t* qzeros, const uint16_t* scales_f16,
                         const float* bias, const float* x, int M, int K, int N, int group_size,
                         const int32_t* cols, int ncols, int threads, int w_f16, float* y)
{
    if (M <= 0 || K <= 0 || N <= 0 || group_size <= 0 || group_size % 8 != 0 || ncols < 0)
        return ORC_E_DIMS;
    for (int j = 0; j < ncols; j++)
        if (cols[j] < 0 || cols[j] >= N) return ORC_E_DIMS;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    cols_job J = {qweight, qzeros, scales_f16, bias, x, M, K, N, group_size, cols, ncols, y, w_f16,
                  0, PTHREAD_MUTEX_INITIALIZER, ORC_OK};
    pthread_t tid[64];
    int started = 0;
    for (int t = 1; t < threads; t++) {
        if (pthread_create(&tid[started], NULL, cols_worker, &J) != 0) break;
        started++;
    }
    cols_worker(&J);
    for (int t = 0; t < started; t++) pthread_join(tid[t], NULL);
    return J.rc;
}
