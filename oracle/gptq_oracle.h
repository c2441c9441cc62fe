/*
 * CPU oracle for the GPTQ int4 quantized-linear path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU path (intplusplus/webllm, TypeScript).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this.
 * The product library (libqlinear.so) never links or calls it.
 *
 * Each function names the reference file:line it restates, and how it is pinned
 * (tests/test_oracle_*.py):
 *   orc_f32_to_f16_bits   src/gpu/buffer.ts:57-100        exhaustive 2^32 vs F16C hardware RNE
 *   orc_f16_bits_to_f32   src/weights/safetensors.ts:144  exhaustive 2^16 vs numpy float16
 *   orc_dequant_gptq_int4 src/weights/quant.ts:42-118     reference KAT (tests/qwen/weights.ts:62-137),
 *                                                         numpy brute force, invariants, error classes
 *   orc_gemm_nt           src/reference/qwen-ref.ts:126   numpy float64 matmul, hand cases
 *   orc_gptq_linear_cols  (the same, column subset, threaded) bit-identical to orc_gptq_linear
 *   orc_plan_gemv_split   src/model/qwen.ts:61-74         documented table qwen.ts:54-59 + brute force
 *   orc_check_tolerance   src/reference/cpu-ref.ts:27-47  hand cases
 *   orc_rng_*             src/reference/cpu-ref.ts:57-67  xorshift32 closed form in Python ints
 *   orc_random_f32        src/reference/cpu-ref.ts:50-54  closed form over Python-int xorshift + numpy f32
 *   orc_normal_next       src/model/init.ts:36-52         numpy float64 Box-Muller (1 ulp), moments
 */
#ifndef GPTQ_ORACLE_H
#define GPTQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error classes of dequantizeGptqInt4's validation, in the order quant.ts checks them. */
enum {
    ORC_OK = 0,
    ORC_E_BITS = -1,          /* quant.ts:46  bits != 4                    */
    ORC_E_GROUP = -2,         /* quant.ts:47  groupSize <= 0               */
    ORC_E_DIMS = -3,          /* quant.ts:48  in/out <= 0                  */
    ORC_E_QWEIGHT_SHORT = -4, /* quant.ts:58  qweight byteLength too small */
    ORC_E_SCALES_SHORT = -5,  /* quant.ts:62  scales length too small      */
    ORC_E_QZEROS_SHORT = -6,  /* quant.ts:69  qzeros byteLength too small  */
    ORC_E_GROUP_PACK = -7     /* quant.ts:76  groupSize % 8 != 0           */
};

uint16_t orc_f32_to_f16_bits(float value);
float orc_f16_bits_to_f32(uint16_t bits);
void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);
void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* Exhaustive scan: compares orc_f32_to_f16_bits with the F16C hardware conversion (IEEE RNE)
 * over all 2^32 f32 patterns. Returns mismatch counts per class (see the .c file). */
void orc_f16_exhaustive_check(uint64_t counts[4]);

int orc_dequant_gptq_int4(const uint8_t* qweight, size_t qweight_bytes,
                          const uint8_t* qzeros, size_t qzeros_bytes, /* qzeros may be NULL */
                          const float* scales, size_t n_scales,
                          int in_features, int out_features, int group_size, int bits,
                          float* out /* [out_features, in_features] */);

/* dequant with raw f16 scales, followed by f32->f16 encoding: the uploaded fp16 [N,K] arena. */
int orc_dequant_gptq_int4_f16(const uint8_t* qweight, size_t qweight_bytes,
                              const uint8_t* qzeros, size_t qzeros_bytes,
                              const uint16_t* scales_f16, size_t n_scales,
                              int in_features, int out_features, int group_size,
                              uint16_t* out /* [N,K] f16 bits */);

void orc_gemm_nt(const float* A, const float* W, int M, int N, int K, const float* bias, float* C);

/* rmsNormRef (qwen-ref.ts:12-28) after an optional residual add; siluMulRef (:114-121). */
void orc_add_rmsnorm(const float* x, const float* d, const float* w, int rows, int D, double eps, float* s_out,
                     float* out);
void orc_silu_mul(const float* gate, const float* up, size_t n, float* out);

/* attentionGqaRef (qwen-ref.ts:65-111) over a KV cache: q [M,H,D], caches [past+M, KV*D]. */
int orc_attention_gqa_cache(const float* q, const float* kc, const float* vc, int M, int H, int KV, int D,
                            int past, float* out);

/* Fused CPU reference for one GPTQ linear: dequant (as quant.ts) then gemmNTRef, row by row,
 * so memory stays O(K) instead of O(N*K). Bit-identical to orc_dequant + orc_gemm_nt. */
int orc_gptq_linear(const uint8_t* qweight, const uint8_t* qzeros, const uint16_t* scales_f16,
                    const float* bias, const float* x, int M, int K, int N, int group_size,
                    float* y);

/* orc_gptq_linear for the output columns cols[0..ncols) only (y [M, ncols]), on `threads` threads;
 * each output bit-identical to orc_gptq_linear's. For checking full-size launches quickly.
 * w_f16: each weight rounded to fp16 first (f32ToF16Bits, the uploaded arena), so the result is
 * gemmNTRef over the fp16 weights, the operand of the reference's M > 1 GEMM. */
int orc_gptq_linear_cols(const uint8_t* qweight, const uint8_t* qzeros, const uint16_t* scales_f16,
                         const float* bias, const float* x, int M, int K, int N, int group_size,
                         const int32_t* cols, int ncols, int threads, int w_f16, float* y);

int orc_plan_gemv_split(int wg_n, int K);

int orc_check_tolerance(const float* got, const float* ref, size_t n, double atol, double rtol,
                        double* max_abs, double* max_rel);

uint32_t orc_rng_step(uint32_t* state);
double orc_rng_next(uint32_t* state);
void orc_rng_seed(uint32_t* state, uint32_t seed);
/* randomF32 (cpu-ref.ts:50-54) and makeNormal's Box-Muller (model/init.ts:36-52) over makeRng */
void orc_random_f32(uint32_t* state, size_t n, float* out);
double orc_normal_next(uint32_t* state, double* spare, int* has_spare);

#ifdef __cplusplus
}
#endif
#endif
