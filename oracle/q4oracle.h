/*
 * q4oracle.h - CPU restatement of the reference's q4g32a.t64 arithmetic. TEST INFRASTRUCTURE ONLY: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, as the checker; the product library never
 * links or calls it. Argument structs are the C ABI's own (include/p0pc0rn.h), with HOST pointers.
 */
#ifndef Q4ORACLE_H
#define Q4ORACLE_H
#include <stdint.h>
#include <stddef.h>
#include "../include/p0pc0rn.h"

#ifdef __cplusplus
extern "C" {
#endif

uint16_t p0o_f2h(float v);                 /* engine/core/gpu.js:274-289 */
float p0o_h2f(uint16_t h);                 /* engine/core/gpu.js:290-295 */
void p0o_f2h_n(const float* in, uint16_t* out, int64_t n);
void p0o_h2f_n(const uint16_t* in, float* out, int64_t n);

/* xorshift32 uniform stream and Box-Muller randn, engine/kcheck.js:10-11 */
void p0o_rng_uniform(uint32_t seed, double* out, int64_t n);
void p0o_randn(uint32_t seed, double scale, float* out, int64_t n);

/* packQ4 (engine/kcheck.js:22-38): W [N][K] f32 -> records (N/64 * K/32 * 1280 B) + the exact dequantized f32 */
void p0o_pack_q4(const float* W, int64_t N, int64_t K, uint8_t* bytes, float* deq);
/* packQ8 (engine/kcheck.js:39-52): W [N][K] f32 -> q8g64s.t64 records (N/64 * K/64 * 4224 B) + the exact dequant */
void p0o_pack_q8(const float* W, int64_t N, int64_t K, uint8_t* bytes, float* deq);
/* q8g64s.t64 record reader (engine/llm/lops.js:74-80): q * s, [N][K] */
void p0o_dequant_q8(const uint8_t* w, int64_t N, int64_t K, int64_t wG, float* out32);
/* record reader (engine/llm/lops.js:67-71, engine/ops/gemm.js:139-149): fl32(q*s+m) and fl16 of it, [N][K] */
void p0o_dequant_q4(const uint8_t* w, int64_t N, int64_t K, int64_t wG, float* out32, uint16_t* out16);

/* symmetric synthetic records (the same counter hash as p0_fill_q4_sym) */
uint32_t p0o_hash(uint32_t x);
void p0o_fill_q4_sym(uint8_t* w, int64_t N, int64_t K, uint32_t seed, float sigma);
void p0o_fill_randn(float* out32, uint16_t* out16, int64_t n, uint32_t seed, float sigma);

/* reference results (float64 dot over the exact dequantized weights, of either encoding, w_enc); returns the number of
 * splits */
int p0o_q4_gemv(const p0_gemv_args_t* a);      /* engine/llm/lops.js:30-141 */
int p0o_q4_gemvM(const p0_gemvm_args_t* a);    /* engine/llm/lops_spec.js:44-191 */
int p0o_q4_gemm(const p0_gemm_args_t* a);      /* engine/ops/gemm.js:25-322 */

/* the CPU baseline: lgemv's own fp32 summation order (4 quarter-lanes of 8 k per row, summed in order),
 * engine/llm/lops.js:60-88, raw prologue, store epilogue, rows split over `threads` OpenMP threads */
void p0o_lgemv_f32(const uint8_t* w, int64_t wG, const float* x, int64_t N, int64_t K, float* y, int threads);
/* the CPU baseline of the dequant-GEMM: fp16 tiles, fp32 FMA in k order (engine/ops/gemm.js:139-185) */
void p0o_gemm_f32(const uint8_t* w, int64_t wG, const uint16_t* x16, int64_t M, int64_t N, int64_t K, float* y,
                  int threads);
int p0o_max_threads(void);

/* the GEMV's producer and consumers, in the reference's own fp32 summation order (256 strided partial sums, then a
 * halving tree): rowstats (engine/ops/misc.js:13-40), normadd (engine/llm/lops.js:143-178), argmax / argmaxM
 * (engine/llm/lops.js:416-436, engine/llm/lops_spec.js:327-348). Host pointers, the C ABI's argument structs. */
void p0o_rowstats(const p0_rowstats_args_t* a);
void p0o_normadd(const p0_normadd_args_t* a);
void p0o_argmaxM(const float* mx, int64_t n, int64_t M, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
