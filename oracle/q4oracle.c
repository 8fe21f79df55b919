/*
 * q4oracle.c - CPU restatement of the reference's q4g32a.t64 quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. The product library (p0pc0rn_amd/) never links, loads or calls this file. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker / the timed CPU port.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference repository).
 * Pinning of each function (tests/test_oracle.py):
 *   p0o_f2h / p0o_h2f      exhaustive and edge-case comparison with numpy float16 (IEEE RNE, the textbook routine)
 *   p0o_rng_uniform/randn  known-answer values computed by hand from the xorshift recurrence; Box-Muller moments
 *   p0o_pack_q4            decode of its bytes by the kernels' word/nibble rule (independent of the packer's byte rule),
 *                          |deq - W| <= s/2, code range, fp16 scale/min recorded, symmetric data round-trips exactly
 *   p0o_dequant_q4         equals packQ4's own dequantized output bit for bit; fp16 tile = numpy float16 of it
 *   p0o_q4_gemv/gemvM/gemm numpy float64 matmul of the dequantized matrix (textbook routine); split partials sum to the
 *                          unsplit value; gemvM row m == gemv on row m; geglu/softcap/argmax against numpy closed forms
 *   p0o_q4_gemm branches   (tests/test_gemm_oracle.py) numpy closed forms on data far from zero mean: the lnmod
 *                          prologue's centring and its shift base with a negative, wrapped stride; rms; bf16 -> fp16
 *                          round-to-nearest-even; resadd's gate x (acc + bias) in store and accumulate form; the bias
 *                          epilogue rounding once; swiglu's interleaved gate/up rows; the heads epilogue (per-head
 *                          QK-RMSNorm, both RoPE modes, head-major fp16 rows) and a variant without norm or rotation
 *                          that must differ
 *   p0o_lgemv_f32/gemm_f32 within fp32 rounding of the float64 results above
 */
#include "q4oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ fp16 helpers */
/* engine/core/gpu.js:274-289: f32 -> f16 bits, round to nearest even, subnormals, Inf, NaN -> quiet 0x7e00 */
uint16_t p0o_f2h(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
  uint32_t sign = (x >> 16) & 0x8000u, e = (x >> 23) & 0xffu, m = x & 0x7fffffu;
  if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
  int ne = (int)e - 112;
  if (ne >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (ne <= 0) {
    if (ne < -10) return (uint16_t)sign;
    m |= 0x800000u;
    int sh = 14 - ne;
    uint32_t hm = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t r = sign | ((uint32_t)ne << 10) | (m >> 13), rem2 = m & 0x1fffu;
  if (rem2 > 0x1000u || (rem2 == 0x1000u && (r & 1u))) r++;
  return (uint16_t)r;
}

/* engine/core/gpu.js:290-295 */
float p0o_h2f(uint16_t h) {
  double s = (h & 0x8000u) ? -1.0 : 1.0;
  int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) return (float)(s * m * 5.960464477539063e-8);
  if (e == 31) return m ? NAN : (float)(s * INFINITY);
  return (float)(s * (1.0 + m / 1024.0) * ldexp(1.0, e - 15));
}

void p0o_f2h_n(const float* in, uint16_t* out, int64_t n) { for (int64_t i = 0; i < n; i++) out[i] = p0o_f2h(in[i]); }
void p0o_h2f_n(const uint16_t* in, float* out, int64_t n) { for (int64_t i = 0; i < n; i++) out[i] = p0o_h2f(in[i]); }
static inline float rf16(double x) { return p0o_h2f(p0o_f2h((float)x)); }   /* kcheck.js:12: double -> f32 -> f16 */

/* ------------------------------------------------------------------------------------------------ RNG */
/* engine/kcheck.js:10. JS evaluates `s >> 17` on the int32 view of s (arithmetic shift), so the high bits fill with the
 * sign bit; this is restated as written rather than as the textbook logical-shift xorshift32. */
void p0o_rng_uniform(uint32_t seed, double* out, int64_t n) {
  uint32_t s = seed ? seed : 1u;
  for (int64_t i = 0; i < n; i++) {
    s ^= s << 13;
    s ^= (uint32_t)(((int32_t)s) >> 17);
    s ^= s << 5;
    out[i] = (double)s / 4294967296.0;
  }
}

/* engine/kcheck.js:11: Box-Muller in float64, stored as float32 */
void p0o_randn(uint32_t seed, double scale, float* out, int64_t n) {
  int64_t nu = n + (n & 1);
  double* u = (double*)malloc(sizeof(double) * (size_t)nu);
  p0o_rng_uniform(seed, u, nu);
  double sc = scale;
  for (int64_t i = 0; i < n; i += 2) {
    double uu = u[i] > 1e-9 ? u[i] : 1e-9, v = u[i + 1], m = sqrt(-2.0 * log(uu)) * sc;
    out[i] = (float)(m * cos(2.0 * M_PI * v));
    if (i + 1 < n) out[i + 1] = (float)(m * sin(2.0 * M_PI * v));
  }
  free(u);
}

/* ------------------------------------------------------------------------------------------------ packQ4 */
static double rhe(double x) {   /* engine/kcheck.js:14 round half to even */
  double f = floor(x), d = x - f;
  return d > 0.5 ? f + 1 : d < 0.5 ? f : (fmod(f, 2.0) == 0.0 ? f : f + 1);
}

/* engine/kcheck.js:22-38 */
void p0o_pack_q4(const float* W, int64_t N, int64_t K, uint8_t* out, float* deq) {
  int64_t NT = N / 64, G = K / 32;
  for (int64_t t = 0; t < NT; t++)
    for (int64_t g = 0; g < G; g++) {
      uint8_t* rec = out + (t * G + g) * 1280;
      for (int r = 0; r < 64; r++) {
        int64_t n = t * 64 + r, base = n * K + g * 32;
        double mnv = INFINITY, mxv = -INFINITY;
        for (int i = 0; i < 32; i++) {
          double v = W[base + i];
          if (v < mnv) mnv = v;
          if (v > mxv) mxv = v;
        }
        double mn = rf16(mnv), s = rf16((mxv - mn) / 15.0);
        if (s == 0) s = 1;
        for (int j = 0; j < 16; j++) {
          double q0 = fmin(15, fmax(0, rhe((W[base + 2 * j] - mn) / s)));
          double q1 = fmin(15, fmax(0, rhe((W[base + 2 * j + 1] - mn) / s)));
          rec[r * 16 + j] = (uint8_t)((int)q0 | ((int)q1 << 4));
          if (deq) {
            deq[base + 2 * j] = (float)(q0 * s + mn);
            deq[base + 2 * j + 1] = (float)(q1 * s + mn);
          }
        }
        uint32_t sm = (uint32_t)p0o_f2h((float)s) | ((uint32_t)p0o_f2h((float)mn) << 16);
        memcpy(rec + 1024 + r * 4, &sm, 4);   /* little-endian host, as DataView.setUint32(.., true) */
      }
    }
}

/* packQ8 (engine/kcheck.js:39-52): per (row, 64-group) s = fl16(absmax / 127) (1 if 0), q = clamp(rhe(w / s), -128, 127);
 * record (tile, group) = 4224 bytes: row r's 64 int8 codes at 64 r (k order), fp16 scales at 4096 + 2 r */
void p0o_pack_q8(const float* W, int64_t N, int64_t K, uint8_t* out, float* deq) {
  const int64_t NT = N / 64, G = K / 64;
  for (int64_t t = 0; t < NT; t++)
    for (int64_t g = 0; g < G; g++) {
      uint8_t* rec = out + (t * G + g) * 4224;
      for (int r = 0; r < 64; r++) {
        const int64_t n = t * 64 + r, base = n * K + g * 64;
        double am = 0;
        for (int i = 0; i < 64; i++) am = fmax(am, fabs((double)W[base + i]));
        float s = rf16(am / 127.0);
        if (s == 0.0f) s = 1.0f;
        for (int i = 0; i < 64; i++) {
          double q = rhe((double)W[base + i] / (double)s);
          q = q < -128 ? -128 : q > 127 ? 127 : q;
          rec[r * 64 + i] = (uint8_t)((int)q & 255);
          if (deq) deq[base + i] = (float)(q * s);
        }
        const uint16_t h = p0o_f2h(s);
        memcpy(rec + 4096 + r * 2, &h, 2);
      }
    }
}

/* ------------------------------------------------------------------------------------------------ dequant */
static inline uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }

/* engine/llm/lops.js:67-71 (word w of row r: nibble i is k = 32g + 8w + i; u32 256 + r = f16 scale | f16 min << 16)
 * and engine/ops/gemm.js:139-149 (fp16 tile value = fl16(fl32(q * s + m))) */
static inline float deq_one(const uint8_t* w, int64_t wG, int64_t n, int64_t k) {
  const uint8_t* rec = w + (((n >> 6) * wG + (k >> 5)) * 1280);
  int r = (int)(n & 63), i = (int)(k & 31);
  uint32_t word = rd32(rec + r * 16 + (i >> 3) * 4), sm = rd32(rec + 1024 + r * 4);
  float q = (float)((word >> (4 * (i & 7))) & 15u);
  float s = p0o_h2f((uint16_t)(sm & 0xffffu)), m = p0o_h2f((uint16_t)(sm >> 16));
  volatile float qs = q * s;   /* exact (4-bit times 11-bit significands) */
  return qs + m;               /* one f32 rounding */
}

/* engine/llm/lops.js:74-80: q8g64s.t64 record (tile, k / 64); byte (r, k % 64) is a signed code; word 1024 + r / 2
 * holds the fp16 scales of rows 2j (low half) and 2j + 1; the weight is q s, exact in f32 (8 x 11 bits) */
static inline float deq_one_q8(const uint8_t* w, int64_t wG, int64_t n, int64_t k) {
  const uint8_t* rec = w + (((n >> 6) * wG + (k >> 6)) * 4224);
  const int r = (int)(n & 63);
  const int8_t q = (int8_t)rec[r * 64 + (k & 63)];
  uint16_t h;
  memcpy(&h, rec + 4096 + r * 2, 2);
  return (float)q * p0o_h2f(h);
}
void p0o_dequant_q8(const uint8_t* w, int64_t N, int64_t K, int64_t wG, float* out32) {
  for (int64_t n = 0; n < N; n++)
    for (int64_t k = 0; k < K; k++) out32[n * K + k] = deq_one_q8(w, wG, n, k);
}

void p0o_dequant_q4(const uint8_t* w, int64_t N, int64_t K, int64_t wG, float* out32, uint16_t* out16) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++)
    for (int64_t k = 0; k < K; k++) {
      float v = deq_one(w, wG, n, k);
      if (out32) out32[n * K + k] = v;
      if (out16) out16[n * K + k] = p0o_f2h(v);
    }
}

/* ------------------------------------------------------------------------------------------------ synthetic data */
/* The PCG RXS-M-XS output hash of a 32-bit counter (M. Jarzynski, M. Olano, "Hash Functions for GPU Rendering",
 * JCGT 9(3), 2020) - the same published hash the reference's GPU filler uses (engine/tune/autotune.js:76). */
uint32_t p0o_hash(uint32_t x) {
  uint32_t v = x * 747796405u + 2891336453u;
  uint32_t w = ((v >> ((v >> 28) + 4u)) ^ v) * 277803737u;
  return (w >> 22) ^ w;
}
static inline double u01(uint32_t h) { return ((double)(h >> 8) + 0.5) * (1.0 / 16777216.0); }   /* (0, 1) */
static inline double hnorm(uint32_t idx, uint32_t seed) {   /* Box-Muller from two hashed uniforms, float64 */
  double a = u01(p0o_hash((2u * idx) ^ seed)), b = u01(p0o_hash((2u * idx + 1u) ^ seed ^ 0x9E3779B9u));
  return sqrt(-2.0 * log(a)) * cos(6.283185307179586 * b);
}

/* The BASELINE symmetric weights in q4g32a.t64: code word i (counting only code words, record-major) = hash(i ^ seed),
 * scale of (tile, group, row) j = fl16(|N(0, sigma)|) from hnorm(j, seed'), min = -8 * scale (exact in fp16).
 * Mirrored bit for bit by p0_fill_q4_sym on the device (codes; scales up to libm rounding of log/cos in float64). */
void p0o_fill_q4_sym(uint8_t* w, int64_t N, int64_t K, uint32_t seed, float sigma) {
  int64_t nrec = (N / 64) * (K / 32);
#pragma omp parallel for schedule(static)
  for (int64_t rc = 0; rc < nrec; rc++) {
    uint8_t* rec = w + rc * 1280;
    for (int j = 0; j < 256; j++) {
      uint32_t h = p0o_hash((uint32_t)(rc * 256 + j) ^ seed);
      memcpy(rec + 4 * j, &h, 4);
    }
    for (int r = 0; r < 64; r++) {
      double z = hnorm((uint32_t)(rc * 64 + r), seed ^ 0x5bd1e995u);
      uint16_t sh = p0o_f2h((float)(fabs(z) * (double)sigma));
      uint16_t mh = p0o_f2h(-8.0f * p0o_h2f(sh));
      uint32_t sm = (uint32_t)sh | ((uint32_t)mh << 16);
      memcpy(rec + 1024 + 4 * r, &sm, 4);
    }
  }
}

/* fp16-valued N(0, sigma) activations: out16 = fl16(z * sigma), out32 = the same value as f32 */
void p0o_fill_randn(float* out32, uint16_t* out16, int64_t n, uint32_t seed, float sigma) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) {
    uint16_t h = p0o_f2h((float)(hnorm((uint32_t)i, seed) * (double)sigma));
    if (out16) out16[i] = h;
    if (out32) out32[i] = p0o_h2f(h);
  }
}

/* ------------------------------------------------------------------------------------------------ GEMV / GEMV-M */
/* engine/llm/lops.js:26 (tanh GELU, argument clamped to +-15) */
static inline float gelu_f(float v) {
  double d = v;
  return (float)(d * 0.5 * (1.0 + tanh(fmin(15.0, fmax(-15.0, 0.7978845608028654 * (d + 0.044715 * d * d * d))))));
}
static inline float softcap_f(double v, float cap) {   /* engine/llm/lops.js:96 */
  return (float)((double)cap * tanh(fmin(15.0, fmax(-15.0, v / (double)cap))));
}

static double dot_row(const uint8_t* w, int enc, int64_t wG, int64_t n, const float* xp, int64_t k0, int64_t k1) {
  double acc = 0;
  if (enc == P0_ENC_Q8G64S_T64)
    for (int64_t k = k0; k < k1; k++) acc += (double)deq_one_q8(w, wG, n, k) * (double)xp[k - k0];
  else
    for (int64_t k = k0; k < k1; k++) acc += (double)deq_one(w, wG, n, k) * (double)xp[k - k0];
  return acc;
}

/* one GEMV-M pass; gemv is M = 1 with its own argument defaults (engine/llm/lops.js:111-141 vs lops_spec.js:163-191) */
typedef struct {
  const uint8_t* w; int enc; int64_t wG;
  const float* X; int64_t ldx, rowB;
  int64_t M, N, K, kPer;
  int pro, epi;
  float* Y; int64_t ldy, ldm;
  const float* ST; int64_t statOff, statLd;
  const float* NW; int64_t nOff;
  int64_t nsrc, ldp;
  const float* EV; int64_t evOff, evLd;
  float* MX; float cap;
} gv_t;

static int run_gemv(const gv_t* p) {
  int64_t nsplit = (p->K + p->kPer - 1) / p->kPer, NT = p->N / 64;
  float* xp = (float*)malloc(sizeof(float) * (size_t)(p->kPer > 0 ? p->kPer : 1));
  double* tot = (double*)malloc(sizeof(double) * (size_t)(2 * p->N));
  for (int64_t s = 0; s < nsplit; s++) {
    int64_t k0 = s * p->kPer, k1 = k0 + p->kPer < p->K ? k0 + p->kPer : p->K;
    for (int64_t m = 0; m < p->M; m++) {
      /* prologue: engine/llm/lops.js:50-57, engine/llm/lops_spec.js:61-64 */
      for (int64_t k = k0; k < k1; k++) {
        float v;
        if (p->pro == P0_PRO_RAW) v = p->X[m * p->ldx + p->rowB + k];
        else if (p->pro == P0_PRO_RMS) v = p->X[m * p->ldx + p->rowB + k] * p->ST[p->statOff + m * p->statLd] * p->NW[p->nOff + k];
        else {
          float su = 0.f;
          for (int64_t j = 0; j < p->nsrc; j++) su += p->X[j * p->ldp + m * p->ldx + k];
          v = p->pro == P0_PRO_SUM ? su : gelu_f(su) * p->EV[p->evOff + m * p->evLd + k];
        }
        xp[k - k0] = v;
      }
      int64_t rows = p->epi == P0_EPI_GEGLU ? 2 * p->N : p->N;
#pragma omp parallel for schedule(static)
      for (int64_t n = 0; n < rows; n++) tot[n] = dot_row(p->w, p->enc, p->wG, n, xp, k0, k1);
      /* epilogues: engine/llm/lops.js:92-103, engine/llm/lops_spec.js:130-153 */
      if (p->epi == P0_EPI_STORE) {
        for (int64_t n = 0; n < p->N; n++) p->Y[s * p->ldy + m * p->ldm + n] = (float)tot[n];
      } else if (p->epi == P0_EPI_GEGLU) {
        for (int64_t n = 0; n < p->N; n++) p->Y[m * p->ldm + n] = gelu_f((float)tot[n]) * (float)tot[n + p->N];
      } else {
        for (int64_t t = 0; t < NT; t++) {
          float best = 0; uint32_t bi = 0;
          for (int r = 0; r < 64; r++) {
            int64_t n = t * 64 + r;
            float v = softcap_f((float)tot[n], p->cap);
            p->Y[m * p->ldm + n] = v;
            if (r == 0 || v > best) { best = v; bi = (uint32_t)r; }   /* ties keep the lower row */
          }
          uint32_t id = (uint32_t)(t * 64) + bi;
          p->MX[(m * NT + t) * 2] = best;
          memcpy(&p->MX[(m * NT + t) * 2 + 1], &id, 4);
        }
      }
    }
  }
  free(xp);
  free(tot);
  return (int)nsplit;
}

int p0o_q4_gemv(const p0_gemv_args_t* a) {   /* engine/llm/lops.js:111-141 */
  int64_t K = a->K, kch = (!a->kPer && K > 2048) ? ((K + 255) / 256) * 256 : 2048;
  int64_t kPer = a->kPer ? a->kPer : K;
  if (kPer > kch) kPer = kch;
  const int enc = a->w_enc == P0_ENC_Q8G64S_T64 ? P0_ENC_Q8G64S_T64 : P0_ENC_Q4G32A_T64;
  gv_t p = {(const uint8_t*)a->w + a->w_off, enc, a->w_cols / (enc == P0_ENC_Q8G64S_T64 ? 64 : 32), a->x, 0, a->x_rowB, 1,
            a->N, K, kPer, a->pro, a->epi, a->y,
            a->ldy ? a->ldy : a->N, 0, a->epi == P0_EPI_SOFTCAP ? a->mx : a->stat, a->stat_off, 0, a->norm, a->norm_off,
            a->src_n, a->src_ld, a->ev, a->ev_off, 0, a->mx, a->cap != 0.f ? a->cap : 30.f};
  return run_gemv(&p);
}

int p0o_q4_gemvM(const p0_gemvm_args_t* a) {   /* engine/llm/lops_spec.js:163-191 */
  int64_t K = a->K, kPer = a->kPer ? (a->kPer < 2048 ? a->kPer : 2048) : K;
  int64_t ldm = a->y_ldm ? a->y_ldm : a->N, ldy = a->y_ldy ? a->y_ldy : a->M * ldm;
  const int enc = a->w_enc == P0_ENC_Q8G64S_T64 ? P0_ENC_Q8G64S_T64 : P0_ENC_Q4G32A_T64;
  gv_t p = {(const uint8_t*)a->w + a->w_off, enc, a->w_cols / (enc == P0_ENC_Q8G64S_T64 ? 64 : 32), a->x,
            a->x_ldx ? a->x_ldx : K, a->x_rowB, a->M, a->N, K, kPer,
            a->pro, a->epi, a->y, ldy, ldm, a->stat, a->stat_off, a->stat_ld ? a->stat_ld : 2, a->norm, a->norm_off,
            a->src_n ? a->src_n : 1, a->src_ld, a->ev, a->ev_off, a->ev_ld, a->mx, a->cap != 0.f ? a->cap : 30.f};
  return run_gemv(&p);
}

/* ------------------------------------------------------------------------------------------------ GEMM */
static inline float bf16_to_f32(uint16_t b) { uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return f; }

/* engine/ops/gemm.js:55-63 (x prologues), :94-97 (wrow), :139-149 (tile dequant), :187-211 (epilogues) */
/* the heads epilogue of one output row m (engine/ops/gemm.js:212-250): for each 128-wide head h, sec = 0 (query,
 * h < Hq), 1 (key, h < Hq + Hkv) or 2 (value). Query and key heads: v = acc * inv * nw[c] with inv = 1 / sqrt(mean of
 * acc^2 over the head + eps) and nw at ev_off (+ 128 for keys), then RoPE from the table row rowOff + m: 'inter' rotates
 * the pair (2p, 2p + 1) by entry p (:241-244), 'half' the pair (d, d + 64) by entry d (:237-239). Every head is stored
 * as fp16 at ((h * Ltot) + rowOff + m) * 128 + c (:240, :245). */
static void heads_row(const p0_gemm_args_t* a, const float* acc, int64_t m, uint8_t* yb) {
  const int64_t H = a->N / 128, row = a->heads_row_off + m;
  const double eps = a->heads_eps != 0.0f ? (double)a->heads_eps : 1e-6;
  const float* rp = a->rope + row * 128;
  for (int64_t h = 0; h < H; h++) {
    const float* v = acc + h * 128;
    const int sec = h < a->heads_hq ? 0 : h < a->heads_hq + a->heads_hkv ? 1 : 2;
    double out[128];
    if (sec == 2) {
      for (int c = 0; c < 128; c++) out[c] = v[c];
    } else {
      double ss = 0, t[128];
      for (int c = 0; c < 128; c++) ss += (double)v[c] * v[c];
      const float inv = (float)(1.0 / sqrt(ss / 128.0 + eps));
      const float* nw = a->ev + a->ev_off + (sec ? 128 : 0);
      for (int c = 0; c < 128; c++) t[c] = (double)v[c] * inv * nw[c];
      if (a->heads_rope == P0_ROPE_HALF) {
        for (int d = 0; d < 64; d++) {
          const double cs = rp[2 * d], sn = rp[2 * d + 1];
          out[d] = t[d] * cs - t[d + 64] * sn;
          out[d + 64] = t[d + 64] * cs + t[d] * sn;
        }
      } else {
        for (int q = 0; q < 64; q++) {
          const double cs = rp[2 * q], sn = rp[2 * q + 1];
          out[2 * q] = t[2 * q] * cs - t[2 * q + 1] * sn;
          out[2 * q + 1] = t[2 * q] * sn + t[2 * q + 1] * cs;
        }
      }
    }
    for (int c = 0; c < 128; c++) {
      const uint16_t hv = p0o_f2h((float)out[c]);
      memcpy(yb + 2 * ((h * a->heads_ltot + row) * 128 + c), &hv, 2);
    }
  }
}

int p0o_q4_gemm(const p0_gemm_args_t* a) {
  int64_t M = a->M, N = a->N, K = a->K, ldx = a->x_ld ? a->x_ld : K, ldy = a->y_ld ? a->y_ld : N;
  int64_t wG = a->w_cols / 32, Nw = a->w_rows;
  const uint8_t* w = (const uint8_t*)a->w + a->w_off;
  const uint8_t* xb = (const uint8_t*)a->x + a->x_off;
  uint8_t* yb = (uint8_t*)a->y + a->y_off;
  int xf32 = a->x_mode == P0_XMODE_LNMOD || a->x_mode == P0_XMODE_RMS;
  uint32_t shiftBase = (uint32_t)(a->pv_off + a->pv_stride);   /* u32 wrap, as the reference's uniform */
  float* acc = (float*)malloc(sizeof(float) * (size_t)N);
  float* xr = (float*)malloc(sizeof(float) * (size_t)K);
  /* the fp16 tile value of every weight the call reads, once: wt[n][k] = fl16(deq32(W[wrow(n)][wk0 + k])) */
  float* wt = (float*)malloc(sizeof(float) * (size_t)(N * K));
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    int64_t row = a->epi == P0_GEPI_SWIGLU ? ((n & 1) ? a->wr1 : a->wr0) + (n >> 1)
                                            : (a->wr0 + n < Nw - 1 ? a->wr0 + n : Nw - 1);
    for (int64_t k = 0; k < K; k++) wt[n * K + k] = rf16(deq_one(w, wG, row, a->wk0 + k));
  }
  for (int64_t m = 0; m < M; m++) {
    for (int64_t k = 0; k < K; k++) {
      int64_t idx = m * ldx + a->x_k0 + k;
      float v;
      if (!xf32) {
        uint16_t h;
        memcpy(&h, xb + 2 * idx, 2);
        v = a->x_mode == P0_XMODE_BF16 ? rf16(bf16_to_f32(h)) : p0o_h2f(h);
      } else {
        float x;
        memcpy(&x, xb + 4 * idx, 4);
        const float* st = a->stats + (a->stats_off + m) * 2;
        int64_t kk = a->x_k0 + k;
        float t = a->x_mode == P0_XMODE_LNMOD ? (x - st[0]) * st[1] * (1.0f + a->pv[a->pv_off + kk]) + a->pv[shiftBase + kk]
                                              : x * st[1] * a->pv[a->pv_off + kk];
        v = rf16(t);
      }
      xr[k] = v;
    }
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++) {
      const float* wr = wt + n * K;
      double s = 0;
      for (int64_t k = 0; k < K; k++) s += (double)xr[k] * (double)wr[k];
      acc[n] = (float)s;
    }
    if (a->epi == P0_GEPI_HEADS) {   /* engine/ops/gemm.js:212-250 */
      heads_row(a, acc, m, yb);
      continue;
    }
    for (int64_t n = 0; n < N; n++) {
      int64_t o = m * ldy + a->y_n0;
      if (a->epi == P0_GEPI_F16) {
        uint16_t h = p0o_f2h(acc[n]);
        memcpy(yb + 2 * (o + n), &h, 2);
      } else if (a->epi == P0_GEPI_F32) {
        memcpy(yb + 4 * (o + n), &acc[n], 4);
      } else if (a->epi == P0_GEPI_RESADD) {
        float g = a->ev ? a->ev[a->ev_off + n] : 1.0f, b = a->bv ? a->bv[a->bv_off + n] : 0.0f, prev = 0;
        if (!a->store) memcpy(&prev, yb + 4 * (o + n), 4);
        float r = a->store ? g * (acc[n] + b) : prev + g * (acc[n] + b);
        memcpy(yb + 4 * (o + n), &r, 4);
      } else if (a->epi == P0_GEPI_BIAS) {
        float r = acc[n] + a->ev[a->ev_off + n];
        if (a->res) { uint16_t h; memcpy(&h, yb + 2 * (o + n), 2); r += p0o_h2f(h); }
        uint16_t h = p0o_f2h(r);
        memcpy(yb + 2 * (o + n), &h, 2);
      } else if (a->epi == P0_GEPI_SWIGLU && !(n & 1)) {
        int64_t j = n >> 1;
        float gB = a->bv ? a->bv[a->bv_off + j] : 0.f, uB = a->bv ? a->bv[a->bv_off + a->bv_up + j] : 0.f;
        double g = (double)(acc[n] + gB), u = (double)(acc[n + 1] + uB), act;
        if (a->act == P0_ACT_GELU) act = g * 0.5 * (1.0 + tanh(fmin(15.0, fmax(-15.0, 0.7978845608 * (g + 0.044715 * g * g * g)))));
        else act = g / (1.0 + exp(-g));
        uint16_t h = p0o_f2h((float)(act * u));
        memcpy(yb + 2 * (o + j), &h, 2);
      }
    }
  }
  free(acc);
  free(xr);
  free(wt);
  return 0;
}

/* ------------------------------------------------------------------------------------------------ CPU baselines */
int p0o_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* engine/llm/lops.js:60-88: thread (r, w) sums s * (qa.a + qb.b) + m * (sum a + sum b) over the groups, then the four
 * quarter sums of a row are added in lane order. fp32 throughout. */
void p0o_lgemv_f32(const uint8_t* w, int64_t wG, const float* x, int64_t N, int64_t K, float* y, int threads) {
  int64_t G = K / 32;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (int64_t n = 0; n < N; n++) {
    const uint8_t* tb = w + (n >> 6) * wG * 1280;
    int r = (int)(n & 63);
    float q4[4] = {0, 0, 0, 0};
    for (int qw = 0; qw < 4; qw++) {
      float acc = 0.f;
      for (int64_t g = 0; g < G; g++) {
        const uint8_t* rec = tb + g * 1280;
        uint32_t q = rd32(rec + r * 16 + qw * 4), sm = rd32(rec + 1024 + r * 4);
        float s = p0o_h2f((uint16_t)(sm & 0xffffu)), mn = p0o_h2f((uint16_t)(sm >> 16));
        const float* xa = x + g * 32 + qw * 8;
        float da = (float)(q & 15u) * xa[0] + (float)((q >> 4) & 15u) * xa[1] + (float)((q >> 8) & 15u) * xa[2] +
                   (float)((q >> 12) & 15u) * xa[3];
        float db = (float)((q >> 16) & 15u) * xa[4] + (float)((q >> 20) & 15u) * xa[5] + (float)((q >> 24) & 15u) * xa[6] +
                   (float)((q >> 28) & 15u) * xa[7];
        float sa = xa[0] + xa[1] + xa[2] + xa[3], sb = xa[4] + xa[5] + xa[6] + xa[7];
        acc = acc + s * (da + db) + mn * (sa + sb);
      }
      q4[qw] = acc;
    }
    y[n] = q4[0] + q4[1] + q4[2] + q4[3];
  }
}

/* engine/ops/gemm.js:139-185: fp16 weight and x tiles, fp32 FMA accumulation in k order */
void p0o_gemm_f32(const uint8_t* w, int64_t wG, const uint16_t* x16, int64_t M, int64_t N, int64_t K, float* y,
                  int threads) {
  float* wt = (float*)malloc(sizeof(float) * (size_t)(N * K));
#pragma omp parallel for schedule(static) num_threads(threads)
  for (int64_t n = 0; n < N; n++)
    for (int64_t k = 0; k < K; k++) wt[n * K + k] = rf16(deq_one(w, wG, n, k));
#pragma omp parallel for schedule(static) num_threads(threads)
  for (int64_t m = 0; m < M; m++) {
    float* xr = (float*)malloc(sizeof(float) * (size_t)K);
    for (int64_t k = 0; k < K; k++) xr[k] = p0o_h2f(x16[m * K + k]);
    for (int64_t n = 0; n < N; n++) {
      const float* wr = wt + n * K;
      float acc = 0.f;
      for (int64_t k = 0; k < K; k++) acc = fmaf(xr[k], wr[k], acc);
      y[m * N + n] = acc;
    }
    free(xr);
  }
  free(wt);
}

/* ---- rowstats / normadd / argmax --------------------------------------------------------------------------------- */
/* the reference's 256-lane reduction: lane t sums elements t, t + 256, ... in turn (engine/ops/misc.js:26-27), then
 * level s = 128, 64, ..., 1 adds lane t + s into lane t (engine/ops/misc.js:20-23) */
static float tree256(const float* part) {
  float red[256];
  memcpy(red, part, sizeof red);
  for (int s = 128; s > 0; s >>= 1)
    for (int t = 0; t < s; ++t) red[t] = red[t] + red[t + s];
  return red[0];
}
static float rsqrt_cr(float v) { return 1.0f / sqrtf(v); }

void p0o_rowstats(const p0_rowstats_args_t* a) {   /* engine/ops/misc.js:17-30 */
  const int64_t ld = a->x_ld ? a->x_ld : a->cols;
  const float* x = (const float*)((const uint8_t*)a->x + a->x_off);
  for (int64_t r = 0; r < a->rows; ++r) {
    const float* xr = x + r * ld + a->x_c0;
    float part[256], mean = 0.0f;
    if (a->mode == 0) {
      for (int t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (int64_t i = t; i < a->cols; i += 256) s = s + xr[i];
        part[t] = s;
      }
      mean = tree256(part) / (float)a->cols;
    }
    for (int t = 0; t < 256; ++t) {
      float q = 0.0f;
      for (int64_t i = t; i < a->cols; i += 256) {
        const float d = xr[i] - mean;
        q = q + d * d;
      }
      part[t] = q;
    }
    const float var = tree256(part) / (float)a->cols;
    a->st[(a->st_off + r) * 2] = mean;
    a->st[(a->st_off + r) * 2 + 1] = rsqrt_cr(var + a->eps);
  }
}

void p0o_normadd(const p0_normadd_args_t* a) {   /* engine/llm/lops.js:153-170, defaults of :175-177 */
  const int64_t D = a->D, M = a->M ? a->M : 1, nsrc = a->t_n ? a->t_n : 1, ldp = a->t_ld ? a->t_ld : D * M;
  const float eps = a->eps != 0.0f ? a->eps : 1e-6f;
  float* tv = (float*)malloc((size_t)D * sizeof(float));
  float part[256];
  for (int64_t m = 0; m < M; ++m) {
    const int64_t xb = m * D;
    for (int t = 0; t < 256; ++t) {
      float s = 0.0f;
      for (int64_t i = t; i < D; i += 256) {
        float v = 0.0f;
        for (int64_t j = 0; j < nsrc; ++j) v = v + a->t[j * ldp + xb + i];
        tv[i] = v;
        s = s + v * v;
      }
      part[t] = s;
    }
    const float rs = rsqrt_cr(tree256(part) / (float)D + eps);
    for (int t = 0; t < 256; ++t) {
      float s2 = 0.0f;
      for (int64_t i = t; i < D; i += 256) {
        float x = a->x[xb + i];
        if (a->mode == 0) x = (x + tv[i] * rs * a->w[a->w_off + i]) * a->scale;
        else x = tv[i];
        a->x[xb + i] = x;
        s2 = s2 + x * x;
      }
      part[t] = s2;
    }
    a->st[a->st_off + m] = rsqrt_cr(tree256(part) / (float)D + eps);
  }
  free(tv);
}

/* engine/llm/lops_spec.js:333-343 (argmax is the M = 1 case, engine/llm/lops.js:422-432): lane t keeps the best of
 * pairs t, t + 256, ..., then the halving tree; larger value wins, ties go to the lower index */
void p0o_argmaxM(const float* mx, int64_t n, int64_t M, uint32_t* out) {
  for (int64_t m = 0; m < M; ++m) {
    float rv[256];
    uint32_t ri[256];
    for (int t = 0; t < 256; ++t) {
      float bv = -3.4e38f;
      uint32_t bi = 0xFFFFFFFFu;
      for (int64_t i = t; i < n; i += 256) {
        const float v = mx[2 * (m * n + i)];
        uint32_t id;
        memcpy(&id, &mx[2 * (m * n + i) + 1], 4);
        if (v > bv || (v == bv && id < bi)) { bv = v; bi = id; }
      }
      rv[t] = bv;
      ri[t] = bi;
    }
    for (int s = 128; s > 0; s >>= 1)
      for (int t = 0; t < s; ++t)
        if (rv[t + s] > rv[t] || (rv[t + s] == rv[t] && ri[t + s] < ri[t])) { rv[t] = rv[t + s]; ri[t] = ri[t + s]; }
    out[2 * m] = ri[0];
    memcpy(&out[2 * m + 1], &rv[0], 4);
  }
}
