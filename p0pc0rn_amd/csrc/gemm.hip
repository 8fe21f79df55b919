// gemm.hip - q4g32a.t64 dequant-GEMM on gfx950 MFMA: Y[m, n] = sum_k X'[m, k] * fl16(fl32(q s + m))[n, k].
//
// Replaces the WebGPU dispatch of gemm (engine/ops/gemm.js:255-322) for the q4 encoding, with its prologues
// f16 | lnmod | rms (engine/ops/gemm.js:55-63; plus bf16 activations converted to fp16) and epilogues
// f16 | f32 | resadd | swiglu | bias | heads (engine/ops/gemm.js:187-250).
//
// Two kernels:
//  * x_stage_kernel<XM> writes X' (the prologue-applied activations, fp16, dense rows of K) into the context's staging
//    workspace, once per call, when X is not already fp16 rows the MFMA kernel can stream (bf16, lnmod, rms, or fp16
//    rows that are not 16-byte aligned). The reference applies the prologue inside its tile loads; doing it once here
//    instead of once per output-column block costs one streaming pass over X.
//  * q4_gemm_kernel: a workgroup of 8 waves owns a 256 x 256 output tile; per 64-k step (two q4 groups) it
//      - streams the fp16 X tile straight from global memory into LDS (global_load_lds_dwordx4: no registers, no ALU),
//      - dequantises the W tile from its records exactly (fl16 of the fp32 value, the reference's own tile rounding,
//        engine/ops/gemm.js:147-148) into LDS,
//      - runs 4 x 2 blocks of v_mfma_f32_32x32x16_f16 per wave over its 128 x 64 sub-tile (fp32 accumulators),
//    with two LDS stages: the next step's X loads and the next-but-one step's W records are in flight during this
//    step's MFMAs, issued a few at a time between them (the step's memory work is paced over its MFMAs). LDS rows are
//    128 B (64 k); the 16-byte chunk c of row r sits at a swizzled position (swz_key), which makes the direct-load
//    writes, the dequant writes and the MFMA fragment reads all bank-conflict free.
#include "common.hpp"

namespace p0 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));   // a 16-byte load at 4-byte alignment
typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));               // 16-byte aligned (LDS, registers)
typedef float float16v __attribute__((ext_vector_type(16)));

struct GemmP {
  const uint8_t* w; int64_t wG; int64_t Nw;
  const _Float16* x; int64_t ldx;   // fp16 X' rows (the caller's, or the staging workspace), k offset folded in
  int M, N, K;
  int64_t wr0, wr1, wk0;
  int epi;
  uint8_t* y; int64_t ldy, ny0;
  const float* ev; int64_t evOff;
  const float* bv; int64_t bvOff, bvUp;
  int act, store, res;
  // heads epilogue: head-major rows of Ltot, query / key head counts, eps, RoPE mode and table
  int64_t hLtot, hRow0;
  int hq, hkv, hrope;
  float heps;
  const float* rope;
};

struct XStageP {   // the prologue of engine/ops/gemm.js:55-63 over the caller's X
  const uint8_t* x; int64_t ldx, kx0; int xmode;
  int M, K;
  const float* st; int64_t stOff;
  const float* pv; int64_t pvOff; uint32_t pvShift;   // shift base = (pv_off + pv_stride) mod 2^32
  _Float16* out;     // [M][K]
  int vec;           // rows and the k offset are 16-byte aligned: vector loads
};

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kStage = (BM + BN) * BK * 2;     // one stage: X and W tiles, 64 KB
constexpr int kGemmLds = 2 * kStage;           // two stages: 128 KB of the 160 KB

__device__ __forceinline__ _Float16 to_h(float v) { return (_Float16)v; }   // RNE
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, to_h(lo)) | ((uint32_t)__builtin_bit_cast(uint16_t, to_h(hi)) << 16);
}
// byte offset of the 16-byte chunk c (0..7) of tile row r. The position c ^ key(r) puts one logical chunk of any 8
// consecutive rows into 8 distinct positions, and of any 16 consecutive rows into distinct (row parity, position)
// pairs, so both ways an LDS can serve a 16-byte access (8 lanes x 128 B or 16 lanes x 256 B per pass) are free of bank
// conflicts (the SQ_LDS_BANK_CONFLICT counter reads 0 on MI355X; (r >> 1) & 7 read 20% of the LDS-active cycles). The key
// depends on r mod 32 only: the 32-row blocks of a wave's fragments share one offset.
__device__ __forceinline__ int swz_key(int r) { return (r ^ ((r >> 3) & 3)) & 7; }
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ swz_key(r)) << 4); }

// ------------------------------------------------------------------------------------------------ X staging
__global__ __launch_bounds__(256) void x_stage_kernel(XStageP p) {
  const int64_t chunks = (int64_t)p.M * (p.K / 8);
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (int64_t)gridDim.x * 256) {
    const int m = (int)(c / (p.K / 8)), k = (int)(c % (p.K / 8)) * 8;
    const int64_t idx = (int64_t)m * p.ldx + p.kx0 + k;
    float f[8];
    if (p.xmode == P0_XMODE_F16 || p.xmode == P0_XMODE_BF16) {
      const uint16_t* src = (const uint16_t*)p.x + idx;
      uint16_t v[8];
      if (p.vec) {
        const u32x4n d = *(const u32x4n*)src;
#pragma unroll
        for (int i = 0; i < 4; ++i) { v[2 * i] = (uint16_t)d[i]; v[2 * i + 1] = (uint16_t)(d[i] >> 16); }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = src[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        f[j] = p.xmode == P0_XMODE_F16 ? (float)__builtin_bit_cast(_Float16, v[j]) : __uint_as_float((uint32_t)v[j] << 16);
    } else {   // engine/ops/gemm.js:59-63
      const float* src = (const float*)p.x + idx;
      const float mean = p.st[(p.stOff + m) * 2], rstd = p.st[(p.stOff + m) * 2 + 1];
      const int64_t kk = p.kx0 + k;
      float xv[8];
      if (p.vec) {
        const u32x4n d0 = *(const u32x4n*)src, d1 = *(const u32x4n*)(src + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) { xv[i] = __uint_as_float(d0[i]); xv[i + 4] = __uint_as_float(d1[i]); }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[j] = src[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        f[j] = p.xmode == P0_XMODE_LNMOD
                   ? (xv[j] - mean) * rstd * (1.0f + p.pv[p.pvOff + kk + j]) + p.pv[(int64_t)p.pvShift + kk + j]
                   : xv[j] * rstd * p.pv[p.pvOff + kk + j];
    }
    u32x4n o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_h2(f[2 * i], f[2 * i + 1]);
    *(u32x4n*)(p.out + (int64_t)m * p.K + k) = o;
  }
}

// ------------------------------------------------------------------------------------------------ the GEMM
// weight row of output column n (engine/ops/gemm.js:94-97)
__device__ __forceinline__ int64_t wrow(const GemmP& p, int n) {
  if (p.epi == P0_GEPI_SWIGLU) return ((n & 1) ? p.wr1 : p.wr0) + (n >> 1);
  const int64_t r = p.wr0 + n;
  return r < p.Nw - 1 ? r : p.Nw - 1;
}

__device__ __forceinline__ float act_f(const GemmP& p, float g) {
  if (p.act == P0_ACT_GELU) {
    float t = 0.7978845608f * (g + 0.044715f * g * g * g);
    t = fminf(15.0f, fmaxf(-15.0f, t));
    return g * 0.5f * (1.0f + tanhf(t));
  }
  return g / (1.0f + __expf(-g));
}

// q s + m is exact in fp32 for every q in [0, 15] when the fp16 exponent fields a = max(e_s, 1), b = max(e_m, 1)
// satisfy -12 <= a - b <= 8 (the sum then spans at most 24 bits), or when s or m is zero
__device__ __forceinline__ bool pk_exact(uint32_t sm) {
  const int es = (sm >> 10) & 31, em = (sm >> 26) & 31;
  const int a = es > 1 ? es : 1, b = em > 1 ? em : 1;
  const bool zero = (sm & 0x7FFFu) == 0 || (sm & 0x7FFF0000u) == 0;
  return zero || (a - b <= 8 && a - b >= -12);
}

// One q4 code word (k = 8 w .. 8 w + 7 of one row) -> 8 fp16 weights in k order, each fl16(fl32(q s + m)).
// Fast path: the byte j of the word holds k 2j (low nibble) and 2j + 1 (high nibble); a byte permute spreads the
// nibbles of byte j into the two halves of pair j, OR-ing 0x6400 makes them fp16 1024 + q, v_pk_add_f16 takes 1024 off
// exactly and v_pk_fma_f16 rounds q s + m once to fp16. That single rounding equals fl16(fl32(q s + m)) whenever q s + m
// is exact in fp32 (pk_exact); otherwise the fp32 path rounds twice, exactly as the reference does.
__device__ __forceinline__ u32x4n deq_word(uint32_t v, uint32_t sm, bool fast) {
  u32x4n o;
  if (fast) {
    const h2 s2 = {__builtin_bit_cast(h2, sm).x, __builtin_bit_cast(h2, sm).x};
    const h2 m2 = {__builtin_bit_cast(h2, sm).y, __builtin_bit_cast(h2, sm).y};
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;   // byte j: k 2j | k 2j + 1
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // bytes [lo.j, 0, hi.j, 0] (selector 0x0C gives zero); then the fp16 exponent of 1024
      const uint32_t sel = (uint32_t)j | (0x0Cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0Cu << 24);
      const uint32_t b = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
      const h2 q = __builtin_bit_cast(h2, b) - k1024;
      o[j] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, s2, m2));
    }
  } else {
    const float s = (float)__builtin_bit_cast(h2, sm).x, m = (float)__builtin_bit_cast(h2, sm).y;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q0 = (float)((v >> (8 * j)) & 15u), q1 = (float)((v >> (8 * j + 4)) & 15u);
      o[j] = pack_h2(__builtin_fmaf(q0, s, m), __builtin_fmaf(q1, s, m));
    }
  }
  return o;
}

// 8 waves in 2 (M) x 4 (N), two per SIMD so that one wave's waits are covered by the other's MFMAs; each wave owns a
// 128 x 64 sub-tile as 4 x 2 blocks of 32 x 32 (128 fp32 accumulators per lane)
constexpr int kWaves = 8, kThreads = 64 * kWaves, WTM = 128, WTN = 64, IB = WTM / 32, JB = WTN / 32;
// ---- the heads epilogue (engine/ops/gemm.js:212-250): QK-RMSNorm over each 128-wide head, RoPE, head-major fp16 rows.
// A 256-wide output tile holds two whole heads (n0 is a multiple of 256): head hp of the tile is the wave pair
// wn = 2 hp (head columns 0..63) and 2 hp + 1 (64..127), in each of the two wave rows wm. acc[i][j][e] is row
// 32 i + 8 (e / 4) + e % 4 + 4 (lane / 32) of the wave's 128 and column 32 j + lane % 32 of its 64.
//  * sum of squares per row: a lane adds its two columns; per 32-row block i, a transposing butterfly over the 32 lanes
//    of each half-wave (offsets 16, 8, 4, 2: a lane keeps one half of its 16 sums and takes the partner's matching half,
//    then offset 1 adds the last pair) leaves a lane the sum of one row over the wave's 64 columns; the two waves' sums
//    of a head are added through LDS, even wave first, so both waves see the same sum;
//  * query / key heads: v = acc * inv * nw[c], inv = 1 / sqrt(sum / 128 + eps), then the rotation: 'inter' pairs the
//    columns (2p, 2p + 1), which sit in neighbouring lanes; 'half' pairs (d, d + 64), which sit in the two waves of the
//    pair, so the values cross through LDS, one block i (32 rows) per round;
//  * every head is stored fp16 at ((head Ltot) + row0 + m) 128 + c.
__device__ __forceinline__ void heads_epilogue(const GemmP& p, float16v (&acc)[WTM / 32][WTN / 32], uint8_t* lds,
                                               int m0, int n0, int wm, int wn, int lane) {
  constexpr int IBh = WTM / 32, JBh = WTN / 32;
  float* red = (float*)lds;                       // [wn][wm * 128 + row]: 4 x 256 floats
  float* xch = (float*)(lds + 4096);              // [wave][j][e][lane]: the 'half' exchange, 8 x 2 x 16 x 64 floats
  const int wv = wm * 4 + wn, hh = lane >> 5;
  __syncthreads();   // every wave has read its last fragments: the stage memory is free
#pragma unroll
  for (int i = 0; i < IBh; ++i) {
    float ss[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) ss[e] = __builtin_fmaf(acc[i][0][e], acc[i][0][e], acc[i][1][e] * acc[i][1][e]);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int o = 16 >> st, half = 8 >> st;
      const bool up = (lane & o) != 0;
#pragma unroll
      for (int k = 0; k < half; ++k) {
        const float send = up ? ss[k] : ss[k + half], keep = up ? ss[k + half] : ss[k];
        ss[k] = keep + __shfl_xor(send, o, 64);
      }
    }
    const float tot = ss[0] + __shfl_xor(ss[0], 1, 64);
    const int e = ((lane & 16) ? 8 : 0) + ((lane & 8) ? 4 : 0) + ((lane & 4) ? 2 : 0) + ((lane & 2) ? 1 : 0);
    if (!(lane & 1)) red[wn * 256 + wm * 128 + 32 * i + 8 * (e >> 2) + (e & 3) + 4 * hh] = tot;
  }
  __syncthreads();
  // when N / 128 is odd, the last column tile's second head (waves wn = 2, 3) does not exist: those waves stay in the
  // barriers, read no norm weights or RoPE entries (treated as a value head) and store nothing
  const int hd = (n0 >> 7) + (wn >> 1);
  const bool live = hd < (p.N >> 7);
  const int sec = !live ? 2 : hd < p.hq ? 0 : hd < p.hq + p.hkv ? 1 : 2;
  const int c0 = (wn & 1) * 64 + (lane & 31);   // head column of j = 0 (j = 1: + 32)
  float nw[JBh];
#pragma unroll
  for (int j = 0; j < JBh; ++j) nw[j] = sec < 2 ? p.ev[p.evOff + (sec ? 128 : 0) + c0 + 32 * j] : 1.0f;
  const float* rede = red + (wn & ~1) * 256 + wm * 128;
  const float* redo = red + (wn | 1) * 256 + wm * 128;
  _Float16* y = (_Float16*)p.y;
#pragma unroll
  for (int i = 0; i < IBh; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {   // normalised values, in place
      const int r = 32 * i + 8 * (e >> 2) + (e & 3) + 4 * hh;
      const float inv = sec < 2 ? 1.0f / sqrtf((rede[r] + redo[r]) / 128.0f + p.heps) : 1.0f;
#pragma unroll
      for (int j = 0; j < JBh; ++j) acc[i][j][e] = sec < 2 ? acc[i][j][e] * inv * nw[j] : acc[i][j][e];
    }
    float pv[JBh][16];   // the rotation partner of each value
    if (p.hrope == P0_ROPE_HALF) {
#pragma unroll
      for (int j = 0; j < JBh; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) xch[((wv * JBh + j) * 16 + e) * 64 + lane] = acc[i][j][e];
      __syncthreads();
#pragma unroll
      for (int j = 0; j < JBh; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) pv[j][e] = xch[(((wv ^ 1) * JBh + j) * 16 + e) * 64 + lane];
      __syncthreads();   // the next round rewrites the exchange area
    } else {
#pragma unroll
      for (int j = 0; j < JBh; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) pv[j][e] = __shfl_xor(acc[i][j][e], 1, 64);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + wm * WTM + 32 * i + 8 * (e >> 2) + (e & 3) + 4 * hh;
      const int64_t row = p.hRow0 + (m < p.M ? m : p.M - 1);
#pragma unroll
      for (int j = 0; j < JBh; ++j) {
        const int c = c0 + 32 * j;
        const float v = acc[i][j][e];
        float out = v;
        if (sec < 2) {
          if (p.hrope == P0_ROPE_HALF) {   // pair (d, d + 64), entry d: the low half subtracts, the high half adds
            const float* rp = p.rope + row * 128 + 2 * (c & 63);
            out = (wn & 1) ? v * rp[0] + pv[j][e] * rp[1] : v * rp[0] - pv[j][e] * rp[1];
          } else {                         // pair (2q, 2q + 1), entry q
            const float* rp = p.rope + row * 128 + (c & ~1);
            out = (c & 1) ? pv[j][e] * rp[1] + v * rp[0] : v * rp[0] - pv[j][e] * rp[1];
          }
        }
        if (live && m < p.M) y[(hd * p.hLtot + p.hRow0 + m) * 128 + c] = to_h(out);
      }
    }
  }
}


// ---- the epilogues: acc[i][j][e] is row 8 (e / 4) + 4 (lane / 32) + e % 4, column lane % 32 of
// block (i, j) of the wave's 128 x 64 sub-tile. One loop per epilogue (a uniform branch), each small enough to unroll
// completely: the accumulators stay in registers.
template <bool HEADS>
__device__ __forceinline__ void gemm_epilogue(const GemmP& p, float16v (&acc)[WTM / 32][WTN / 32], uint8_t* lds, int m0,
                                              int n0, int wm, int wn, int lane) {
  const int mb = m0 + wm * WTM + 4 * (lane >> 5), nb = n0 + wn * WTN + (lane & 31);
  // paired accesses: rows of an even number of elements, an even first column, a 4-byte aligned Y (8-byte aligned
  // for the 8-byte fp32 accesses)
  const bool pair_ok = ((p.ldy | p.ny0) & 1) == 0 && ((uintptr_t)p.y & 3) == 0;
  const bool pair8 = ((uintptr_t)p.y & 7) == 0;
#define P0_EPI_LOOP(...)                                                    \
  _Pragma("unroll") for (int i = 0; i < IB; ++i)                            \
  _Pragma("unroll") for (int j = 0; j < JB; ++j)                            \
  _Pragma("unroll") for (int e = 0; e < 16; ++e) {                          \
    const int m = mb + i * 32 + 8 * (e >> 2) + (e & 3), n = nb + j * 32;    \
    const float a = acc[i][j][e];                                           \
    const int64_t o = (int64_t)m * p.ldy + p.ny0;                           \
    __VA_ARGS__                                                             \
  }
  if (HEADS) {
    heads_epilogue(p, acc, lds, m0, n0, wm, wn, lane);
  } else if (pair_ok && p.epi != P0_GEPI_SWIGLU) {
    // lane pairs (l, l ^ 1) trade one value per pair of rows (e, e + 1): the even lane takes columns (c, c + 1) of
    // row e, the odd lane columns (c - 1, c) of row e + 1, each read and written with one access of two elements
    const bool odd = lane & 1;
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int n = nb + j * 32 - (odd ? 1 : 0);   // even: the pair's first column
        const bool n0in = n < p.N, n1in = n + 1 < p.N;
        // per-column vectors, once per block
        float g0 = 1.0f, g1 = 1.0f, b0 = 0.0f, b1 = 0.0f;
        if (p.epi == P0_GEPI_RESADD) {
          if (p.ev) { g0 = n0in ? p.ev[p.evOff + n] : 0.0f; g1 = n1in ? p.ev[p.evOff + n + 1] : 0.0f; }
          if (p.bv) { b0 = n0in ? p.bv[p.bvOff + n] : 0.0f; b1 = n1in ? p.bv[p.bvOff + n + 1] : 0.0f; }
        } else if (p.epi == P0_GEPI_BIAS) {
          b0 = n0in ? p.ev[p.evOff + n] : 0.0f;
          b1 = n1in ? p.ev[p.evOff + n + 1] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float a0 = acc[i][j][e], a1 = acc[i][j][e + 1];
          const float recv = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                 __builtin_bit_cast(int, odd ? a0 : a1), 0xB1, 0xF, 0xF, true));   // lane ^ 1
          const int m = mb + i * 32 + 8 * (e >> 2) + (e & 3) + (odd ? 1 : 0);
          const float lo = odd ? recv : a0, hi = odd ? a1 : recv;
          if (m >= p.M || !n0in) continue;
          const int64_t o = (int64_t)m * p.ldy + p.ny0 + n;
          if (p.epi == P0_GEPI_F16) {
            _Float16* yp = (_Float16*)p.y + o;
            if (n1in) *(uint32_t*)yp = pack_h2(lo, hi);
            else *yp = to_h(lo);
          } else if (p.epi == P0_GEPI_BIAS) {   // fp16 y, optionally accumulated (engine/ops/gemm.js:207-211)
            _Float16* yp = (_Float16*)p.y + o;
            if (n1in) {
              float r0 = lo + b0, r1 = hi + b1;
              if (p.res) {
                const h2 old = __builtin_bit_cast(h2, *(const uint32_t*)yp);
                r0 += (float)old.x;
                r1 += (float)old.y;
              }
              *(uint32_t*)yp = pack_h2(r0, r1);
            } else {
              float r = lo + b0;
              if (p.res) r += (float)*yp;
              *yp = to_h(r);
            }
          } else {   // f32 y (plain, or resadd: engine/ops/gemm.js:192-197), 8-byte accesses where aligned
            float* yp = (float*)p.y + o;
            float r0 = lo, r1 = hi;
            if (p.epi == P0_GEPI_RESADD) {
              r0 = g0 * (lo + b0);
              r1 = g1 * (hi + b1);
            }
            if (n1in && pair8) {
              if (p.epi == P0_GEPI_RESADD && !p.store) {
                const float2 old = *(const float2*)yp;
                r0 = old.x + r0;
                r1 = old.y + r1;
              }
              *(float2*)yp = float2{r0, r1};
            } else {
              if (p.epi == P0_GEPI_RESADD && !p.store) r0 = yp[0] + r0;
              yp[0] = r0;
              if (n1in) {
                if (p.epi == P0_GEPI_RESADD && !p.store) r1 = yp[1] + r1;
                yp[1] = r1;
              }
            }
          }
        }
      }
  } else if (p.epi == P0_GEPI_F16) {
    P0_EPI_LOOP(if (m < p.M && n < p.N) ((_Float16*)p.y)[o + n] = to_h(a);)
  } else if (p.epi == P0_GEPI_F32) {
    P0_EPI_LOOP(if (m < p.M && n < p.N) ((float*)p.y)[o + n] = a;)
  } else if (p.epi == P0_GEPI_RESADD) {   // engine/ops/gemm.js:192-197
    P0_EPI_LOOP(if (m < p.M && n < p.N) {
      const float g = p.ev ? p.ev[p.evOff + n] : 1.0f, b = p.bv ? p.bv[p.bvOff + n] : 0.0f;
      float* yp = (float*)p.y + o + n;
      *yp = p.store ? g * (a + b) : *yp + g * (a + b);
    })
  } else if (p.epi == P0_GEPI_BIAS) {
    P0_EPI_LOOP(if (m < p.M && n < p.N) {
      _Float16* yp = (_Float16*)p.y + o + n;
      float r = a + p.ev[p.evOff + n];
      if (p.res) r += (float)*yp;
      *yp = to_h(r);
    })
  } else {   // swiglu: gate = even column, up = the next one, in the neighbouring lane (engine/ops/gemm.js:200-206)
    // per pair of rows (e, e + 1) the lane pair trades one value: the even lane takes the up value of row e, the odd
    // lane the gate value of row e + 1, and each computes and stores one output (every lane busy, one activation each)
    const bool odd = lane & 1;
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int n = nb + j * 32 - (odd ? 1 : 0), jn = n >> 1;   // the pair's gate column and output column
        const bool nin = n < p.N;
        const float gB = p.bv && nin ? p.bv[p.bvOff + jn] : 0.0f, uB = p.bv && nin ? p.bv[p.bvOff + p.bvUp + jn] : 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float a0 = acc[i][j][e], a1 = acc[i][j][e + 1];
          const float recv = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                 __builtin_bit_cast(int, odd ? a0 : a1), 0xB1, 0xF, 0xF, true));   // lane ^ 1
          const float gate = odd ? recv : a0, up = odd ? a1 : recv;
          const int m = mb + i * 32 + 8 * (e >> 2) + (e & 3) + (odd ? 1 : 0);
          if (m < p.M && nin) ((_Float16*)p.y)[(int64_t)m * p.ldy + p.ny0 + jn] = to_h(act_f(p, gate + gB) * (up + uB));
        }
      }
  }
#undef P0_EPI_LOOP
}

// HEADS: the instantiation with the heads epilogue (the others' register allocation stays as it is without it)
template <bool HEADS>
__global__ __launch_bounds__(kThreads) void q4_gemm_kernel(GemmP p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 2, wn = wv & 3;

  // XCD-aware tile order: consecutive workgroups go to the 8 XCDs in turn, so tile t is given to workgroup
  // (t % per) * 8 + t / per: each XCD walks a contiguous run of row-major tiles and keeps their X rows in its L2
  const int nbx = (p.N + BN - 1) / BN, nby = (p.M + BM - 1) / BM, T = nbx * nby;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (blockIdx.x % 8) * (T / 8) + blockIdx.x / 8;
  const int m0 = (t / nbx) * BM, n0 = (t % nbx) * BN;

  float16v acc[IB][JB];
#pragma unroll
  for (int i = 0; i < IB; ++i)
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // X direct loads: instruction r of wave wv fills tile rows wv * 32 + 8 r .. + 7 (1 KB); lane l lands at byte 16 l,
  // i.e. row wv * 32 + 8 r + l / 8, position l % 8, which must hold logical chunk (l % 8) ^ key(row)
  const _Float16* xsrc[4];
  int xk[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int trow = wv * 32 + 8 * r + (lane >> 3);
    const int row = min(m0 + trow, p.M - 1);   // rows past M repeat the last row (never stored)
    xk[r] = ((lane & 7) ^ swz_key(trow)) << 3;
    xsrc[r] = p.x + (int64_t)row * p.ldx + xk[r];
  }
  // W: thread -> (row tid % 256 of the tile, group tid / 256 of a K step); rows past N are dequantised as zero
  const int wrow_t = tid & (BN - 1), wg = tid >> 8;
  const int ncol = n0 + wrow_t;
  const bool wvalid = ncol < p.N;
  const int64_t wr = wrow(p, wvalid ? ncol : n0);
  const uint8_t* wtile = p.w + (wr >> 6) * p.wG * 1280;   // the row's tile: one 1280-byte record per group
  const int wr64 = (int)(wr & 63);
  const int wkey = swz_key(wrow_t);

  auto x_load = [&](int k0, int buf, int r0, int r1) {   // this wave's instructions r0 .. r1 - 1
    uint8_t* xs = lds + buf * kStage + wv * 32 * 128;
#pragma unroll
    for (int r = r0; r < r1; ++r) {   // a chunk past K (a last step of one group) reads k0's: finite, never used
      const int kc = k0 + xk[r] < p.K ? k0 : 0;
      __builtin_amdgcn_global_load_lds((const void*)(xsrc[r] + kc), (__attribute__((address_space(3))) void*)(xs + r * 1024),
                                       16, 0, 0);
    }
  };
  // W records of one step, two register sets (see `step`)
  u32x4n wq[2];
  uint32_t wsm[2];
  auto w_load = [&](int k0, int set) {
    const bool in = k0 + 32 * wg < p.K;
    const uint8_t* rec = wtile + (((p.wk0 + k0) >> 5) + (in ? wg : 0)) * 1280;
    wq[set] = u32x4n(*(const u32x4*)(rec + wr64 * 16));   // weight offsets guarantee 4-byte alignment only
    wsm[set] = *(const uint32_t*)(rec + 1024 + wr64 * 4);
  };
  // dequantise this thread's group of one step into a stage. The fast path is straight-line code (it interleaves with
  // the MFMAs); a group whose q s + m may not be exact in fp32 is redone by the fp32 path afterwards (rare: a branch)
  auto w_stage_fast = [&](int k0, int buf, int set, int w0, int w1) {   // code words w0 .. w1 - 1 of the group
    uint8_t* ws = lds + buf * kStage + BM * 128 + wrow_t * 128;
    const uint32_t sm = (wvalid && k0 + 32 * wg < p.K) ? wsm[set] : 0u;   // scale 0, min 0: zero weights
#pragma unroll
    for (int w = w0; w < w1; ++w) *(u32x4n*)(ws + (((4 * wg + w) ^ wkey) << 4)) = deq_word(wq[set][w], sm, true);
  };
  auto w_stage_fix = [&](int k0, int buf, int set) {
    uint8_t* ws = lds + buf * kStage + BM * 128 + wrow_t * 128;
    const uint32_t sm = (wvalid && k0 + 32 * wg < p.K) ? wsm[set] : 0u;
    const bool fast = pk_exact(sm);
    if (__builtin_amdgcn_ballot_w64(!fast) != 0 && !fast) {
#pragma unroll
      for (int w = 0; w < 4; ++w) *(u32x4n*)(ws + (((4 * wg + w) ^ wkey) << 4)) = deq_word(wq[set][w], sm, false);
    }
  };

  // MFMA operand addresses: rows wm * 128 + 32 i + lane % 32 (A) and wn * 64 + 32 j + lane % 32 (B) share the swizzle
  // key of lane % 32, so one offset per k-step serves all fragments (the 32-row blocks are 4096 B apart)
  const int frow = lane & 31, fkey = swz_key(frow), fhalf = lane >> 5;
  const int aoff = (wm * WTM + frow) * 128, boff = BM * 128 + (wn * WTN + frow) * 128;
  u32x4n av[2][IB], bv[2][JB];
  auto frag = [&](const uint8_t* st, int s, int h) {
    const int cs = ((2 * s + fhalf) ^ fkey) << 4;
#pragma unroll
    for (int i = 0; i < IB; ++i) av[h][i] = *(const u32x4n*)(st + aoff + i * 4096 + cs);
#pragma unroll
    for (int j = 0; j < JB; ++j) bv[h][j] = *(const u32x4n*)(st + boff + j * 4096 + cs);
  };
  auto mfmas = [&](int h) {
#pragma unroll
    for (int i = 0; i < IB; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av[h][i]),
                                                           __builtin_bit_cast(half8, bv[h][j]), acc[i][j], 0, 0, 0);
  };
  // half a k-step's MFMAs: blocks i0, i0 + 1 of the fragment set h
  auto mfh = [&](int h, int i0) {
#pragma unroll
    for (int i = i0; i < i0 + 2; ++i)
#pragma unroll
      for (int j = 0; j < JB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av[h][i]),
                                                           __builtin_bit_cast(half8, bv[h][j]), acc[i][j], 0, 0, 0);
  };
  // one steady-state step (all four k-steps; the next stage exists). Step j's W records live in register set j & 1:
  // on entry SET = (it + 1) & 1 holds step it + 1 (dequantised now) and the other set, free since the last step's
  // dequant, is refilled with step it + 2.
  // The step is paced: 8 scheduling regions of 4 MFMAs each (sched_barrier between them), with the step's memory
  // work dealt out over the first six: one X load instruction per region, the W record loads and the four code words'
  // dequant + LDS stores one per region, the next fragments where their registers come free. The vector L1 holds a
  // bounded number of pending misses; issued together at the step's start, the loads stalled the issuing waves (and
  // with them their MFMAs) until the misses drained, 16-19% of the cycles by TCP_PENDING_STALL_CYCLES.
  auto step = [&](int it, int set) {
    const int buf = it & 1, k0 = it * BK;
    const uint8_t* st = lds + buf * kStage;
    frag(st, 0, 0);
    frag(st, 1, 1);
    __builtin_amdgcn_sched_barrier(0);
    x_load(k0 + BK, buf ^ 1, 0, 1);   // the next step's X streams into the other stage
    mfh(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    w_load(min(k0 + 2 * BK, (p.K - 1) / BK * BK), set ^ 1);   // step it + 2's records (clamped: the last is re-read)
    w_stage_fast(k0 + BK, buf ^ 1, set, 0, 1);                // W of the next step, word by word
    mfh(0, 2);
    __builtin_amdgcn_sched_barrier(0);
    x_load(k0 + BK, buf ^ 1, 1, 2);
    w_stage_fast(k0 + BK, buf ^ 1, set, 1, 2);
    mfh(1, 0);
    __builtin_amdgcn_sched_barrier(0);
    frag(st, 2, 0);
    x_load(k0 + BK, buf ^ 1, 2, 3);
    w_stage_fast(k0 + BK, buf ^ 1, set, 2, 3);
    mfh(1, 2);
    __builtin_amdgcn_sched_barrier(0);
    x_load(k0 + BK, buf ^ 1, 3, 4);
    w_stage_fast(k0 + BK, buf ^ 1, set, 3, 4);
    mfh(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    frag(st, 3, 1);
    mfh(0, 2);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(1);
    w_stage_fix(k0 + BK, buf ^ 1, set);
    // every memory operation of this step was issued by its sixth region: waiting for all of them here (this wave's
    // direct X loads of the next stage in particular) costs little once the last MFMAs have run
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  const int nk = (p.K + BK - 1) / BK;
  x_load(0, 0, 0, 4);
  w_load(0, 0);
  if (nk > 1) w_load(BK, 1);
  w_stage_fast(0, 0, 0, 0, 4);
  w_stage_fix(0, 0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int it = 0;
  for (; it + 2 < nk; it += 2) {   // two steps per trip: the register sets are compile-time
    step(it, 1);
    step(it + 1, 0);
  }
  if (it + 1 < nk) {
    step(it, 1);
    ++it;
  }
  {   // the last step (possibly one group only: two of the four k-steps)
    const int buf = it & 1, k0 = it * BK;
    const uint8_t* st = lds + buf * kStage;
    const int ksteps = p.K - k0 >= BK ? 4 : (p.K - k0) / 16;
    for (int s = 0; s < ksteps; ++s) {
      frag(st, s, 0);
      mfmas(0);
    }
  }

  gemm_epilogue<HEADS>(p, acc, lds, m0, n0, wm, wn, lane);
}

static const char* gepi_name(int e) {
  switch (e) {
    case P0_GEPI_F16: return "f16";
    case P0_GEPI_F32: return "f32";
    case P0_GEPI_RESADD: return "resadd";
    case P0_GEPI_SWIGLU: return "swiglu";
    case P0_GEPI_BIAS: return "bias";
    case P0_GEPI_HEADS: return "heads";
  }
  return "?";
}

}  // namespace p0

namespace p0 {
// The no-allocation GEMM's activation staging: a file-scope device array, 32 MiB (M K fp16 values of X', e.g. the
// FLUX.2-klein block's 4608 x 3072 rows with room to spare), held by every GPU the library runs on until the process
// ends. Host code never uses the array's name as an address: its device address on each GPU is looked up once, at
// p0_open with that device current, and kept per device.
constexpr size_t kScratchBytes = 32ull << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static void* g_scratch[kScratchDevices] = {};

// more than 64 KB of dynamic LDS must be allowed once per kernel; done at p0_open, so no call sets it lazily (for
// instance while its stream is being captured). Also looks up the scratch address on the current device.
int gemm_init() {
  int dv = -1;
  P0_HIP(hipGetDevice(&dv), "p0_open: gemm");
  if (dv >= 0 && dv < kScratchDevices && !g_scratch[dv]) {
    void* ptr = nullptr;
    P0_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "p0_open: gemm scratch address");
    g_scratch[dv] = ptr;
  }
  P0_HIP(hipFuncSetAttribute((const void*)q4_gemm_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds),
         "p0_open: gemm");
  P0_HIP(hipFuncSetAttribute((const void*)q4_gemm_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds),
         "p0_open: gemm");
  return P0_OK;
}
}  // namespace p0

using namespace p0;

// The GEMM call. stage_fixed != nullptr: the activation staging goes to that buffer of stage_cap bytes (the
// no-allocation entry point's static scratch) instead of the context's workspace, which may grow (hipMalloc).
static int gemm_call(const p0_gemm_args_t* a, double* flops_out, void* stage_fixed, size_t stage_cap) {
  if (!a) { set_error("gemm: no arguments"); return P0_EINVAL; }
  if (a->w_enc != P0_ENC_Q4G32A_T64) {   // engine/ops/gemm.js:266-267
    set_error(a->w_enc == P0_ENC_Q8G64S_T64 ? "gemm: unsupported weight encoding q8g64s.t64 (this build: q4g32a.t64)"
              : a->w_enc == P0_ENC_F16 ? "gemm: unsupported weight encoding f16 (this build: q4g32a.t64)"
                                       : "gemm: unsupported weight encoding %d", (int)a->w_enc);
    return P0_EINVAL;
  }
  const int64_t M = a->M, N = a->N, K = a->K;
  if (K % 32) { set_error("gemm: K must be a multiple of 32"); return P0_EINVAL; }   // engine/ops/gemm.js:278
  if (M <= 0 || N <= 0 || K <= 0) { set_error("gemm: M, N and K must be positive"); return P0_EINVAL; }
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) { set_error("gemm: dimension too large"); return P0_EINVAL; }
  if (a->wk0 % 32) { set_error("gemm: wk0 must be a multiple of 32"); return P0_EINVAL; }
  if (a->w_cols % 32 || a->w_rows % 64 || a->w_cols < a->wk0 + K) { set_error("gemm: weight shape"); return P0_EINVAL; }
  if (a->w_off % 4) { set_error("gemm: weight offset"); return P0_EINVAL; }
  // the weight rows the call reads (engine/ops/gemm.js:94-97): wr0 .. wr0 + N - 1, or for a swiglu the gate rows
  // wr0 .. wr0 + N/2 - 1 and the up rows wr1 .. wr1 + N/2 - 1
  if (a->wr0 < 0 || a->wr1 < 0) { set_error("gemm: negative weight row"); return P0_EINVAL; }
  {
    const bool sw = a->epi == P0_GEPI_SWIGLU;
    const int64_t span = sw ? N / 2 : N, top = sw && a->wr1 > a->wr0 ? a->wr1 : a->wr0;
    if (top + span > a->w_rows) {
      set_error("gemm: weight rows %lld + %lld past the %lld rows of the weight", (long long)top, (long long)span,
                (long long)a->w_rows);
      return P0_EINVAL;
    }
  }
  if (a->x_mode < P0_XMODE_F16 || a->x_mode > P0_XMODE_BF16) { set_error("gemm: x mode %d", a->x_mode); return P0_EINVAL; }
  if (a->epi < P0_GEPI_F16 || a->epi > P0_GEPI_HEADS) { set_error("gemm: epilogue %d", a->epi); return P0_EINVAL; }
  if (a->epi == P0_GEPI_HEADS) {   // one head per 128 output columns (engine/ops/gemm.js:213)
    if (N % 128) { set_error("gemm: heads needs N a multiple of 128"); return P0_EINVAL; }
    if (!a->ev || !a->rope) { set_error("gemm: heads needs ev (the norm weights) and heads.rope"); return P0_EINVAL; }
    if (a->heads_rope != P0_ROPE_INTER && a->heads_rope != P0_ROPE_HALF) {
      set_error("gemm: heads rope mode %d", a->heads_rope); return P0_EINVAL;
    }
    if (a->heads_hq < 0 || a->heads_hkv < 0 || a->heads_row_off < 0 || a->heads_row_off + M > a->heads_ltot) {
      set_error("gemm: heads rows %lld + %lld past Ltot %lld", (long long)a->heads_row_off, (long long)M,
                (long long)a->heads_ltot);
      return P0_EINVAL;
    }
  }
  if (a->epi == P0_GEPI_SWIGLU && (N & 1)) { set_error("gemm: swiglu needs an even N"); return P0_EINVAL; }
  if (!a->w || !a->x || !a->y) { set_error("gemm: missing w, x or y buffer"); return P0_EINVAL; }
  if ((a->x_mode == P0_XMODE_LNMOD || a->x_mode == P0_XMODE_RMS) && (!a->stats || !a->pv)) {
    set_error("gemm: %s needs stats and pv", a->x_mode == P0_XMODE_LNMOD ? "lnmod" : "rms"); return P0_EINVAL;
  }
  if (a->epi == P0_GEPI_BIAS && !a->ev) { set_error("gemm: bias needs ev"); return P0_EINVAL; }
  // X': the caller's fp16 rows when they can be streamed as they are (16-byte aligned rows), else one staging pass
  const int64_t ldx = a->x_ld ? a->x_ld : K;
  const uint8_t* xbase = (const uint8_t*)a->x + a->x_off;
  const bool direct = a->x_mode == P0_XMODE_F16 && ((uintptr_t)(xbase + 2 * a->x_k0) % 16 == 0) && (2 * ldx) % 16 == 0;
  if (!direct && stage_cap && (size_t)M * K * 2 > stage_cap) {
    set_error("gemm_noalloc: the activations need %lld B of fp16 staging; the static scratch holds %zu B",
              (long long)(M * K * 2), stage_cap);
    return P0_EINVAL;
  }
  if (int r = require_open("gemm")) return r;
  if (int r = refuse_in_chain("gemm")) return r;
  if (stage_cap && !stage_fixed) { set_error("gemm_noalloc: no scratch on device %d", ctx().device); return P0_ENODEV; }

  GemmP p{};
  p.w = (const uint8_t*)a->w + a->w_off;
  p.wG = a->w_cols / 32;
  p.Nw = a->w_rows;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.wr0 = a->wr0; p.wr1 = a->wr1; p.wk0 = a->wk0;
  p.epi = a->epi;
  p.y = (uint8_t*)a->y + a->y_off;
  p.ldy = a->y_ld ? a->y_ld : N;
  p.ny0 = a->y_n0;
  p.ev = a->ev; p.evOff = a->ev_off;
  p.bv = a->bv; p.bvOff = a->bv_off; p.bvUp = a->bv_up;
  p.act = a->act; p.store = a->store; p.res = a->res;
  p.hLtot = a->heads_ltot; p.hRow0 = a->heads_row_off; p.hq = a->heads_hq; p.hkv = a->heads_hkv;
  p.hrope = a->heads_rope; p.heps = a->heads_eps != 0.0f ? a->heads_eps : 1e-6f; p.rope = a->rope;
  (void)gepi_name;

  if (direct) {
    p.x = (const _Float16*)xbase + a->x_k0;
    p.ldx = ldx;
  } else {
    void* stage = stage_fixed;
    if (!stage) {
      if (int r = ensure_xstage((size_t)M * K * 2, "gemm")) return r;
      keep_for_recording(ctx().xstage_keep);
      stage = ctx().xstage;
    }
    XStageP q{};
    q.x = xbase; q.ldx = ldx; q.kx0 = a->x_k0; q.xmode = a->x_mode;
    q.M = (int)M; q.K = (int)K;
    q.st = a->stats; q.stOff = a->stats_off;
    q.pv = a->pv; q.pvOff = a->pv_off; q.pvShift = (uint32_t)(a->pv_off + a->pv_stride);
    q.out = (_Float16*)stage;
    const int esz = (a->x_mode == P0_XMODE_F16 || a->x_mode == P0_XMODE_BF16) ? 2 : 4;
    q.vec = ((uintptr_t)(xbase + esz * a->x_k0) % 16 == 0) && (esz * ldx) % 16 == 0;
    const int64_t chunks = M * (K / 8);
    const int64_t blocks = (chunks + 255) / 256 < 8192 ? (chunks + 255) / 256 : 8192;
    hipLaunchKernelGGL(x_stage_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx().cur, q);
    P0_LAUNCHED("gemm");
    p.x = (const _Float16*)stage;
    p.ldx = K;
  }
  const int64_t tiles = ((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  const bool heads = a->epi == P0_GEPI_HEADS;
  hipLaunchKernelGGL(heads ? q4_gemm_kernel<true> : q4_gemm_kernel<false>, dim3((unsigned)tiles), dim3(kThreads),
                     kGemmLds, ctx().cur, p);
  P0_LAUNCHED("gemm");
  if (flops_out) *flops_out = 2.0 * (double)M * (double)N * (double)K;
  return P0_OK;
}

extern "C" int p0_q4_gemm(const p0_gemm_args_t* a, double* flops_out) { return gemm_call(a, flops_out, nullptr, 0); }

// The no-allocation variant: the same kernels, the activation staging in the static scratch of this file (its
// address on the open device was looked up at p0_open); nothing is allocated or freed.
extern "C" int p0_q4_gemm_noalloc(const p0_gemm_args_t* a, double* flops_out) {
  const int dv = ctx().device;
  return gemm_call(a, flops_out, dv >= 0 && dv < kScratchDevices ? g_scratch[dv] : nullptr, kScratchBytes);
}
