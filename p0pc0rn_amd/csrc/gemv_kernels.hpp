// gemv_kernels.hpp - device code of the q4g32a.t64 GEMV (M = 1), GEMV-M (M <= 16) and GEMV chains for gfx950.
//
// Replaces the WebGPU dispatch of gemv (engine/llm/lops.js:108-141) and gemvM (engine/llm/lops_spec.js:159-191) with
// the same arguments, the same split semantics (nsplit partial rows Y[split * ldy + m * ldm + n]) and the same errors.
//
// Data layout (q4g32a.t64, engine/kcheck.js:22-38): a weight W[N][K] is a sequence of 1280-byte records, record
// (tile, g) = rows 64 tile .. 64 tile + 63, k = 32 g .. 32 g + 31, tile-major. Bytes [16 r, 16 r + 16) hold row r's 32
// codes (u32 word w, nibble i = k 8 w + i); u32 256 + r = fp16 scale | fp16 min << 16.
//
// Kernel mapping (MI355X: 64-lane waves, 160 KB LDS per CU, 256 CUs in 8 XCDs):
//  * one wave owns one 64-row tile (lane = row; T = 2 tiles per wave on large N, or the gate/up pair of a geglu);
//  * per record, a lane issues ONE 16-byte load of its row's codes and one 4-byte load of its scale/min: the wave reads
//    the record's 1024 + 256 bytes as two fully coalesced requests;
//  * a code word is split with masks into fp16 bit patterns that ARE the codes as subnormals (q * 2^-24; the odd
//    nibbles land as 16 q * 2^-24), which v_fma_mix_f32 multiplies into fp32 accumulators exactly: 13 VALU ops per
//    8 weights, no int->float conversion;
//  * x' = prologue(x) is staged once per workgroup in LDS for the workgroup's K-slice, the odd-k entries pre-scaled by
//    1/16 (exact) to undo the odd nibbles' factor 16, plus the per-group sums of x' for the min term:
//    y = sum_g (s_g 2^24) * (2^-24 sum q x') + m_g * sum x'   (the reference's s * sum q x + m * sum x split,
//    engine/llm/lops.js:71);
//  * when N alone gives too few waves for 256 CUs, K is split across workgroups; each writes its partial sums to the
//    context workspace and the LAST workgroup to arrive at a (split, tile block) adds them in K-slice order (so the
//    result does not depend on arrival order) and runs the epilogue.
#pragma once
#include "common.hpp"

namespace p0 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
// 4-byte alignment is all a record base guarantees (weight offsets are multiples of 4, engine/llm/lops.js:124);
// global_load_dwordx4 needs only dword alignment, so one 16-byte load per lane serves both cases
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4l __attribute__((ext_vector_type(4)));   // 16-byte aligned (LDS)
// Global-memory view of a pointer. Pointers read from memory (a chain's op table) are generic to the compiler, which
// then emits flat instructions; flat loads also count on the LDS wait counter, so every LDS wait would wait for the
// weight stream too. The cast makes them global loads / stores / atomics again.
#define P0_GLOBAL(T, ptr) ((__attribute__((address_space(1))) T*)(ptr))


struct GemvP {
  const uint8_t* w;   // weight base (buf + w_off)
  int64_t wG;         // groups per weight row (w_cols / 32)
  int N, K, kPer, nsplit, NT;
  int pro, epi;
  const float* X; int64_t ldx, rowB;
  const float* ST; int64_t statOff, statLd;
  const float* NW; int64_t nOff;
  int nsrc; int64_t ldp;
  const float* EV; int64_t evOff, evLd;
  float* Y; int64_t ldy, ldm;
  float* MX; float cap;
  int gps;            // groups per workgroup K-slice
  int nks;            // workgroup K-slices per split (> 1: cross-workgroup reduction through the workspace)
  int kw;             // waves per tile slot inside a workgroup (each takes a contiguous share of the K-slice)
  int tgw;            // tile slots per workgroup (waves = tgw * kw)
  int ntb;            // tile blocks (grid.x)
  int rowsTot;        // rows that carry partials: N, or 2N for a geglu
  int mode;           // kernel mode (chain ops choose their code path from it)
  // chain ops: bit 0 = read the inputs with device-coherent loads (an earlier op of the chain writes into them), bit
  // 1 = write the outputs with device-coherent stores (a later op reads them, or another op writes the same lines)
  int coh;
  float* part; unsigned* cnt;
  // staged chain ops (mode 3, q4_gemv_chain_kernel): the op's rows are dealt as units of 16 snrb rows (a geglu's unit
  // also holds the matching up rows) x one split, unit u to workgroup position (scur + u) mod grid
  int su, scur, snrb, sngp;   // units, first position, 16-row blocks per unit, groups per split rounded up to 16
  int sred;                   // LDS float offset of the reduction area (after x' and its group sums)
  int swoff;                  // LDS byte offset of the staged weights
  int enc;                    // P0_ENC_Q4G32A_T64, or P0_ENC_Q8G64S_T64 (gemv_q8.hip)
  int mrows;                  // rows of x (M)
  // pipelined M = 1 chains: an op whose only input is the previous op's output takes it from that op's mailbox, one
  // 64-bit word per output row (run tag << 32 | the value's bits) in the chain state, instead of waiting for the
  // previous op's completion flags and then loading x: one memory round trip instead of two
  unsigned long long* mbxOut;       // this op's mailbox (row n at n), or null
  const unsigned long long* mbxIn;  // x[k] of this op at mbxIn[k], or null
  // a mailbox op (whose mailbox says only that the elements it reads are written) whose outputs overlap what an earlier
  // op reads or writes waits for op i - wback's completion flags before it writes them: 1 if op i - 1 reads them, 2 if
  // only ops before i - 1 do, 0 if none does
  int wback;
  int mf;             // M >= 2: the MFMA arithmetic (standalone: gemv_item; pipelined chains: the slots), else fp32 VALU
  // pipelined M > 1 chains on the matrix cores: an op whose input is one split of the previous op's output takes its x'
  // already staged by that op (stgIn), which writes, besides its outputs, the next op's prologue values as the matrix
  // cores' fp16 hi / lo A operands and the group sums as 16-row halves (stgOut, layout at stg_half_at): the consumer
  // copies bytes where it would otherwise split and sum M rows of values on the VALU after its wait
  uint32_t* stgOut;             // the next op's staged x', or null
  const uint32_t* stgIn;        // this op's staged x', or null
  int64_t stgR0;                // output row of the split stgSp that is the next op's k = 0
  int stgK, stgSp, stgPro;      // the next op's K, the split it reads, its prologue (raw or rms)
  const float* stgST; int64_t stgStatOff, stgStatLd;   // the next op's rstd slots (rms)
  const float* stgNW; int64_t stgNOff;                  // the next op's norm weights (rms)
  // ops of a pipelined chain that are not GEMVs (kind != kOpGemv): p0_copy, p0_argmax / p0_argmaxM, p0_rowstats and
  // p0_normadd called while a chain is being built (chain_aux.hpp). They have no units and stream no weights (su = 0):
  // the workgroups that take part wait for op i - 1 in every workgroup, do the op and publish their flags.
  //   copy:     an words from asrc to adst
  //   argmax:   arows rows of acols (max, index) pairs at asrc -> adst[2 m], adst[2 m + 1]
  //   rowstats: arows rows of acols floats at asrc[r ald + ac0 + c] -> (mean, rstd) pairs at adst[(astOff + r) 2]
  //   normadd:  arows rows of acols floats: t = sum of the an partials asrc[j aldp + m acols + i], the residual adst
  //             updated (amode 0, norm weights aw + awOff) or replaced (amode 1), ast[astOff + m] = its rstd
  int kind;
  int abefore;   // the op whose completion flags the workers wait for first (-1: none; set by p0_chain_end)
  const float* asrc; float* adst; float* ast; const float* aw;
  int64_t arows, acols, ald, ac0, an, aldp, astOff, awOff;
  float aeps, ascale;
  int amode;
};
constexpr int kOpGemv = 0, kOpCopy = 1, kOpArgmax = 2, kOpRowstats = 3, kOpNormadd = 4;
// staged x' of an op of K inputs and M x rows: per group g = k / 32 and code word w = (k / 8) % 4, the hi halves of the
// M rows then their lo halves, 8 halves each in the word's nibble order (k 8w + 0, 4, 1, 5, 2, 6, 3, 7) (the LDS layout
// of stage_x_mf / stage_rows, group by group); then the group sums as [g][half of 16 k][M] floats, a NaN half meaning
// some |x'| of it reached kMfBig (or was not finite)
__host__ __device__ inline int64_t stg_half_at(int M, int64_t k, int m, int lo) {
  const int64_t g = k >> 5;
  const int w = (int)(k >> 3) & 3, j = (int)k & 7;
  return (((g * 4 + w) * 2 + lo) * M + m) * 8 + (((j & 3) << 1) | (j >> 2));
}
// then the fp32 x' values themselves, [m][k], which the wide chain's producers also write (chain_wide.hip: a consumer
// wave whose staged halves overflowed the 2^8 scale takes these instead, with a scale of its own)
__host__ __device__ inline int64_t stg_f32_at(int M, int64_t K) { return K * M + (K >> 5) * 2 * M; }
__host__ __device__ inline int64_t stg_words(int M, int64_t K) { return stg_f32_at(M, K) + K * M; }

// Op i of a chain's op table, read through the constant address space. The table is read-only for the whole launch,
// so every field read at a uniform op index becomes a scalar load. Through a global pointer the compiler has to
// assume that the chain loop's waits and atomics may write the table, and reads each field with a vector load; every
// such load then waits behind the wave's other memory traffic (the outputs' stores, the loaders' LDS-DMA), one field
// at a time. The index goes through readfirstlane: the op loops leave early on a timed-out wait, and the compiler may
// then hold the loop counter in a vector register, which would make the address (and the loads) per lane again.
__device__ __forceinline__ const GemvP& op_at(const GemvP* ops, int i) {
  return *(const GemvP*)((const __attribute__((address_space(4))) GemvP*)ops + __builtin_amdgcn_readfirstlane(i));
}

__device__ __forceinline__ float gelu_tanh(float v) {   // engine/llm/lops.js:26
  float t = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  t = fminf(15.0f, fmaxf(-15.0f, t));
  return v * 0.5f * (1.0f + tanhf(t));
}

// Activation loads and output stores. Inside a chain (COH), ops hand data to each other within one launch: outputs are
// written with device-coherent stores and inputs read with device-coherent loads (relaxed agent-scope atomics: they
// bypass the non-coherent per-XCD L2 copies), so no whole-L2 writeback / invalidate is needed around the hand-off.
template <bool COH>
__device__ __forceinline__ float ldf(const float* a) {
  if (COH) return __hip_atomic_load(P0_GLOBAL(float, const_cast<float*>(a)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *P0_GLOBAL(const float, a);
}
template <bool COH>
__device__ __forceinline__ void stf(float* a, float v) {
  if (COH) __hip_atomic_store(P0_GLOBAL(float, a), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *P0_GLOBAL(float, a) = v;
}

// prologue value x'[m][k] (engine/llm/lops.js:50-57, engine/llm/lops_spec.js:61-64)
template <bool COH>
__device__ __forceinline__ float prologue(const GemvP& p, int m, int k) {
  if (p.pro == P0_PRO_RAW) return ldf<COH>(&p.X[m * p.ldx + p.rowB + k]);
  if (p.pro == P0_PRO_RMS)
    return ldf<COH>(&p.X[m * p.ldx + p.rowB + k]) * ldf<COH>(&p.ST[p.statOff + m * p.statLd]) *
           ldf<COH>(&p.NW[p.nOff + k]);
  float s = 0.0f;
  for (int j = 0; j < p.nsrc; ++j) s += ldf<COH>(&p.X[j * p.ldp + m * p.ldx + k]);
  if (p.pro == P0_PRO_SUM) return s;
  return gelu_tanh(s) * ldf<COH>(&p.EV[p.evOff + m * p.evLd + k]);
}

// U prologue values of one thread, every load issued before any is used (the device-coherent loads of a chain are
// ordered memory operations: interleaved with their uses they would wait one at a time). Element u is x'[m[u]][kb +
// kl[u]]; only the first nu (the same in the whole wave) are loaded, the rest are 0, and so are entries at or past
// ke (which read the slice's last element, in bounds).
template <bool COH, int U, int M>
__device__ __forceinline__ void prologue_batch(const GemvP& p, int nu, const int (&m)[U], int kb, int ke,
                                               const int (&kl)[U], float (&v)[U]) {
  int k[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    k[u] = min(kb + kl[u], ke - 1);
    v[u] = 0.0f;
  }
  if (p.pro == P0_PRO_RAW || p.pro == P0_PRO_RMS) {
    float a[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (u < nu) a[u] = ldf<COH>(&p.X[m[u] * p.ldx + p.rowB + k[u]]);
    if (p.pro == P0_PRO_RMS) {
      float b[U], c[U];
      if (M == 1) {
        const float b0 = ldf<COH>(&p.ST[p.statOff]);
#pragma unroll
        for (int u = 0; u < U; ++u) b[u] = b0;
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (u < nu) b[u] = ldf<COH>(&p.ST[p.statOff + m[u] * p.statLd]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < nu) c[u] = ldf<COH>(&p.NW[p.nOff + k[u]]);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < nu) a[u] = a[u] * b[u] * c[u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (u < nu && kb + kl[u] < ke) v[u] = a[u];
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (u < nu && kb + kl[u] < ke) v[u] = prologue<COH>(p, m[u], k[u]);
  }
}

// sum over the 32 lanes 32j .. 32j + 31 (a pairwise tree: quads, halves of rows, rows of 16, then the two rows); every
// lane of the 32 gets the same value
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float sum32(float v) {
  v += dpp_f<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  v += dpp_f<0x140>(v);   // row_mirror
  // lane ^ 16: the gfx950 row swap hands back the value and its partner's in two registers (a VALU lane move, where a
  // ds_swizzle would take an LDS round trip); the two sums are the same in every lane
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x'[m][k] of the groups [g0, g1) -> LDS xs[m * 32 gps + k - 32 g0] (odd k scaled by `odd`: 1/16 for the q4 dot
// products, 1 for q8 ones), and the per-group sums of
// x' -> xsum[m * gps + group - g0]; entries of the gps groups past g1 are zero. Thread tid takes elements u * blockDim +
// tid of each batch of U: the 32 lanes of a 32-aligned lane group hold one group's 32 k (the slice length and the
// block size are multiples of 32), which they sum with cross-lane adds. Every thread runs the same number of
// batches, so all lanes take part in the cross-lane adds.
// tid / nt: the calling thread's index among the nt threads that stage (whole waves; every one of them calls).
template <int M, bool COH>
__device__ __forceinline__ void stage_x(const GemvP& p, int g0, int g1, int gps, float* xs, float* xsum,
                                        int tid = threadIdx.x, int nt = blockDim.x, float odd = 0.0625f) {
  constexpr int U = M == 1 ? 4 : 8;
  const int lane = tid & 63, wv = tid >> 6;
  const int KL = gps * 32, kb = g0 * 32, ke = g1 * 32, nx = M * KL;
  for (int i0 = 0; i0 < nx; i0 += U * nt) {
    int mm[U], kl[U];
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = i0 + u * nt + tid;
      mm[u] = M == 1 ? 0 : min(idx / KL, M - 1);
      kl[u] = idx - mm[u] * KL;   // >= KL (so past ke) for idx >= nx
    }
    // batches of this wave that hold elements (u * nt + the wave's first thread < nx - i0)
    const int nu = ke > kb ? min(U, max(0, (nx - i0 - (wv << 6) + nt - 1) / nt)) : 0;
    prologue_batch<COH, U, M>(p, nu, mm, kb, ke, kl, v);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float gs = sum32(v[u]);
      if (i0 + u * nt + tid < nx) {
        xs[mm[u] * KL + kl[u]] = (kl[u] & 1) ? v[u] * odd : v[u];   // kb is even: k and kl share parity
        if ((lane & 31) == 0) xsum[mm[u] * gps + (kl[u] >> 5)] = gs;
      }
    }
  }
}

struct Rec {
  u32x4 q;
  uint32_t sm;
};

// ---- GEMV-M on MFMA (standalone launches, M >= 2). Per q4 group and 16 weight rows, two v_mfma_f32_16x16x32_f16
// compute D[m][n] = 2^8 sum_k x'[m][k] q[n][k]: the A operand holds 2^8 x' split into fp16 hi + lo (2^8 x' = hi + lo to
// 2^-22), the B operand the codes as exact fp16 values q (even k) and 16 q (odd k, whose x' carry the 1/16). Every
// operand is a normal fp16 number: the codes come out of a code word as 1024 + q (the masked nibbles with the exponent
// of 1024 OR-ed in, one v_and_or_b32 per pair) minus 1024, and the 2^8 keeps lo normal down to |x'| ~ 2^-11. (Fed as
// subnormals, q 2^-24 straight from the mask, the codes cost 4 VALU less per word, but a GEMV-M row then moved from
// ~3e-7 to 3.4e-6 relative L2 off the M = 1 row on MI355X: the matrix cores do not take fp16 subnormals at full
// precision.)
// Rounding: these rows are not bit-identical to the fp32 VALU path's (which p0_q4_gemv and the chain kernels use);
// they agree to ~3e-7 relative L2. The VALU path for every M is p0_gemv_tune knob 4 = 17.
// Lane l holds D[4 (l / 16) + i][l % 16]: one weight row per lane, so each lane applies its row's scale and min
// (2^-8 s D + m sum x') in fp32.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
constexpr float kMfScale = 256.0f;   // 2^8 x' in the A operand
constexpr float kMfDeq = 1.0f / kMfScale;   // D back to sum x' q
constexpr float kMfBig = 255.0f;     // |x'| from which a workgroup keeps the fp32 VALU path (fp16 hi would overflow)

// x' of the slice as MFMA A operands: [group][word w][hi, lo][M rows][8 halves], the 8 halves of word w in the code
// word's nibble order (k 8w + 0, 4, 1, 5, 2, 6, 3, 7), odd k scaled 1/16; group sums [group][XSS] (rows >= M zero).
// tid / nt: the calling thread among the nt staging threads (whole waves). True in a thread that saw some
// |x'| >= kMfBig (or not finite): the caller then stages fp32 x' for the VALU arithmetic instead.
template <int M, bool COH, int XSS>
__device__ __forceinline__ bool stage_x_mf(const GemvP& p, int g0, int g1, int gps, _Float16* xh, float* xsum, int tid,
                                           int nt) {
  constexpr int U = 8;
  const int lane = tid & 63, wv = tid >> 6;
  const int KL = gps * 32, kb = g0 * 32, ke = g1 * 32, nx = M * KL;
  if (M < XSS)
    for (int i = tid; i < gps * (XSS - M); i += nt) xsum[(i / (XSS - M)) * XSS + M + i % (XSS - M)] = 0.0f;
  bool bad = false;
  for (int i0 = 0; i0 < nx; i0 += U * nt) {
    int mm[U], kl[U];
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int idx = i0 + u * nt + tid;
      mm[u] = min(idx / KL, M - 1);
      kl[u] = idx - mm[u] * KL;
    }
    const int nu = ke > kb ? min(U, max(0, (nx - i0 - (wv << 6) + nt - 1) / nt)) : 0;
    prologue_batch<COH, U, M>(p, nu, mm, kb, ke, kl, v);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float gs = sum32(v[u]);
      if (i0 + u * nt + tid < nx) {
        const int g = kl[u] >> 5, kk = kl[u] & 31, w = kk >> 3, j = kk & 7;
        const float x = (kl[u] & 1) ? v[u] * 0.0625f : v[u];
        const float xs8 = x * kMfScale;
        const _Float16 hi = (_Float16)xs8;
        const _Float16 lo = (_Float16)(xs8 - (float)hi);
        const int at = (((g * 4 + w) * 2) * M + mm[u]) * 8 + (((j & 3) << 1) | (j >> 2));
        xh[at] = hi;
        xh[at + M * 8] = lo;
        bad = bad || !(__builtin_fabsf(x) < kMfBig);
        if ((lane & 31) == 0) xsum[g * XSS + mm[u]] = gs;
      }
    }
  }
  return bad;
}

// one group's records of one 64-row tile as loaded: lane = row, its four code words and its scale/min word (two loads
// per lane; quarter_transpose turns them into the MFMA B layout)
struct RecM {
  u32x4 q;
  uint32_t sm;
};
__device__ __forceinline__ RecM load_rec_mf(const GemvP& p, int64_t tile, int g, int lane) {
  const uint8_t* rec = p.w + (int64_t)__builtin_amdgcn_readfirstlane((int)(tile * p.wG + g)) * 1280;
  RecM r;
  r.q = *P0_GLOBAL(const u32x4, rec + lane * 16);
  r.sm = *P0_GLOBAL(const uint32_t, rec + 1024 + lane * 4);
  return r;
}
// w[j] at lane 16 Q + i (Q the lane's 16-lane row) holds word j of weight row 16 Q + i; afterwards w[b] at lane 16 q + i
// holds word q of weight row 16 b + i, the B layout of block b (lane l: word l / 16 of row 16 b + l % 16). A 4 x 4
// transpose of (lane row, word) with the gfx950 lane swaps: permlane32_swap exchanges lanes 32-63 of its first operand
// with lanes 0-31 of its second, permlane16_swap the odd 16-lane rows of its first operand with the even rows of its
// second. Four copies of one word per lane come out as its row's word broadcast to the block's lanes.
__device__ __forceinline__ void quarter_transpose(uint32_t (&w)[4]) {
  const auto s02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
  const auto s13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
  const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  w[0] = s01[0];
  w[1] = s01[1];
  w[2] = s23[0];
  w[3] = s23[1];
}
// (v & mask) | e1024: with e1024 held in a vector register (its value hidden from the compiler) the and + or fold into
// one v_and_or_b32 (VOP3, which takes no literal on gfx950: the mask goes to a scalar register); with both constants
// literal the compiler keeps two instructions
__device__ __forceinline__ uint32_t and_or_1024(uint32_t v, uint32_t mask, uint32_t e1024) { return (v & mask) | e1024; }
// a code word's 8 codes as B operand values, in the nibble order of stage_x_mf's A operand
__device__ __forceinline__ half8_t codes_b(uint32_t v) {
  uint32_t e = 0x64006400u;
  asm("" : "+v"(e));
  const uint32_t v8 = v >> 8;
  const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2_t a = __builtin_bit_cast(h2_t, and_or_1024(v, 0x000F000Fu, e)) - k1024;    // q: k 8w, 8w + 4
  const h2_t b = __builtin_bit_cast(h2_t, and_or_1024(v, 0x00F000F0u, e)) - k1024;    // 16 q: k 8w + 1, 8w + 5
  const h2_t c = __builtin_bit_cast(h2_t, and_or_1024(v8, 0x000F000Fu, e)) - k1024;   // q: k 8w + 2, 8w + 6
  const h2_t d = __builtin_bit_cast(h2_t, and_or_1024(v8, 0x00F000F0u, e)) - k1024;   // 16 q: k 8w + 3, 8w + 7
  const u32x4l u = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, c),
                    __builtin_bit_cast(uint32_t, d)};
  return __builtin_bit_cast(half8_t, u);
}

// One record's lane slice: 16 bytes of the lane's row codes and its 4-byte scale/min. Nontemporal loads (STREAM) for
// ops that stream hundreds of MB (the two-tiles-per-wave mode): they keep the cache for the activations; plain loads
// otherwise, whose latency is lower (measured on MI355X: dependent HBM loads 280 ns plain, 330 ns nontemporal), which is
// what a small, latency-bound op waits on.
template <bool STREAM>
__device__ __forceinline__ Rec load_rec(const GemvP& p, int64_t tile, int g, int lane) {
  const uint8_t* rec = p.w + (int64_t)__builtin_amdgcn_readfirstlane((int)(tile * p.wG + g)) * 1280;
  Rec r;
  if (STREAM) {
    r.q = __builtin_nontemporal_load(P0_GLOBAL(const u32x4, rec + lane * 16));
    r.sm = __builtin_nontemporal_load(P0_GLOBAL(const uint32_t, rec + 1024 + lane * 4));
  } else {
    r.q = *P0_GLOBAL(const u32x4, rec + lane * 16);
    r.sm = *P0_GLOBAL(const uint32_t, rec + 1024 + lane * 4);
  }
  return r;
}

// 2^-24 * sum_k q_k x'_k over one row's 32 codes; x points at the group's 32 staged values (odd k pre-scaled 1/16)
__device__ __forceinline__ float dot32(const u32x4 q, const float* __restrict__ x) {
  const float4* x4 = (const float4*)x;
  const uint32_t u[4] = {q.x, q.y, q.z, q.w};
  float da = 0.0f, db = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 xa = x4[2 * w], xb = x4[2 * w + 1];   // k = 8w .. 8w+3, 8w+4 .. 8w+7
    const uint32_t v = u[w], v8 = v >> 8;
    const h2_t a = __builtin_bit_cast(h2_t, v & 0x000F000Fu);    // nibbles 0 | 4      (k 8w, 8w+4)
    const h2_t b = __builtin_bit_cast(h2_t, v & 0x00F000F0u);    // nibbles 1 | 5 x16  (k 8w+1, 8w+5)
    const h2_t c = __builtin_bit_cast(h2_t, v8 & 0x000F000Fu);   // nibbles 2 | 6      (k 8w+2, 8w+6)
    const h2_t e = __builtin_bit_cast(h2_t, v8 & 0x00F000F0u);   // nibbles 3 | 7 x16  (k 8w+3, 8w+7)
    da = __builtin_fmaf((float)a.x, xa.x, da);
    db = __builtin_fmaf((float)a.y, xb.x, db);
    da = __builtin_fmaf((float)b.x, xa.y, da);
    db = __builtin_fmaf((float)b.y, xb.y, db);
    da = __builtin_fmaf((float)c.x, xa.z, da);
    db = __builtin_fmaf((float)c.y, xb.z, db);
    da = __builtin_fmaf((float)e.x, xa.w, da);
    db = __builtin_fmaf((float)e.y, xb.w, db);
  }
  return da + db;
}

__device__ __forceinline__ float h2f_lo(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).x; }
__device__ __forceinline__ float h2f_hi(uint32_t v) { return (float)__builtin_bit_cast(h2_t, v).y; }

// wave-wide (max, lowest index) of the softcapped row values: engine/llm/lops.js:96-102
__device__ __forceinline__ void wave_argmax(float& v, int& r) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float ov = __shfl_xor(v, off, 64);
    int orr = __shfl_xor(r, off, 64);
    if (ov > v || (ov == v && orr < r)) { v = ov; r = orr; }
  }
}

// the epilogue of one wave for x row m: tot0 = row sums of tile0 (gate tile for a geglu), tot1 = the up tile's;
// returns the value stored at row n of y. P: GemvP, or any type with its epi, Y, ldy, ldm, cap, MX and NT members
template <bool COH, class P = GemvP>
__device__ __forceinline__ float epilogue(const P& p, int split, int m, int tile0, int lane, float tot0, float tot1) {
  const int n = tile0 * 64 + lane;
  if (p.epi == P0_EPI_STORE) {
    stf<COH>(&p.Y[split * p.ldy + m * p.ldm + n], tot0);
    return tot0;
  } else if (p.epi == P0_EPI_GEGLU) {
    const float v = gelu_tanh(tot0) * tot1;
    stf<COH>(&p.Y[m * p.ldm + n], v);
    return v;
  } else {
    float v = p.cap * tanhf(fminf(15.0f, fmaxf(-15.0f, tot0 / p.cap)));
    stf<COH>(&p.Y[m * p.ldm + n], v);
    int r = lane;
    wave_argmax(v, r);
    if (lane == 0) {
      const int o = (m * p.NT + tile0) * 2;
      stf<COH>(&p.MX[o], v);
      stf<COH>(&p.MX[o + 1], __int_as_float(tile0 * 64 + r));
    }
    return v;
  }
}

// One work item of one op, run by the calling workgroup: tile block bx, (split, K-slice) by. MODE 0: one tile per
// wave; MODE 1: two tiles per wave; MODE 2: geglu (gate tile + its up tile N/64 tiles later). A workgroup = tgw tile
// slots x kw waves per slot; it owns the K-slice [g0, g1) of one split, and the kw waves of a slot take contiguous
// shares of it, reduced through LDS in wave order. `ready()` runs after the item's first weight loads are issued and
// before its input is read (the chain executor waits for the producing op there; a standalone launch has nothing to
// wait for); it returns false (in every thread) to abandon the item. Returns true when this workgroup wrote the
// final outputs of its (split, tile block): always for one K-slice per split, only the last arriving workgroup
// otherwise. The value is the same in every thread. CHAIN: activations that ops hand to each other move through
// device-coherent accesses (GemvP::coh). Every wave issues its first chunk before the wait, the polling wave too: its
// first poll then returns behind those loads (a wave's loads complete in order), which costs nothing when the wait is
// longer than the loads' latency, and a wave that issued them after the wait would hold the whole workgroup at the
// prologue's barrier for a full HBM latency.
template <int M, int MODE, bool CHAIN, class Ready, bool MFK = false>
__device__ __forceinline__ bool gemv_item(const GemvP& p, int bx, int by, float* smem, int* s_last, Ready&& ready) {
  constexpr int T = MODE == 0 ? 1 : 2;
  constexpr int TPW = MODE == 1 ? 2 : 1;   // distinct output tiles per wave
  // Chunks of D groups: all D (x T) records of a chunk are issued, then consumed in order. No load is carried across
  // the loop's back edge, so the compiler's wait counts stay exact (each consume waits for its own record only; a
  // rotating pipeline carried across the back edge made the counts collapse to near-full drains). The latency at
  // the start of each chunk is hidden by the other resident waves. Loads past the share's end re-read its last group
  // (in bounds, value unused), so every load is unconditional.
  constexpr int D = MODE == 0 ? 8 : 4;
  const int tid = threadIdx.x, lane = tid & 63;
  const bool coh_in = CHAIN && (p.coh & 1), coh_out = CHAIN && (p.coh & 2);
  // wave-uniform indices live in SGPRs: record addresses become a scalar base plus the lane's constant 16-byte offset
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kwv = wv % p.kw, tw = wv / p.kw;
  const int KL = p.gps * 32;
  // MF: GEMV-M on MFMA (stage_x_mf); the fp32 VALU path stays for a workgroup whose x' is too large for fp16
  constexpr bool MF = MFK && !CHAIN && M >= 2;
  constexpr bool mf = MF;
  const int XS = mf && M < 16 ? 16 : M;   // group-sum entries per group (MF: a 16-row A operand)
  float* xs = smem;                    // [M][KL]   x' of the slice, odd k scaled 1/16 (MF: the A operands, same size)
  float* xsum = smem + M * KL;         // [M][gps]  group sums of x' (MF: [gps][16])
  float* red = xsum + XS * p.gps;      // [waves][T][64] in-workgroup reduction

  const int split = by / p.nks, ks = by - split * p.nks;
  const int k0s = split * p.kPer, k1s = min(p.K, k0s + p.kPer);
  const int gs0 = k0s >> 5, gs1 = k1s >> 5;
  const int g0 = min(gs1, gs0 + ks * p.gps), g1 = min(gs1, g0 + p.gps);
  const int sub = (g1 - g0 + p.kw - 1) / p.kw;
  const int wg0 = min(g1, g0 + kwv * sub), wg1 = min(g1, wg0 + sub);   // this wave's share

  // tiles of this wave
  const int slot = bx * p.tgw + tw;
  int tile[T];
  if (MODE == 2) {
    tile[0] = slot;
    tile[T - 1] = slot + p.NT;
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) tile[t] = slot * TPW + t;
  }
  const bool active = tile[0] < p.NT;
  // a wave's second tile past N (odd tile count, MODE 1) re-reads its first tile; its results are never stored
  auto tl = [&](int t) -> int64_t { return (MODE == 1 && tile[t] >= p.NT) ? tile[0] : tile[t]; };
  const int glast = wg1 - 1;
  const bool streams = active && wg0 < wg1;

  // ---- the share's first chunk is issued before the input is read: its latency overlaps the wait and the prologue
  if (mf && tid == 0) *s_last = 0;   // MF: the "x' too large" flag until the split-K arrival reuses the word
  __syncthreads();   // the previous item of this workgroup is done with the LDS
  float acc[T][M];
  bool mfd = false;   // MF: acc filled by the MFMA path
  if constexpr (MF) {
    constexpr int DM = 4;   // groups per chunk of records (8 registers per group and tile)
    RecM m0[DM][T];
    if (streams) {
#pragma unroll
      for (int i = 0; i < DM; ++i)
#pragma unroll
        for (int t = 0; t < T; ++t) m0[i][t] = load_rec_mf(p, tl(t), min(wg0 + i, glast), lane);
    }
    if (stage_x_mf<M, false, (M < 16 ? 16 : M)>(p, g0, g1, p.gps, (_Float16*)xs, xsum, tid, blockDim.x)) *s_last = 1;
    __syncthreads();
    if (*s_last == 0) {
      float am[T][4][4];   // [tile][16-row block][i]: rows 16 b + lane % 16, x row 4 (lane / 16) + i
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) am[t][b][i] = 0.0f;
      const _Float16* xh = (const _Float16*)xs;
      const int arow = min(lane & 15, M - 1), aw = lane >> 4;
      auto consume_mf = [&](const RecM (&cur)[T], int g) {
        const int gl = g - g0;
        const half8_t* ap = (const half8_t*)(xh + (((gl * 4 + aw) * 2) * M + arow) * 8);
        // rows >= M read row M - 1 (finite); their D rows are never used
        const half8_t ahi = ap[0], alo = ap[M];
        const f4_t sx = *(const f4_t*)(xsum + gl * 16 + 4 * aw);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          uint32_t qb[4] = {cur[t].q.x, cur[t].q.y, cur[t].q.z, cur[t].q.w};
          uint32_t sb[4] = {cur[t].sm, cur[t].sm, cur[t].sm, cur[t].sm};
          quarter_transpose(qb);
          quarter_transpose(sb);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const half8_t bq = codes_b(qb[b]);
            f4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bq, d, 0, 0, 0);
            const float s8 = h2f_lo(sb[b]) * kMfDeq, mn = h2f_hi(sb[b]);
#pragma unroll
            for (int i = 0; i < 4; ++i) am[t][b][i] = __builtin_fmaf(s8, d[i], __builtin_fmaf(mn, sx[i], am[t][b][i]));
          }
        }
      };
      if (streams) {
#pragma unroll
        for (int i = 0; i < DM; ++i)
          if (wg0 + i < wg1) consume_mf(m0[i], wg0 + i);
        for (int c0 = wg0 + DM; c0 < wg1; c0 += DM) {
          RecM r[DM][T];
#pragma unroll
          for (int i = 0; i < DM; ++i)
#pragma unroll
            for (int t = 0; t < T; ++t) r[i][t] = load_rec_mf(p, tl(t), min(c0 + i, glast), lane);
#pragma unroll
          for (int i = 0; i < DM; ++i)
            if (c0 + i < wg1) consume_mf(r[i], c0 + i);
        }
      }
      // back to one weight row per lane (acc[t][m] at lane = row) through this wave's reduction row: x row m lives in
      // the 16 lanes l / 16 == m / 4, element m % 4, for rows 16 b + l % 16. Lanes hand values to other lanes here, so
      // a wavefront fence on each side keeps the compiler from moving a read above other lanes' writes (the LDS itself
      // serves one wave's accesses in order)
      auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      };
#pragma unroll
      for (int t = 0; t < T; ++t) {
        float* tr = red + (wv * T + t) * 64;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          wave_sync();
          if ((lane >> 4) == (m >> 2)) {
#pragma unroll
            for (int b = 0; b < 4; ++b) tr[16 * b + (lane & 15)] = am[t][b][m & 3];
          }
          wave_sync();
          acc[t][m] = tr[lane];
        }
      }
      mfd = true;
    } else {
      __syncthreads();   // x' too large for fp16: this workgroup stages fp32 x' and takes the VALU path
      stage_x<M, false>(p, g0, g1, p.gps, xs, xsum);
      __syncthreads();
    }
  }
  if (!mfd) {
  Rec r0[D][T];
  if (streams) {
#pragma unroll
    for (int i = 0; i < D; ++i)
#pragma unroll
      for (int t = 0; t < T; ++t) r0[i][t] = load_rec<MODE == 1>(p, tl(t), min(wg0 + i, glast), lane);
  }
  if (!ready()) return false;

  // ---- prologue: x'[m][k] for the workgroup's K-slice -> LDS (odd k scaled 1/16), and the per-group sums of x'
  if (!mf) {
    if (coh_in) stage_x<M, true>(p, g0, g1, p.gps, xs, xsum);
    else stage_x<M, false>(p, g0, g1, p.gps, xs, xsum);
    __syncthreads();
  }

  // ---- stream the records of the wave's share
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[t][m] = 0.0f;

  // one group's records: scale/min unpack, then the M x-rows against each tile's codes
  auto consume = [&](const Rec (&cur)[T], int g) {
    const int gl = g - g0;
    float s24[T], mn[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      s24[t] = h2f_lo(cur[t].sm) * 16777216.0f;   // scale * 2^24 (exact)
      mn[t] = h2f_hi(cur[t].sm);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float* xg = xs + m * KL + gl * 32;
      const float sx = xsum[m * p.gps + gl];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float d = dot32(cur[t].q, xg);
        acc[t][m] = __builtin_fmaf(s24[t], d, __builtin_fmaf(mn[t], sx, acc[t][m]));
      }
    }
  };
  if (streams) {
#pragma unroll
    for (int i = 0; i < D; ++i)
      if (wg0 + i < wg1) consume(r0[i], wg0 + i);
    for (int c0 = wg0 + D; c0 < wg1; c0 += D) {
      Rec r[D][T];
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int t = 0; t < T; ++t) r[i][t] = load_rec<MODE == 1>(p, tl(t), min(c0 + i, glast), lane);
#pragma unroll
      for (int i = 0; i < D; ++i)
        if (c0 + i < wg1) consume(r[i], c0 + i);
    }
  }
  }   // !mfd

  // ---- the kw waves of a slot: sum their shares in wave order into wave kwv == 0. The reads are unrolled to the
  // largest kw (the workgroup's wave count) with clamped indices, so they issue back to back and wait once; the
  // entries past kw add an exact zero.
  if (p.kw > 1) {
    constexpr int KWMAX = M <= 2 ? 16 : 8;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      __syncthreads();
#pragma unroll
      for (int t = 0; t < T; ++t) red[(wv * T + t) * 64 + lane] = acc[t][m];
      __syncthreads();
      if (kwv == 0) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float v[KWMAX];
#pragma unroll
          for (int j = 0; j < KWMAX; ++j) v[j] = red[((wv + min(j, p.kw - 1)) * T + t) * 64 + lane];
          float s = v[0];
#pragma unroll
          for (int j = 1; j < KWMAX; ++j) s += j < p.kw ? v[j] : 0.0f;
          acc[t][m] = s;
        }
      }
    }
  }

  // ---- one K-slice per split: the epilogue straight from registers
  const bool owner = active && kwv == 0;
  auto epi = [&](int sp, int m, int t0, float v0, float v1) {
    if (coh_out) epilogue<true>(p, sp, m, t0, lane, v0, v1);
    else epilogue<false>(p, sp, m, t0, lane, v0, v1);
  };
  if (p.nks == 1) {
    if (owner) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if (MODE == 2) {
          epi(split, m, tile[0], acc[0][m], acc[T - 1][m]);
        } else {
#pragma unroll
          for (int t = 0; t < T; ++t)
            if (tile[t] < p.NT) epi(split, m, tile[t], acc[t][m], 0.0f);
        }
      }
    }
    return true;
  }

  // ---- several K-slices per split: partials -> workspace; the last workgroup of (split, tile block) to arrive
  // reduces them in K-slice order. The workspace is uncached device memory, written and read with device-scope
  // accesses (no cache of any level serves a stale line, also to a persistent chain workgroup that reduced the same
  // slots for an earlier op): a partial is in memory once its store is acknowledged, so no fence (a device-scope
  // release / acquire writes back / invalidates the whole L2 of the XCD) is needed: every wave waits for its own
  // stores, then one thread counts the workgroup's arrival.
  const size_t sliceBase = (size_t)(split * p.nks) * M * p.rowsTot;
  if (owner) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int row = (MODE == 2 && t == 1) ? p.N + tile[0] * 64 + lane : tile[t] * 64 + lane;
      if (MODE != 1 || tile[t] < p.NT) {
#pragma unroll
        for (int m = 0; m < M; ++m) stf<true>(&p.part[sliceBase + ((size_t)ks * M + m) * p.rowsTot + row], acc[t][m]);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);   // every wave: its partials (uncached memory) are written before the arrival count
  __syncthreads();
  if (tid == 0) {
    auto* c = P0_GLOBAL(unsigned, p.cnt + (size_t)split * p.ntb + bx);
    const unsigned prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == (unsigned)(p.nks - 1);
    if (last) {
      __hip_atomic_exchange(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // leave the counter at zero
    }
    *s_last = last;
  }
  __syncthreads();
  const bool last = *s_last != 0;
  if (!last || !owner) return last;

  // the partials of SB K-slices (every x row and tile) are loaded together and then added in K-slice order: one
  // memory round trip per SB slices, where a load per add took one per partial
  constexpr int SB = M * T >= 16 ? 1 : 16 / (M * T);
  float tot[T][M];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int m = 0; m < M; ++m) tot[t][m] = 0.0f;
  for (int s0 = 0; s0 < p.nks; s0 += SB) {
    float v[SB][T][M];
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const int s = min(s0 + j, p.nks - 1);   // past the last slice: re-read it (in bounds, not added)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int row = (MODE == 2 && t == 1) ? p.N + tile[0] * 64 + lane : tile[t] * 64 + lane;
        const bool live = MODE != 1 || tile[t] < p.NT;
#pragma unroll
        for (int m = 0; m < M; ++m)
          v[j][t][m] = live ? ldf<true>(&p.part[sliceBase + ((size_t)s * M + m) * p.rowsTot + row]) : 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < SB; ++j)
      if (s0 + j < p.nks) {
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int m = 0; m < M; ++m) tot[t][m] += v[j][t][m];
      }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if (MODE == 2) {
      epi(split, m, tile[0], tot[0][m], tot[T - 1][m]);
    } else {
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (tile[t] < p.NT) epi(split, m, tile[t], tot[t][m], 0.0f);
    }
  }
  return true;
}

// ---- staged chain ops (mode 3). A workgroup's share of the op is a few units of 16-row blocks; it copies their
// records into LDS with LDS-DMA loads (global_load_lds_dwordx4: no registers, no ALU) BEFORE it waits for the
// producing op, so the weights stream while the chain's previous op finishes, and after the wait only x' is read
// from memory. Every unit holds whole rows of one split, so no partial sum leaves the workgroup.
//
// LDS per 16-row part (16 rows of one weight tile, the split's groups, padded to ngp, a multiple of 16):
//   codes  [ngp][16 rows][16 B] (ngp 256 B)  then  scale/min  [ngp][16 rows][4 B] (ngp 64 B)
// One 1-KB DMA instruction moves the codes of 4 groups (lane l: group 4 i + l / 16, row l % 16) or the scale words of
// 16 groups (lane l: group 16 j + l / 4, rows 4 (l % 4) .. + 3). The arithmetic maps thread t to the (group, row)
// pairs t, t + 64 W, ... of a part (pair p = group 16 + row, so a row's lanes sit 16 apart): dot32 against the
// group's x', scaled, summed over the wave's 4 groups with two cross-lane adds, then over the waves in wave order.
constexpr int kStageRows = 16;

// position of workgroup b in the dealing order: consecutive positions on one XCD (workgroups are dispatched to the 8
// XCDs round-robin), so units that share records' cache lines share an L2
__device__ __forceinline__ int stage_pos(int b, int G) { return (G & 7) ? b : (b & 7) * (G >> 3) + (b >> 3); }

template <int M, int W, class Ready>
__device__ __forceinline__ void staged_op(const GemvP& p, int b, int G, float* smem, Ready&& ready) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pos = stage_pos(b, G);
  const int first = pos >= p.scur ? pos - p.scur : pos - p.scur + G;   // this workgroup's first unit
  if (first >= p.su) return;
  const int nu = (p.su - first + G - 1) / G;
  const int parts = p.epi == P0_EPI_GEGLU ? 2 : 1, nrb = p.snrb, ngp = p.sngp;
  const int nrp = nu * nrb * parts;
  // every unit of a workgroup has the same split (the host deals split-minor units only when the split count
  // divides the grid)
  const int split = first % p.nsplit;
  const int gA = split * (p.kPer >> 5);
  const int ngs = (min(p.K, (split + 1) * p.kPer) >> 5) - gA;
  const int RPB = ngp * 320, IPR = ngp / 4 + ngp / 16;
  uint8_t* const wl = (uint8_t*)smem + p.swoff;
  float* const xs = smem;                  // [M][32 ngp]
  float* const xsum = smem + M * ngp * 32; // [M][ngp]
  float* const red = smem + p.sred;        // [nrp][M][W][16]

  // rows of part rp: unit j = rp / (nrb parts), block r, part (0 gate / plain, 1 up)
  auto part_row = [&](int rp) -> int {
    const int j = rp / (nrb * parts), rem = rp - j * (nrb * parts), r = rem / parts, pt = rem - r * parts;
    const int rb = (first + j * G) / p.nsplit;
    return (rb * nrb + r) * kStageRows + (pt ? p.N : 0);
  };

  __syncthreads();   // the previous op of this workgroup is done with the LDS
  for (int k = wv; k < nrp * IPR; k += W) {
    const int rp = k / IPR, i = k - rp * IPR;
    const int n = part_row(rp);
    const uint8_t* tb = p.w + ((int64_t)(n >> 6) * p.wG + gA) * 1280;
    const int r0 = n & 63;
    const uint8_t* src;
    uint8_t* dst;
    if (i < ngp / 4) {
      const int gi = min(4 * i + (lane >> 4), ngs - 1);   // padding groups re-read the last group (in bounds)
      src = tb + (int64_t)gi * 1280 + (r0 + (lane & 15)) * 16;
      dst = wl + rp * RPB + i * 1024;
    } else {
      const int j = i - ngp / 4;
      const int gi = min(16 * j + (lane >> 2), ngs - 1);
      src = tb + (int64_t)gi * 1280 + 1024 + (r0 + 4 * (lane & 3)) * 4;
      dst = wl + rp * RPB + ngp * 256 + j * 1024;
    }
    __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
  }
  if (!ready()) return;
  if (p.coh & 1) stage_x<M, true>(p, gA, gA + ngs, ngp, xs, xsum);
  else stage_x<M, false>(p, gA, gA + ngs, ngp, xs, xsum);
  __builtin_amdgcn_s_waitcnt(0);   // this wave's DMA loads have landed in LDS
  __syncthreads();

  const int npairs = ngs * kStageRows;
  for (int rp = 0; rp < nrp; ++rp) {
    const uint8_t* cb = wl + rp * RPB;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    for (int pp = tid; pp < npairs; pp += 64 * W) {
      const u32x4 q = *(const u32x4l*)(cb + pp * 16);
      const uint32_t sm = *(const uint32_t*)(cb + ngp * 256 + pp * 4);
      const int gi = pp >> 4;
      const float s24 = h2f_lo(sm) * 16777216.0f, mn = h2f_hi(sm);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float d = dot32(q, xs + m * ngp * 32 + gi * 32);
        acc[m] = __builtin_fmaf(s24, d, __builtin_fmaf(mn, xsum[m * ngp + gi], acc[m]));
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v = acc[m];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (lane < 16) red[((rp * M + m) * W + wv) * 16 + lane] = v;
    }
  }
  __syncthreads();

  // epilogue: thread t -> row t of the workgroup's share (a whole 64-row tile per wave for a softcap unit)
  const int rows = nu * nrb * kStageRows;
  for (int t0 = 0; t0 < rows; t0 += 64 * W) {
    const int t = t0 + tid;
    if (t0 + (tid & ~63) >= rows) break;   // whole waves leave together (softcap's wave argmax needs all 64 lanes)
    const int tt = min(t, rows - 1);
    const int j = tt / (nrb * kStageRows), rr = tt - j * (nrb * kStageRows);
    const int rpg = (j * nrb + rr / kStageRows) * parts, r16 = rr & 15;
    const int n = (first + j * G) / p.nsplit * nrb * kStageRows + rr;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) v0 += red[((rpg * M + m) * W + w) * 16 + r16];
      if (parts == 2) {
#pragma unroll
        for (int w = 0; w < W; ++w) v1 += red[(((rpg + 1) * M + m) * W + w) * 16 + r16];
      }
      if (t < rows) {
        if (p.coh & 2) epilogue<true>(p, split, m, n >> 6, n & 63, v0, v1);
        else epilogue<false>(p, split, m, n >> 6, n & 63, v0, v1);
      }
    }
  }
}

// One op, one launch: grid (tile blocks, splits x K-slices). Up to 16 waves per workgroup for M <= 2; 8 for larger
// M, whose accumulators need the registers (128 VGPRs per lane at 16 waves would spill).
template <int M, int MODE>
__global__ __launch_bounds__(M <= 2 ? 1024 : 512) void q4_gemv_kernel(GemvP p) {
  extern __shared__ __attribute__((aligned(16))) float smem[];   // 16-byte aligned: ds_read_b128 of x
  __shared__ int s_last;
  gemv_item<M, MODE, false>(p, blockIdx.x, blockIdx.y, smem, &s_last, [] { return true; });
}

// the same GEMV-M on the matrix cores (M >= 2; the host sends p.mf calls here, with at most 8 waves per workgroup)
template <int M, int MODE>
__global__ __launch_bounds__(512) void q4_gemv_mf_kernel(GemvP p) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  __shared__ int s_last;
  auto ready = [] { return true; };
  gemv_item<M, MODE, false, decltype(ready)&, true>(p, blockIdx.x, blockIdx.y, smem, &s_last, ready);
}

// ---- the chain executor: a recorded sequence of GEMV ops in ONE persistent launch (the analogue of the reference's
// per-token command buffer, engine/llm/drunner.js:1-8). Op i may read what ops < i wrote, so its items wait until op
// i - 1 has written all of its outputs; each workgroup issues its first item's weight loads BEFORE that wait, so the
// next op's weights stream while the previous op finishes. Items are dealt to workgroups round-robin; every
// workgroup of the grid is resident at once (the grid is sized from the occupancy), so a wait always ends. Each wait
// is also bounded: past `spin_limit` polls it sets the timed-out word, and every workgroup abandons the rest of the
// chain at its next wait, so a launch always finishes (its results are then invalid and reported as such).
//
// Completion is published per workgroup: a workgroup done with its units or items of op i (or with none) waits
// until its output stores are acknowledged, then writes the run's tag into its flag of op i. A workgroup about to
// read op i - 1's outputs polls op i - 1's flags of all workgroups: one wave loads them (G 4-byte words, one coalesced
// load per lane per 64 workgroups) and votes. No atomic sits on the path, and no workgroup waits for another's
// signal to be relayed. The flags exist in kFlagCopies copies, one per XCD, every producer writing each copy: a
// waiter polls the copy of its own XCD (workgroup b runs on XCD b % 8), so each copy's lines serve 32 pollers
// instead of 256.
// The tag is the last run's tag + 1, read from the state at the start; workgroup 0 stores it back once every
// workgroup has published op 0 (so has read it), so a chain runs any number of times with no reset (capturable).
// State (u32 words): [0] last tag, [kCtrStride] timed out (sticky until p0_chain_status reads and resets it; runs
// started meanwhile do nothing), then from word 2 kCtrStride the flags, (copy c, op i, workgroup w) at
// (c n_ops + i) Gp + w with Gp = G rounded up to whole 256-byte lines.
constexpr int kCtrStride = 32;
constexpr int kFlagCopies = 8;
constexpr int kChainMaxGrid = 512;

__device__ __forceinline__ unsigned ld_coh(const unsigned* a) {
  return __hip_atomic_load(P0_GLOBAL(unsigned, const_cast<unsigned*>(a)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(unsigned* a, unsigned v) {
  __hip_atomic_store(P0_GLOBAL(unsigned, a), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__host__ __device__ constexpr int chain_flag_stride(int G) { return (G + 63) & ~63; }
// words of chain state for n_ops ops on G workgroups
__host__ __device__ constexpr size_t chain_state_words(int n_ops, int G) {
  return (size_t)2 * kCtrStride + (size_t)kFlagCopies * n_ops * chain_flag_stride(G);
}

// true once every one of the G flags at f holds tag: one wave, four loads per lane issued before any is compared
__device__ __forceinline__ bool flags_set(const unsigned* f, int G, unsigned tag, int lane) {
  bool ok = true;
  for (int j0 = 0; j0 < G; j0 += 256) {
    unsigned v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = ld_coh(f + min(j0 + j * 64 + lane, G - 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) ok = ok && v[j] == tag;
  }
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

template <int M, int W>
__global__ __launch_bounds__(64 * W) void q4_gemv_chain_kernel(const GemvP* __restrict__ ops, int n_ops,
                                                               unsigned* __restrict__ st, int spin_limit) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  __shared__ int s_last, s_go;
  __shared__ unsigned s_tag;
  const int tid = threadIdx.x, lane = tid & 63, G = gridDim.x, b = blockIdx.x;
  const int Gp = chain_flag_stride(G);
  unsigned* const timed_out = st + kCtrStride;
  unsigned* const flags = st + 2 * kCtrStride;
  const unsigned* const mine = flags + (size_t)(b % kFlagCopies) * n_ops * Gp;   // this XCD's copy
  if (tid == 0) {
    s_tag = ld_coh(st) + 1;
    s_go = ld_coh(timed_out) == 0u;   // an earlier run gave up: do nothing until p0_chain_status resets the state
  }
  __syncthreads();
  const unsigned tag = s_tag;
  const bool started = s_go != 0;
  bool abandon = !started;
  // wave 0 waits until the G flags at f hold this run's tag; false (in every thread) when the wait gave up
  auto wait_flags = [&](const unsigned* f) -> bool {
    if (tid < 64) {
      // spin_limit < 0: the host asks every wait to give up at once (tests of the timed-out path)
      int go = spin_limit >= 0;
      for (int spins = 0; go && !flags_set(f, G, tag, lane); ++spins) {
        if (spins >= spin_limit || (spins % 64 == 63 && ld_coh(timed_out))) go = 0;
        else __builtin_amdgcn_s_sleep(1);
      }
      if (lane == 0) {
        if (!go) atomicOr(timed_out, 1u);
        s_go = go;
      }
    }
    __syncthreads();
    return s_go != 0;
  };
  for (int i = 0; i < n_ops && !abandon; ++i) {
    const GemvP& p = op_at(ops, i);
    bool waited = i == 0;
    auto ready = [&]() -> bool {
      if (waited) return true;   // only the workgroup's first item of op i waits for op i - 1
      // op i - 1's outputs are read with coherent loads: no L2 invalidate
      abandon = !wait_flags(mine + (size_t)(i - 1) * Gp);
      waited = true;
      return !abandon;
    };
    if (p.mode == 3) {
      staged_op<M, W>(p, b, G, smem, ready);
    } else {
      const int items = p.ntb * p.nsplit * p.nks;
      for (int it = b; it < items; it += G) {
        const int bx = it % p.ntb, by = it / p.ntb;
        if (p.mode == 0) gemv_item<M, 0, true>(p, bx, by, smem, &s_last, ready);
        else if (p.mode == 1) gemv_item<M, 1, true>(p, bx, by, smem, &s_last, ready);
        else gemv_item<M, 2, true>(p, bx, by, smem, &s_last, ready);
        if (abandon) break;
      }
    }
    if (abandon) break;
    // every wave's coherent output stores are complete (acknowledged) before the flag: no L2 writeback
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid < kFlagCopies) st_coh(flags + ((size_t)tid * n_ops + i) * Gp + b, tag);
  }
  // every workgroup has read this run's tag once all have published op 0: store it back for the next run
  if (b == 0 && !abandon && wait_flags(flags + 0) && tid == 0) st_coh(st, tag);
  __builtin_amdgcn_s_waitcnt(0);   // an abandoned staged op may still have LDS-DMA loads in flight
}

// ---- kernel tables: each M's kernels are instantiated in one of the gemv_m*.hip units (parallel compilation)
typedef void (*gemv_kernel_t)(GemvP);
typedef void (*chain_kernel_t)(const GemvP*, int, unsigned*, int);

template <int M>
gemv_kernel_t pick_m(int mode) {   // modes 3..5: modes 0..2 on the matrix cores (M >= 2)
  if constexpr (M >= 2) {
    if (mode == 3) return q4_gemv_mf_kernel<M, 0>;
    if (mode == 4) return q4_gemv_mf_kernel<M, 1>;
    if (mode == 5) return q4_gemv_mf_kernel<M, 2>;
  }
  if (mode == 0) return q4_gemv_kernel<M, 0>;
  if (mode == 1) return q4_gemv_kernel<M, 1>;
  return q4_gemv_kernel<M, 2>;
}

template <int M>
chain_kernel_t pick_chain_m(int W) {   // 16-wave chain workgroups for M = 1, 8-wave ones for every M
  if (M == 1 && W == 16) return q4_gemv_chain_kernel<M, (M == 1 ? 16 : 8)>;
  return q4_gemv_chain_kernel<M, 8>;
}

// the q8g64s.t64 GEMV (gemv_q8.hip): the kernel for M rows and its LDS bytes
typedef void (*q8_kernel_t)(GemvP);
q8_kernel_t q8_kernel(int M);
q8_kernel_t q8_gemv1(bool geglu);   // M = 1, splits of at most 3072 k: 16 waves, the records in flight together
size_t q8_gemv1_lds_bytes();
size_t q8_lds_bytes(int M);

// the pipelined chain (chain_pipe.hip) for M <= pipe_max_m() rows of x: its kernels and their shape
chain_kernel_t pipe_chain_kernel(int M, bool q8);   // q8 (M = 1 only): the instantiation that also runs q8 ops
int pipe_lds_bytes(int M);
int pipe_waves();
int pipe_ring_slots(int M);
int pipe_spread_parts(int M);
int pipe_max_m();
int pipe_cfg_word();   // state word of the loader count (the next word: slots in flight per loader)
// the wide pipelined chain (chain_wide.hip) for pipe_max_m() < M <= wide_max_m() rows of x, one pass
chain_kernel_t wide_chain_kernel(int M);
int wide_lds_bytes(int M);
int wide_ring_slots(int M);
int wide_max_m();

#define P0_GEMV_EXTERN(M) \
  extern template gemv_kernel_t pick_m<M>(int); \
  extern template chain_kernel_t pick_chain_m<M>(int);
P0_GEMV_EXTERN(1) P0_GEMV_EXTERN(2) P0_GEMV_EXTERN(3) P0_GEMV_EXTERN(4)
P0_GEMV_EXTERN(5) P0_GEMV_EXTERN(6) P0_GEMV_EXTERN(7) P0_GEMV_EXTERN(8)
P0_GEMV_EXTERN(9) P0_GEMV_EXTERN(10) P0_GEMV_EXTERN(11) P0_GEMV_EXTERN(12)
P0_GEMV_EXTERN(13) P0_GEMV_EXTERN(14) P0_GEMV_EXTERN(15) P0_GEMV_EXTERN(16)
#undef P0_GEMV_EXTERN

}  // namespace p0
