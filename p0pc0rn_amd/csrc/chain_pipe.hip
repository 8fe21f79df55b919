// chain_pipe.hip - the pipelined GEMV chain for M = 1 (a decode step's GEMVs in ONE persistent launch, the analogue of
// the reference's per-token command buffer, engine/llm/drunner.js:1-8). The planning is in gemv.hip (plan_pipe);
// the op arithmetic, prologues and epilogues are those of gemv_kernels.hpp.
//
// Why a second chain kernel. A decode step is 121 dependent GEMVs of 2.6-21 MB: each op can start its arithmetic
// only once the previous op has written all of its outputs, so the step is a chain of hand-offs, and every hand-off
// costs memory round trips. A wave's loads complete in order, so a wave that has weight loads in flight cannot see a
// completion flag or an activation before those loads land: a workgroup that streams its weights after the hand-off
// puts the whole weight transfer on the chain's critical path, and one that issues them just before still puts the
// rest of the transfer in front of its poll and its x loads. Here the roles are split by wave:
//
//  * 4 loader waves stream every op's weight share into a ring of 12 LDS slots with LDS-DMA loads
//    (global_load_lds_dwordx4), ops ahead of the arithmetic, as far as the ring has room. They never touch
//    activations or flags, so their loads delay nothing but the next slot.
//  * 8 compute waves wait for the previous op (one wave polls its XCD's copy of the completion flags), stage x',
//    take the slots as the loaders publish them, reduce, run the epilogue, and publish this workgroup's completion.
//    They synchronise among themselves through an LDS counter (the hardware barrier would also wait for the
//    loaders), and run at a higher wave priority than the loaders, so the arbiter issues the critical path first.
//
// Work split. Every op is cut into units of 16 rows (64 for a softcap, whose tile maximum needs a whole 64-row tile;
// a geglu unit also holds the matching up rows) x one split (kPer); unit u goes to workgroup position
// (scur + u) mod G (consecutive positions on one XCD). A slot is 16 rows x 32 groups of one unit (10 KB): the rows'
// codes [32 groups][16 rows][16 B] then their scale words [32][16][4 B]. A small share (at most a ring of slots) is
// computed by all 8 compute waves together, one (group, row) pair per lane per slot, and reduced once; a large one
// (the lm_head) by one wave per unit, each lane taking 8 pairs per slot, so the waves stream independently.
#include "chain_common.hpp"

namespace p0 {

constexpr int kPipeMaxM = 5;                 // x rows a pipelined chain takes (gemvM verify passes up to 5)

// LDS layout (bytes) for M rows of x. M = 1 takes splits of up to 3072 k (gemv: kch <= 3072), M > 1 up to 2048
// (gemvM caps kPer at 2048); the ring gives way to the M rows of x' and of the reductions.
template <int M>
struct PipeL {
  static constexpr int KL = M == 1 ? 3072 : 2048;                   // largest split
  static constexpr int RedRp = M == 1 ? 16 : 4;                     // spread shares: most 16-row parts per workgroup
  static constexpr int Ring = M <= 2 ? 12 : M == 3 ? 11 : M == 4 ? 9 : 8;   // slots in the ring
  // x' [M][split] (odd k scaled 1/16 for q4); for M > 1 on the matrix cores, the same bytes hold the fp16 hi / lo A
  // operands (stage_x_mf's layout)
  static constexpr int OffXs = Ring * kSlotB;
  // group sums [M][split / 32]; M > 1 on the matrix cores: [split / 32][16]
  static constexpr int OffXsum = OffXs + M * KL * 4;
  static constexpr int OffRed = OffXsum + (M == 1 ? 1 : 16) * (KL / 32) * 4;   // spread: [part][m][compute wave][16 rows]
  static constexpr int OffWred = OffRed + RedRp * M * kPC * 16 * 4; // per wave: [compute wave][m][2][64 rows]
  static constexpr int OffCtl = OffWred + kPC * M * 2 * 64 * 4;     // control words
  static constexpr int CtlFull = 0, CtlRel = Ring, CtlBar = 2 * Ring, CtlStop = 2 * Ring + 1, CtlGo = 2 * Ring + 2,
                       CtlTag = 2 * Ring + 3, CtlBad = 2 * Ring + 4, CtlWords = 2 * Ring + 5;
  // M > 1, an op that stages the next op's x' (GemvP::stgOut) with an rms prologue: each compute thread's norm weight
  // [512], then the rstd of each x row [16]
  static constexpr int OffStg = OffCtl + CtlWords * 4;
  static constexpr int Lds = OffStg + (M > 1 ? (512 + 16) * 4 : 0);
  static_assert(Lds <= 160 * 1024 - 256, "pipelined chain LDS");
  static_assert(RedRp * M * kPC * 16 >= kAuxLdsFloats, "the aux ops' trees use the reduction area");
};

__host__ int pipe_lds_bytes(int M) {
  return M == 1 ? PipeL<1>::Lds : M == 2 ? PipeL<2>::Lds : M == 3 ? PipeL<3>::Lds : M == 4 ? PipeL<4>::Lds : PipeL<5>::Lds;
}
__host__ int pipe_waves() { return kPW; }
__host__ int pipe_ring_slots(int M) {
  return M == 1 ? PipeL<1>::Ring : M == 2 ? PipeL<2>::Ring : M == 3 ? PipeL<3>::Ring : M == 4 ? PipeL<4>::Ring : PipeL<5>::Ring;
}
__host__ int pipe_spread_parts(int M) { return M == 1 ? PipeL<1>::RedRp : PipeL<2>::RedRp; }
__host__ int pipe_max_m() { return kPipeMaxM; }
__host__ int pipe_cfg_word() { return kCfgLoaders; }

// q8g64s.t64 arithmetic: sum over 16 k of (code + 128) x' (the codes' sign bits flipped make them unsigned bytes,
// which convert with one instruction each; the group's 128 sum x' is taken off after the quarters are added)
__device__ __forceinline__ float dot16_q8(const u32x4 q, const float* __restrict__ x) {
  const float4* x4 = (const float4*)x;
  const uint32_t u[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
  float da = 0.0f, db = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 xv = x4[w];
    da = __builtin_fmaf((float)(u[w] & 0xFFu), xv.x, da);
    db = __builtin_fmaf((float)((u[w] >> 8) & 0xFFu), xv.y, db);
    da = __builtin_fmaf((float)((u[w] >> 16) & 0xFFu), xv.z, da);
    db = __builtin_fmaf((float)(u[w] >> 24), xv.w, db);
  }
  return da + db;
}
// the 16 biased codes of q as floats, once for all M x rows (dot16_q8's conversions)
__device__ __forceinline__ void codes16_q8(const u32x4 q, float (&f)[16]) {
  const uint32_t u[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    f[4 * w] = (float)(u[w] & 0xFFu);
    f[4 * w + 1] = (float)((u[w] >> 8) & 0xFFu);
    f[4 * w + 2] = (float)((u[w] >> 16) & 0xFFu);
    f[4 * w + 3] = (float)(u[w] >> 24);
  }
}
// dot16_q8 on codes16_q8's floats: the same products in the same order
__device__ __forceinline__ float dot16f_q8(const float (&f)[16], const float* __restrict__ x) {
  const float4* x4 = (const float4*)x;
  float da = 0.0f, db = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 xv = x4[w];
    da = __builtin_fmaf(f[4 * w], xv.x, da);
    db = __builtin_fmaf(f[4 * w + 1], xv.y, db);
    da = __builtin_fmaf(f[4 * w + 2], xv.z, da);
    db = __builtin_fmaf(f[4 * w + 3], xv.w, db);
  }
  return da + db;
}
__device__ __forceinline__ float h2f_u16(const uint8_t* p) { return (float)*(const _Float16*)p; }
// v summed over lanes l, l ^ 8, l ^ 16, l ^ 24, ... (lane bits 3-5), with VALU lane moves only: a DPP rotation by 8
// inside each 16-lane row, then the gfx950 row and half swaps (permlane16 / permlane32), each of which hands back
// the value and its partner's in two registers
__device__ __forceinline__ float sum_lanes_8_16_32(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
// dot32 (gemv_kernels.hpp) against a group's 32 x' values held in registers: the same products in the same order
__device__ __forceinline__ float dot32r(const u32x4 q, const float4 (&x4)[8]) {
  const uint32_t u[4] = {q.x, q.y, q.z, q.w};
  float da = 0.0f, db = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 xa = x4[2 * w], xb = x4[2 * w + 1];
    const uint32_t v = u[w], v8 = v >> 8;
    const h2_t a = __builtin_bit_cast(h2_t, v & 0x000F000Fu);
    const h2_t b = __builtin_bit_cast(h2_t, v & 0x00F000F0u);
    const h2_t c = __builtin_bit_cast(h2_t, v8 & 0x000F000Fu);
    const h2_t e = __builtin_bit_cast(h2_t, v8 & 0x00F000F0u);
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

// x' of an M > 1 op's split (raw or rms prologue), every row in one batch of loads. Thread t of the compute threads
// takes four k of one code word: group g = t / 8 of the split, word w = (t / 2) % 4, k 8 w + {2 e, 2 e + 1, 2 e + 4,
// 2 e + 5} with e = t % 2, which are the word's nibble positions 4 e .. 4 e + 3 (the matrix-core operand order 0, 4,
// 1, 5 | 2, 6, 3, 7): so an MF thread writes its hi and lo halves with one 8-byte store each. Its loads for every row
// are in flight together (norm weights once for all rows, the rows' rstd slots once per row). The group sums are
// sum32's balanced tree over the group's 32 k, exactly: pairs in the thread, pairs of pairs with lane ^ 1, octets,
// octet pairs with lane ^ 2, halves with the mirrored half of the 8 lanes. The values are prologue_batch's. MF:
// stage_x_mf's fp16 hi / lo A operands and [group][16] sums (rows >= M zero), and the result is its "too large" flag;
// else stage_x's fp32 layout (result false).
template <int M, bool COH, bool MF>
__device__ __forceinline__ bool stage_rows(const GemvP& p, int g0, int g1, int gps, float* xs, float* xsum, int t) {
  typedef _Float16 half4v __attribute__((ext_vector_type(4)));
  const int KL = gps * 32, kb = g0 * 32, ke = g1 * 32;
  const bool rms = p.pro == P0_PRO_RMS;
  const int g = t >> 3, w = (t >> 1) & 3, e = t & 1;
  const int kl = 32 * g + 8 * w + 2 * e;   // the thread's k: kl, kl + 1, kl + 4, kl + 5 of the split
  const bool act = g < gps;                // whole 8-lane groups
  constexpr int kOff[4] = {0, 1, 4, 5};
  float x[M][4], nw[4], st[M];
  bool in[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) in[j] = act && kb + kl + kOff[j] < ke;
  const bool vec = ((uintptr_t)(p.X + p.rowB) & 15) == 0 && (p.ldx & 3) == 0 &&
                   (!rms || ((uintptr_t)(p.NW + p.nOff) & 15) == 0);
  if (vec) {
    // 16-byte loads of k 8w + 4e .. + 3 (one 1 KB run per row and wave), then the lane pair trades two values:
    // e = 0 keeps k 0, 1 and takes 4, 5; e = 1 takes 2, 3 and keeps 6, 7
    const int k4 = act && kb + 32 * g + 8 * w + 4 * e < ke ? kb + 32 * g + 8 * w + 4 * e : ke - 4;
    auto trade = [&](const float (&r)[4], float (&o)[4]) {
      const float s0 = e ? r[0] : r[2], s1 = e ? r[1] : r[3];
      const float r0 = dpp_f<0xB1>(s0), r1 = dpp_f<0xB1>(s1);   // lane ^ 1
      o[0] = e ? r0 : r[0];
      o[1] = e ? r1 : r[1];
      o[2] = e ? r[2] : r0;
      o[3] = e ? r[3] : r1;
    };
    float raw[M][4], rn[4];
    // a raw buffer over the rows: its 16-byte loads take the device-scope cache policy (sc1) that ldf<true> gives
    // 4-byte loads
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)(p.X + p.rowB), (short)0, 0x7FFFFFFF,
                                                                        0x00020000);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const auto q = __builtin_amdgcn_raw_buffer_load_b128(xr, (m * p.ldx + k4) * 4, 0, COH ? 16 : 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) raw[m][j] = __uint_as_float(q[j]);
    }
    if (rms) {
      const float* a = &p.NW[p.nOff + k4];
      const float4 q = *(const float4*)a;
      rn[0] = q.x; rn[1] = q.y; rn[2] = q.z; rn[3] = q.w;
    }
#pragma unroll
    for (int m = 0; m < M; ++m) trade(raw[m], x[m]);
    if (rms) trade(rn, nw);
    else nw[0] = nw[1] = nw[2] = nw[3] = 1.0f;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = in[j] ? kb + kl + kOff[j] : ke - 1;
#pragma unroll
      for (int m = 0; m < M; ++m) x[m][j] = ldf<COH>(&p.X[m * p.ldx + p.rowB + k]);
      nw[j] = rms ? ldf<COH>(&p.NW[p.nOff + k]) : 1.0f;
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) st[m] = rms ? ldf<COH>(&p.ST[p.statOff + m * p.statLd]) : 1.0f;
  bool bad = false;
  _Float16* xh = (_Float16*)xs;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = in[j] ? (rms ? x[m][j] * st[m] * nw[j] : x[m][j]) : 0.0f;
    float a = v[0] + v[1], c = v[2] + v[3];   // pairs (2e, 2e + 1), (2e + 4, 2e + 5)
    a += dpp_f<0xB1>(a);                      // lane ^ 1: k 0-3 of the word
    c += dpp_f<0xB1>(c);                      // k 4-7
    float o = a + c;                          // the word's 8 k
    o += dpp_f<0x4E>(o);                      // lane ^ 2: words (0, 1), (2, 3)
    o += dpp_f<0x141>(o);                     // the other half of the 8 lanes: the group
    if (act) {
      const float xo[4] = {v[0], v[1] * 0.0625f, v[2], v[3] * 0.0625f};   // odd k pre-scaled 1/16
      if (MF) {
        half4v hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xs8 = xo[j] * kMfScale;
          hi[j] = (_Float16)xs8;
          lo[j] = (_Float16)(xs8 - (float)hi[j]);
          bad = bad || !(__builtin_fabsf(xo[j]) < kMfBig);
        }
        // word positions 4e .. 4e + 3 hold k (2e, 2e + 4, 2e + 1, 2e + 5)
        const half4v hp = {hi[0], hi[2], hi[1], hi[3]}, lp = {lo[0], lo[2], lo[1], lo[3]};
        const int at = (((g * 4 + w) * 2) * M + m) * 8 + 4 * e;
        *(half4v*)(xh + at) = hp;
        *(half4v*)(xh + at + M * 8) = lp;
        if ((t & 7) == 0) xsum[g * 16 + m] = o;
      } else {
        float* xr = xs + m * KL + kl;
        xr[0] = xo[0]; xr[1] = xo[1]; xr[4] = xo[2]; xr[5] = xo[3];
        if ((t & 7) == 0) xsum[m * gps + g] = o;
      }
    }
  }
  if (MF && act && (t & 7) == 0)
#pragma unroll
    for (int m = M; m < 16; ++m) xsum[g * 16 + m] = 0.0f;
  return bad;
}

// x' of an M > 1 op's split [g0, g1) as the previous op staged it (GemvP::stgIn, stg_half_at's layout): the split's
// A-operand bytes are one contiguous run there, copied to LDS by LDS-DMA (16 bytes a lane, 1 KB a wave instruction, no
// registers; device-scope policy: written by other CUs in this run), groups past the split zero; the group sums are the
// two 16-k halves added, rows >= M zero. The values are stage_rows's (MF) bit for bit. True if a half of the split was
// marked too large for the matrix cores (NaN). The copy has landed when the calling wave's vmcnt is 0.
template <int M>
__device__ __forceinline__ bool stage_stg(const GemvP& p, int g0, int g1, int gps, _Float16* xh, float* xsum, int t) {
  constexpr int NT = 64 * kPC, CPG = 8 * M;   // 16-byte pieces per group: 4 words x (hi, lo) x M rows x 8 halves
  constexpr int NS = (64 * 16 + NT - 1) / NT;   // group sums per thread, for splits of <= 64 groups
  const int ng = g1 - g0, wbase = t & ~63;
  const uint8_t* const src = (const uint8_t*)p.stgIn + (int64_t)g0 * CPG * 16;
  const float* ps = (const float*)(p.stgIn + (int64_t)p.K * M);
  float h[NS][2];
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int c = t + u * NT, gl = c >> 4, m = c & 15;
    h[u][0] = h[u][1] = 0.0f;
    if (gl < ng && m < M) {
      h[u][0] = ldf<true>(&ps[((g0 + gl) * 2) * M + m]);
      h[u][1] = ldf<true>(&ps[((g0 + gl) * 2 + 1) * M + m]);
    }
  }
  for (int c0 = wbase; c0 < gps * CPG; c0 += NT) {   // a whole wave per instruction: pieces c0 .. c0 + 63
    const int c = c0 + (t & 63);
    if (c0 + 64 <= ng * CPG) {
      __builtin_amdgcn_global_load_lds((const void*)(src + (int64_t)c * 16),
                                       (__attribute__((address_space(3))) void*)((uint8_t*)xh + c0 * 16), 16, 0, 16);
    } else if (c < gps * CPG) {   // the split's last pieces and the zero groups past it
      u32x4 v = {0u, 0u, 0u, 0u};
      if (c < ng * CPG) v = *P0_GLOBAL(const u32x4, (const u32x4*)(src + (int64_t)c * 16));
      *(u32x4*)((uint8_t*)xh + c * 16) = v;
    }
  }
  bool bad = false;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int c = t + u * NT;
    const float s = h[u][0] + h[u][1];
    bad = bad || s != s;
    if (c < gps * 16) xsum[c] = s;   // [group][16]: c = 16 gl + m
  }
  return bad;
}

// Q8: the instantiation for chains that hold q8g64s.t64 ops (the q4-only one carries none of their code)
template <int M, bool Q8>
__global__ __launch_bounds__(64 * kPW) void q4_chain_pipe_kernel(const GemvP* __restrict__ ops, int n_ops,
                                                                 unsigned* __restrict__ st, int spin_limit) {
  using L = PipeL<M>;
  constexpr int kRing = L::Ring;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  uint8_t* const lds = (uint8_t*)smem;
  unsigned* const ctl = (unsigned*)(lds + L::OffCtl);
  const int tid = threadIdx.x, lane = tid & 63, G = gridDim.x, b = blockIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int Gp = chain_flag_stride(G);
  unsigned* const timed_out = st + kCtrStride;
  unsigned* const flags = st + 2 * kCtrStride;
  if (tid < L::CtlWords) ctl[tid] = 0;
  if (tid == 0) {
    ctl[L::CtlTag] = ld_coh(st) + 1;
    ctl[L::CtlGo] = ld_coh(timed_out) == 0u;   // an earlier run gave up: do nothing until p0_chain_status resets it
  }
  __syncthreads();
  const unsigned tag = ctl[L::CtlTag];
  if (!ctl[L::CtlGo]) return;

  if (wv < kPL) {   // loader waves
    chain_loader<kRing, Q8, 1>(ops, n_ops, st, lds, ctl, L::CtlFull, L::CtlRel, L::CtlStop, b, G, wv, lane);
    return;
  }

  // -------------------------------------------------------------------- compute waves
  const int c = wv - kPL, tc = tid - 64 * kPL;
  // the compute waves issue ahead of the loaders on their SIMD: the chain's critical path (polls, slot arithmetic,
  // epilogue stores) no longer waits behind the loaders' DMA issue and slot-release polls; the loaders keep the ring
  // full with what the arbiter leaves them (measured: M = 1 step 0.596 -> 0.543 ms, M = 5 1.062 -> 0.973 ms; levels
  // 1, 2 and 3 alike)
  __builtin_amdgcn_s_setprio(1);
  lds_u32* const lctl = (lds_u32*)ctl;
  float* const xs = (float*)(lds + L::OffXs);
  float* const xsum = (float*)(lds + L::OffXsum);
  float* const red = (float*)(lds + L::OffRed);
  float* const wred = (float*)(lds + L::OffWred) + c * (M * 128);   // this wave's [m][2][64 rows]
  unsigned gen = 0;
  // barrier of the compute waves: a monotonic LDS counter (every compute wave adds 1 per barrier)
  auto cbar = [&]() {
    gen += kPC;
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's LDS writes are done
    if (lane == 0) ctl_add(lctl + L::CtlBar, 1u);
    while (ctl_ld(lctl + L::CtlBar) < gen) __builtin_amdgcn_s_sleep(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);
  };
  // false if the compute waves gave up meanwhile (a wave that stages its own x' gives up on its own, and the
  // loaders then stop publishing), or if this wait gave up: bounded like every other wait (the loaders run at a lower
  // wave priority; a starved loader would otherwise hold the waves here), it then marks the run timed out and stops
  // the loaders and the other waves' waits
  auto wait_slot = [&](int q) -> bool {
    for (int spins = 0; ctl_ld(lctl + L::CtlFull + q % kRing) != (unsigned)q + 1; ++spins) {
      if (ctl_ld(lctl + L::CtlStop)) return false;
      if (spins >= spin_limit) {
        if (lane == 0) {
          atomicOr(timed_out, 1u);
          ctl_st(lctl + L::CtlStop, 1u);
          ctl_st(lctl + L::CtlGo, 0u);
        }
        return false;
      }
      __builtin_amdgcn_s_sleep(0);
    }
    return true;
  };
  // the G flags at f (and at f2, when not null) hold this run's tag (wave c == 0 polls); false in every compute
  // thread if the wait gave up
  auto wait_flags = [&](const unsigned* f, const unsigned* f2) -> bool {
    if (c == 0) {
      int go = spin_limit >= 0;   // spin_limit < 0: every wait gives up at once (tests of the timed-out path)
      for (int spins = 0; go && !(flags_set(f, G, tag, lane) && (!f2 || flags_set(f2, G, tag, lane))); ++spins) {
        if (spins >= spin_limit || (spins % 64 == 63 && ld_coh(timed_out))) go = 0;
        else __builtin_amdgcn_s_sleep(1);
      }
      if (lane == 0) {
        if (!go) {
          atomicOr(timed_out, 1u);
          ctl_st(lctl + L::CtlStop, 1u);   // the loaders leave their waits
        }
        ctl_st(lctl + L::CtlGo, (unsigned)go);
      }
    }
    cbar();
    return ctl_ld(lctl + L::CtlGo) != 0;
  };
  // wave c == 0: the G flags at f hold this run's tag; on a timeout it sets the stop and go words (the workgroup leaves
  // at its next barrier)
  auto poll_flags = [&](const unsigned* f) {
    int go = spin_limit >= 0;
    for (int spins = 0; go && !flags_set(f, G, tag, lane); ++spins) {
      if (spins >= spin_limit || (spins % 64 == 63 && ld_coh(timed_out))) go = 0;
      else __builtin_amdgcn_s_sleep(1);
    }
    if (!go && lane == 0) {
      atomicOr(timed_out, 1u);
      ctl_st(lctl + L::CtlStop, 1u);
      ctl_st(lctl + L::CtlGo, 0u);
    }
  };
  // x' of groups [g0, g1) from the previous op's mailbox: each compute thread polls its own elements until all of them
  // carry this run's tag (bounded like wait_flags), then writes x' and the group sums as stage_x does (raw or rms
  // prologue: for rms the rstd slot and the thread's norm weights are loaded before the poll, as they are inputs of
  // the chain). The poll is the load: the hand-off costs one memory round trip instead of a flag round trip and then
  // an x load.
  auto stage_mbx = [&](const GemvP& p, int g0, int g1, int gps, float odd) -> bool {
    constexpr int U = 4, NT = 64 * kPC;
    const int KL = gps * 32, kb = g0 * 32, ke = g1 * 32;
    const bool rms = p.pro == P0_PRO_RMS;
    const float rstd = rms ? p.ST[p.statOff] : 1.0f;
    int go = spin_limit >= 0;
    for (int i0 = 0; go && i0 < KL; i0 += U * NT) {
      float nw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) nw[u] = rms ? p.NW[p.nOff + min(kb + i0 + u * NT + tc, ke - 1)] : 1.0f;
      unsigned long long w[U];
      for (int spins = 0;; ++spins) {
        bool ok = true;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int k = min(kb + i0 + u * NT + tc, ke - 1);   // past the slice: its last element (in bounds, unused)
          w[u] = __hip_atomic_load(P0_GLOBAL(unsigned long long, const_cast<unsigned long long*>(p.mbxIn + k)),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) ok = ok && (unsigned)(w[u] >> 32) == tag;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (!go || spins >= spin_limit || (spins % 64 == 63 && ld_coh(timed_out))) {
          go = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!go) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kl = i0 + u * NT + tc;
        const float xv = __uint_as_float((unsigned)w[u]);
        const float v = kb + kl < ke ? (rms ? xv * rstd * nw[u] : xv) : 0.0f;   // the rms prologue's own order
        const float gsum = sum32(v);
        if (kl < KL) {
          xs[kl] = (kl & 1) ? v * odd : v;   // kb is even: k and kl share parity
          if ((lane & 31) == 0) xsum[kl >> 5] = gsum;
        }
      }
    }
    if (!go && lane == 0) {
      atomicOr(timed_out, 1u);
      ctl_st(lctl + L::CtlStop, 1u);   // the loaders leave their waits
      ctl_st(lctl + L::CtlGo, 0u);
    }
    cbar();
    return ctl_ld(lctl + L::CtlGo) != 0;
  };
  // stage_mbx for the 8 groups [gw, gw + 8) of the split [g0, g1) that this compute wave computes with (the two-slot
  // spread path): element k0 + 64 u + lane per lane, so each 32-lane half holds one group, and the x' values and group
  // sums come out bit-identical to stage_mbx's. No other wave reads them, so the wave waits for no other before its
  // slots. On a timeout the wave sets the stop and go words itself (the slot waits of the other waves end on the
  // stop word), and the workgroup leaves at its next barrier.
  auto stage_mbx_wave = [&](const GemvP& p, int g0, int g1, int gw, float odd) -> bool {
    const bool rms = p.pro == P0_PRO_RMS;
    const float rstd = rms ? p.ST[p.statOff] : 1.0f;
    const int ke = g1 * 32, k0 = (g0 + gw) * 32;
    float nw[4];
    unsigned long long w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) nw[u] = rms ? p.NW[p.nOff + min(k0 + u * 64 + lane, ke - 1)] : 1.0f;
    int go = spin_limit >= 0;
    for (int spins = 0;; ++spins) {
      bool ok = true;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        w[u] = __hip_atomic_load(P0_GLOBAL(unsigned long long, const_cast<unsigned long long*>(p.mbxIn + min(k0 + u * 64 + lane, ke - 1))),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < 4; ++u) ok = ok && (unsigned)(w[u] >> 32) == tag;
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
      if (!go || spins >= spin_limit || (spins % 64 == 63 && ld_coh(timed_out))) {
        go = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!go) {
      if (lane == 0) {
        atomicOr(timed_out, 1u);
        ctl_st(lctl + L::CtlStop, 1u);   // the loaders leave their waits, the other waves their slot waits
        ctl_st(lctl + L::CtlGo, 0u);
      }
      return false;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kl = (gw + 2 * u) * 32 + lane;   // offset in the split
      const float xv = __uint_as_float((unsigned)w[u]);
      const float v = k0 + u * 64 + lane < ke ? (rms ? xv * rstd * nw[u] : xv) : 0.0f;
      const float gsum = sum32(v);
      xs[kl] = (kl & 1) ? v * odd : v;
      if ((lane & 31) == 0) xsum[kl >> 5] = gsum;
    }
    // the wave reads its x' back right behind these writes: the LDS serves one wave's accesses in order, so no
    // lgkmcnt wait; the wavefront fences keep the compiler from moving the reads above the other lanes' writes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return true;
  };
  // this op's rows, with their values as stored, into its mailbox (after the epilogue's own stores): the element of
  // split `split`, row n sits at its offset from Y, split * ldy + n
  auto post_mbx = [&](const EpiP& p, int split, int n, float v) {
    __hip_atomic_store(P0_GLOBAL(unsigned long long, p.mbxOut + (int64_t)split * p.ldy + n),
                       ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  const unsigned* const mine = flags + (size_t)(b % kFlagCopies) * n_ops * Gp;   // this XCD's copy
  int q0 = 0;
  bool abandon = false;
  for (int i = 0; i < n_ops; ++i) {
    const GemvP& p = op_at(ops, i);
    if (p.kind != kOpGemv) {
      // copy / argmax / rowstats / normadd (chain_aux.hpp): the workgroups that take part wait for op i - 1 in every
      // workgroup, run the op in the reduction area and publish once their stores are acknowledged; the others publish
      // at once (their flag of op i says, as always, that they are done with every op up to i)
      if (aux_worker(p, b)) {
        if (p.abefore >= 0 && !wait_flags(mine + (size_t)p.abefore * Gp, nullptr)) {
          abandon = true;
          break;
        }
        gen = aux_run(&p, b, G, tc, (lds_f32*)red, lctl + L::CtlBar, gen);
        __builtin_amdgcn_s_waitcnt(0);
        cbar();
      }
      if (c == 0 && lane < kFlagCopies) st_coh(flags + ((size_t)lane * n_ops + i) * Gp + b, tag);
      continue;
    }
    const Share s = share_of<Q8>(p, b, G);
    if (s.nu > 0) {
      const EpiP e = epi_of(p);
      // GemvP::wback: op i - wback's completion flags, loaded now by wave 0 and checked before the op's first store, so
      // that the check costs no round trip of its own when they are set by then
      const unsigned* const wf = mine + (size_t)(i - p.wback) * Gp;
      unsigned w2[4] = {tag, tag, tag, tag};
      if (p.wback && c == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w2[j] = ld_coh(wf + min(j * 64 + lane, G - 1));
      }
      auto check_wback = [&]() {   // wave c == 0, then a barrier of the compute waves
        bool ok = G <= 256;
#pragma unroll
        for (int j = 0; j < 4; ++j) ok = ok && w2[j] == tag;
        if (__builtin_amdgcn_ballot_w64(!ok) != 0) poll_flags(wf);
      };
      // a spread share's epilogue: compute thread tc -> x row m = tc / rows, row tc % rows of the share (rows x M <= 512
      // compute threads, planned so; a softcap unit is one whole wave, rows being a multiple of 64), so the M rows'
      // epilogues run side by side. Its row indices take integer divisions by per-op values; worked out here, before
      // the input wait, and pinned, they stay off the op's critical path.
      const int erows = s.nu * s.nrb * kStageRows;
      int erpg = 0, er16 = 0, en = 0, em = 0;
      if (s.spread) {
        int t = min(tc, erows - 1);
        if (M > 1) {
          const int tm = min(tc, erows * M - 1);
          em = tm / erows;
          t = tm - em * erows;
        }
        const int j = t / (s.nrb * kStageRows), rr = t - j * (s.nrb * kStageRows);
        erpg = (j * s.nrb + rr / kStageRows) * s.parts;
        er16 = rr & 15;
        en = share_row(p, s, G, j, 0, 0) + rr;
        asm volatile("" : "+v"(erpg), "+v"(er16), "+v"(en));
        if (M > 1) asm volatile("" : "+v"(em));
      }
      // M > 1, the next op's x' staged here (GemvP::stgOut): that op's rms inputs for this thread's (x row, output row),
      // loaded now, off the epilogue's path (chain inputs: no op writes them)
      // (they are parked in LDS once the input is staged, so that they hold no registers through the slots)
      const bool stg_rms = M > 1 && s.spread && p.stgOut && p.stgPro == P0_PRO_RMS;
      float stg_nwv = 1.0f, stg_stv = 1.0f;
      if (stg_rms) {
        const int64_t k = (int64_t)en - p.stgR0;
        if (s.split == p.stgSp && k >= 0 && k < p.stgK) stg_nwv = p.stgNW[p.stgNOff + k];
        if (tc < M) stg_stv = p.stgST[p.stgStatOff + tc * p.stgStatLd];
      }
      // x' of the split in 32-k groups; the q4 dot products take odd k pre-scaled 1/16, the q8 ones plain x'
      const bool q8 = Q8 && p.enc == P0_ENC_Q8G64S_T64;
      const int xg0 = q8 ? 2 * s.gA : s.gA, xg1 = q8 ? 2 * (s.gA + s.ngs) : s.gA + s.ngs;
      const int xgps = q8 ? 16 * s.nh : 32 * s.nh;
      const float odd = q8 ? 1.0f : 0.0625f;
      // M > 1 (q4, no mailboxes at M > 1): the slots' arithmetic on the matrix cores (GemvP::mf, p0_chain_tune knob 9)
      bool mf = M >= 2 && !q8 && p.mf;
      // the two-slot q4 spread path stages per wave (see stage_mbx_wave)
      const bool wave_stage = M == 1 && !q8 && s.spread && s.nh == 2 && p.mbxIn;
      bool wgo = true;
      if (wave_stage) {
        wgo = stage_mbx_wave(p, xg0, xg1, 32 * (c >> 2) + 8 * (c & 3), odd);
      } else if (p.mbxIn) {
        // op i - 1's completion is not waited for here: the mailbox words say that the elements op i reads are
        // written; the stores of op i wait for what the other workgroups may still be doing (GemvP::wback)
        if (!stage_mbx(p, xg0, xg1, xgps, odd)) {
          abandon = true;
          break;
        }
      } else {
        if (i > 0 && !wait_flags(mine + (size_t)(i - 1) * Gp, nullptr)) {
          abandon = true;
          break;
        }
        if (stg_rms) {   // the next op's rms inputs, loaded at this op's start, to LDS (read by the epilogue)
          float* const stgl = (float*)(lds + L::OffStg);
          stgl[tc] = stg_nwv;
          if (tc < M) stgl[512 + tc] = stg_stv;
        }
        // op i - 1's outputs are read with coherent loads: no L2 invalidate
        const bool rows1 = M >= 2 && !q8 && (p.pro == P0_PRO_RAW || p.pro == P0_PRO_RMS);   // stage_rows
        if (mf) {
          // M > 1: x' as the matrix cores' fp16 hi / lo operands; a workgroup that holds an x' too large for them
          // (|x'| >= 255, see stage_x_mf) stages fp32 x' instead and runs this op on the VALU
          bool bad;
          if (M > 1 && p.stgIn) {
            bad = stage_stg<M>(p, xg0, xg1, xgps, (_Float16*)xs, xsum, tc);
            __builtin_amdgcn_s_waitcnt(0);   // the LDS-DMA copy has landed (vmcnt) before the barrier
          }
          else if (rows1) bad = (p.coh & 1) ? stage_rows<M, true, true>(p, xg0, xg1, xgps, xs, xsum, tc)
                                            : stage_rows<M, false, true>(p, xg0, xg1, xgps, xs, xsum, tc);
          else bad = (p.coh & 1) ? stage_x_mf<M, true, 16>(p, xg0, xg1, xgps, (_Float16*)xs, xsum, tc, 64 * kPC)
                                 : stage_x_mf<M, false, 16>(p, xg0, xg1, xgps, (_Float16*)xs, xsum, tc, 64 * kPC);
          if (bad) ctl_st(lctl + L::CtlBad, (unsigned)i + 1);
          cbar();
          mf = ctl_ld(lctl + L::CtlBad) != (unsigned)i + 1;
        }
        if (!mf) {
          if (rows1) {
            if (p.coh & 1) stage_rows<M, true, false>(p, xg0, xg1, xgps, xs, xsum, tc);
            else stage_rows<M, false, false>(p, xg0, xg1, xgps, xs, xsum, tc);
          } else if (p.coh & 1) {
            stage_x<M, true>(p, xg0, xg1, xgps, xs, xsum, tc, 64 * kPC, odd);
          } else {
            stage_x<M, false>(p, xg0, xg1, xgps, xs, xsum, tc, 64 * kPC, odd);
          }
          cbar();
        }
      }
      const int nrp = s.nu * s.nrb * s.parts;
      float* const stgl = (float*)(lds + L::OffStg);
      if (s.spread) {
       if (q8) {
        // q8 slots: compute wave c takes group c of every slot, lane = (row lane / 4, quarter lane % 4 of the group's
        // 64 k); the quarters are added across the lane quad, the groups across the waves (red), as for q4; x row m's
        // x' starts at m xgps 32 (fp32, staged by stage_x), its 32-k group sums at m xgps
        const int rr = lane >> 2, qq = lane & 3;
        for (int rp = 0; rp < nrp; ++rp) {
          float acc[M];
#pragma unroll
          for (int m = 0; m < M; ++m) acc[m] = 0.0f;
          for (int h = 0; h < s.nh; ++h) {
            const int q = q0 + rp * s.nh + h;
            wait_slot(q);
            const uint8_t* slot = lds + (q % kRing) * kSlotB;
            const int g = 8 * h + c;   // group of the split (< 8 nh: inside the staged x')
            const u32x4 qv = *(const u32x4l*)(slot + c * 1024 + rr * 64 + qq * 16);
            const float sc = h2f_u16(slot + 8192 + c * 32 + rr * 2);
            float cf[16];
            codes16_q8(qv, cf);
#pragma unroll
            for (int m = 0; m < M; ++m) {
              float d = dot16f_q8(cf, xs + m * xgps * 32 + g * 64 + qq * 16);
              d += __shfl_xor(d, 1, 64);
              d += __shfl_xor(d, 2, 64);
              if (g < s.ngs)
                acc[m] = __builtin_fmaf(sc, d - 128.0f * (xsum[m * xgps + 2 * g] + xsum[m * xgps + 2 * g + 1]), acc[m]);
            }
          }
          if (qq == 0)
#pragma unroll
            for (int m = 0; m < M; ++m) red[((rp * M + m) * kPC + c) * 16 + rr] = acc[m];
        }
       } else if (M >= 2 && mf) {
        // M > 1 on the matrix cores: compute wave c takes groups 4c .. 4c + 3 of every slot. Per group and the slot's
        // 16 weight rows, two v_mfma_f32_16x16x32_f16 (x' hi and lo as A, the codes as B: gemv_kernels.hpp's GEMV-M
        // operands) give D[m][n]: x row m in lanes l / 16 == m / 4 (element m % 4), weight row n = l % 16, to which
        // each lane applies its row's scale and min.
        // A rows >= M read row M - 1 (finite); their D rows are never stored
        const _Float16* xh = (const _Float16*)xs;
        const int aw = lane >> 4, arow = min(lane & 15, M - 1), n16 = lane & 15;
        for (int rp = 0; rp < nrp; ++rp) {
          f4_t am = {0.0f, 0.0f, 0.0f, 0.0f};
          for (int h = 0; h < s.nh; ++h) {
            const int q = q0 + rp * s.nh + h;
            wait_slot(q);
            const uint8_t* slot = lds + (q % kRing) * kSlotB;
#pragma unroll
            for (int jg = 0; jg < 4; ++jg) {
              const int gs = 4 * c + jg, g = 32 * h + gs;   // group of the slot, of the split
              const uint32_t cw = *(const uint32_t*)(slot + (gs * 16 + n16) * 16 + aw * 4);
              const uint32_t sm = *(const uint32_t*)(slot + 8192 + (gs * 16 + n16) * 4);
              const half8_t* ap = (const half8_t*)(xh + (((g * 4 + aw) * 2) * M + arow) * 8);
              const half8_t ahi = ap[0], alo = ap[M];
              const f4_t sx = *(const f4_t*)(xsum + g * 16 + 4 * aw);
              const half8_t bq = codes_b(cw);
              f4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
              d = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bq, d, 0, 0, 0);
              const bool live = g < s.ngs;
              const float s8 = live ? h2f_lo(sm) * kMfDeq : 0.0f, mn = live ? h2f_hi(sm) : 0.0f;
#pragma unroll
              for (int e = 0; e < 4; ++e) am[e] = __builtin_fmaf(s8, d[e], __builtin_fmaf(mn, sx[e], am[e]));
            }
          }
#pragma unroll
          for (int m = 0; m < M; ++m)
            if ((lane >> 4) == (m >> 2)) red[((rp * M + m) * kPC + c) * 16 + n16] = am[m & 3];
        }
       } else if (M == 1 && s.nh == 2) {
        // splits of 33 .. 64 groups (two slots per 16-row part): compute waves 0-3 take the first half's slot of every
        // part, waves 4-7 the second's; lane = (group gl = 8 (c % 4) + lane / 8 of the half, rows lane % 8 and
        // lane % 8 + 8). The lane's 32 x' values are read into registers once for the whole share, so a part costs
        // it two code reads and two scale reads, where one pair per lane and slot would read the 32 x' values for
        // every slot (the LDS reads of all compute waves, issued together after each barrier, set the pace of the
        // slot phase). Odd groups take their two rows in the other order, so that the lanes of a read instruction
        // fall into both halves of the LDS banks.
        const int hh = c >> 2, gl = 8 * (c & 3) + (lane >> 3), r8 = lane & 7;
        const int g = 32 * hh + gl;
        const bool live = g < s.ngs;   // groups past the split add exact zeros (their x' and sums are staged as 0)
        const float4* x4 = (const float4*)(xs + g * 32);
        float4 xr[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) xr[w] = x4[w];
        const float xg = xsum[g];
        const int ra = (gl & 1) ? r8 + 8 : r8, rb = ra ^ 8;
        for (int rp = 0; wgo && rp < nrp; ++rp) {
          const int q = q0 + rp * 2 + hh;
          if (!wait_slot(q)) break;
          const uint8_t* slot = lds + (q % kRing) * kSlotB;
          const u32x4 qa = *(const u32x4l*)(slot + (gl * 16 + ra) * 16), qb = *(const u32x4l*)(slot + (gl * 16 + rb) * 16);
          const uint32_t sa = *(const uint32_t*)(slot + 8192 + (gl * 16 + ra) * 4);
          const uint32_t sb = *(const uint32_t*)(slot + 8192 + (gl * 16 + rb) * 4);
          const float ya = __builtin_fmaf(live ? h2f_lo(sa) * 16777216.0f : 0.0f, dot32r(qa, xr),
                                          (live ? h2f_hi(sa) : 0.0f) * xg);
          const float yb = __builtin_fmaf(live ? h2f_lo(sb) * 16777216.0f : 0.0f, dot32r(qb, xr),
                                          (live ? h2f_hi(sb) : 0.0f) * xg);
          // rows r8 and r8 + 8 summed over the wave's 8 groups (lane bits 3-5)
          const float lo = sum_lanes_8_16_32((gl & 1) ? yb : ya), hi = sum_lanes_8_16_32((gl & 1) ? ya : yb);
          if (lane < 8) {
            red[(rp * kPC + c) * 16 + r8] = lo;
            red[(rp * kPC + c) * 16 + r8 + 8] = hi;
          }
        }
       } else {
        // every compute lane takes pair tc = 16 group + row of each slot; a part's slots are its halves; x' row m
        // starts at m xgps 32
        const int gi = tc >> 4;
        for (int rp = 0; rp < nrp; ++rp) {
          float acc[M];
#pragma unroll
          for (int m = 0; m < M; ++m) acc[m] = 0.0f;
          for (int h = 0; h < s.nh; ++h) {
            const int q = q0 + rp * s.nh + h;
            wait_slot(q);
            const uint8_t* slot = lds + (q % kRing) * kSlotB;
            const int g = 32 * h + gi;
            const u32x4 qv = *(const u32x4l*)(slot + tc * 16);
            const uint32_t sm = *(const uint32_t*)(slot + 8192 + tc * 4);
            if (g < s.ngs) {
              const float s24 = h2f_lo(sm) * 16777216.0f, mn = h2f_hi(sm);
#pragma unroll
              for (int m = 0; m < M; ++m) {
                const float d = dot32(qv, xs + m * xgps * 32 + g * 32);
                acc[m] = __builtin_fmaf(s24, d, __builtin_fmaf(mn, xsum[m * xgps + g], acc[m]));
              }
            }
          }
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float v = acc[m];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (lane < 16) red[((rp * M + m) * kPC + c) * 16 + lane] = v;
          }
        }
       }
        // outputs that an earlier op reads or writes: that op complete in every workgroup first (GemvP::wback)
        if (p.wback && c == 0) check_wback();
        cbar();   // every slot of the share is read, every wave's row sums are in
        // did an input or flag wait give up? (read with the row sums, checked before the first store: one LDS round
        // trip for both; read by every op, since a read under a condition was waited for on its own, measured 0.8%
        // of the M = 1 step)
        const unsigned go = ctl_ld(lctl + L::CtlGo);
        if (tc < s.nslot) ctl_add(lctl + L::CtlRel + (q0 + tc) % kRing, 1u);
        // epilogue (rows and indices from the op's start)
        const int rows = erows * M, rpg = erpg, r16 = er16, n = en, m = em;
        float v0 = 0.0f, v1 = 0.0f;
        if (tc - lane < rows) {
#pragma unroll
          for (int w = 0; w < kPC; ++w) v0 += red[((rpg * M + m) * kPC + w) * 16 + r16];
          if (s.parts == 2) {
#pragma unroll
            for (int w = 0; w < kPC; ++w) v1 += red[(((rpg + 1) * M + m) * kPC + w) * 16 + r16];
          }
        }
        if (!go) {
          abandon = true;
          break;
        }
        if (tc - lane < rows) {
          if (tc < rows) {
            float yv;
            if (M == 1 && e.mbxOut && e.epi != P0_EPI_SOFTCAP) {
              // the mailbox word (what the next op waits on) goes out before the output itself
              yv = e.epi == P0_EPI_GEGLU ? gelu_tanh(v0) * v1 : v0;
              post_mbx(e, s.split, n, yv);
              float* const yp = e.epi == P0_EPI_GEGLU ? &e.Y[n] : &e.Y[s.split * e.ldy + n];
              if (e.coh & 2) stf<true>(yp, yv);
              else stf<false>(yp, yv);
            } else {
              yv = (e.coh & 2) ? epilogue<true>(e, s.split, m, n >> 6, n & 63, v0, v1)
                               : epilogue<false>(e, s.split, m, n >> 6, n & 63, v0, v1);
              if (M == 1 && e.mbxOut) post_mbx(e, s.split, n, yv);
            }
            if (M > 1 && p.stgOut) {
              // the next op's x' of (x row m, k = n - stgR0), as stage_rows computes it: the prologue in its own order,
              // odd k scaled 1/16, 2^8 x' as fp16 hi + lo; the group sum of each 16 k in the balanced tree of stage_rows
              // (pairs, quads, octets, 16: a 16-row block of this share is 16 consecutive lanes, lane % 16 = k % 16), a
              // NaN marking a half with some |x'| too large for the matrix cores. The 16-row blocks lie wholly inside or
              // outside the next op's x (stgR0 and stgK are multiples of 32), so the lane steps see whole blocks.
              const int64_t k = (int64_t)n - p.stgR0;
              if (s.split == p.stgSp && k >= 0 && k < p.stgK) {
                const float x = stg_rms ? yv * stgl[512 + m] * stgl[tc] : yv;
                const float xo = (k & 1) ? x * 0.0625f : x;
                const float xs8 = xo * kMfScale;
                const _Float16 hi = (_Float16)xs8, lo = (_Float16)(xs8 - (float)hi);
                _Float16* const sh = (_Float16*)p.stgOut;
                *P0_GLOBAL(_Float16, sh + stg_half_at(M, k, m, 0)) = hi;
                *P0_GLOBAL(_Float16, sh + stg_half_at(M, k, m, 1)) = lo;
                float g = __builtin_fabsf(xo) < kMfBig ? x : __builtin_nanf("");
                g += dpp_f<0xB1>(g);    // lane ^ 1
                g += dpp_f<0x4E>(g);    // lane ^ 2
                g += dpp_f<0x141>(g);   // the other quad of the 8 lanes
                g += dpp_f<0x140>(g);   // the other 8 of the 16
                if ((k & 15) == 0)
                  *P0_GLOBAL(float, (float*)(p.stgOut + (int64_t)p.stgK * M) + ((k >> 5) * 2 + ((k >> 4) & 1)) * M + m) = g;
              }
            }
          }
        }
      } else {
        if (p.wback) {   // as in the spread path, before the first of this share's stores
          if (c == 0) check_wback();
          cbar();
          if (!ctl_ld(lctl + L::CtlGo)) {
            abandon = true;
            break;
          }
        }
        // a large share (the lm_head), one wave per unit: lane takes pairs lane + 64 kk of each slot (group
        // 4 kk + lane / 16, row lane % 16); it copies them to registers and hands the slot back to the loaders before
        // the arithmetic, so the ring's slots spend their time in flight rather than held
        for (int j = c; j < s.nu; j += kPC) {
          for (int r = 0; r < s.nrb; ++r) {
            for (int pt = 0; pt < s.parts; ++pt) {
              float acc[M];
#pragma unroll
              for (int m = 0; m < M; ++m) acc[m] = 0.0f;
              f4_t am = {0.0f, 0.0f, 0.0f, 0.0f};   // M > 1 on the matrix cores (D layout of the spread path)
              for (int h = 0; h < s.nh; ++h) {
                const int q = q0 + slot_index(s, j, (r * s.parts + pt) * s.nh + h);
                wait_slot(q);
                const uint8_t* slot = lds + (q % kRing) * kSlotB;
                if (M >= 2 && mf) {
                  // the slot's 32 groups in 4 batches of 8 (each group: two v_mfma_f32_16x16x32_f16, as in the spread
                  // path); a batch's code and scale words go to registers first, and the slot goes back to the
                  // loaders once the last batch is read
                  const _Float16* xh = (const _Float16*)xs;   // A rows >= M: row M - 1, never stored
                  const int aw = lane >> 4, arow = min(lane & 15, M - 1), n16 = lane & 15;
#pragma unroll 1
                  for (int b8 = 0; b8 < 4; ++b8) {
                    uint32_t cw[8], smw[8];
#pragma unroll
                    for (int gg = 0; gg < 8; ++gg) {
                      const int gs = 8 * b8 + gg;
                      cw[gg] = *(const uint32_t*)(slot + (gs * 16 + n16) * 16 + aw * 4);
                      smw[gg] = *(const uint32_t*)(slot + 8192 + (gs * 16 + n16) * 4);
                    }
                    if (b8 == 3) {
                      __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's reads of the slot are done
                      if (lane == 0) ctl_add(lctl + L::CtlRel + q % kRing, 1u);
                    }
#pragma unroll
                    for (int gg = 0; gg < 8; ++gg) {
                      const int g = 32 * h + 8 * b8 + gg;
                      const half8_t* ap = (const half8_t*)(xh + (((g * 4 + aw) * 2) * M + arow) * 8);
                      const half8_t ahi = ap[0], alo = ap[M];
                      const f4_t sx = *(const f4_t*)(xsum + g * 16 + 4 * aw);
                      const half8_t bq = codes_b(cw[gg]);
                      f4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bq, d, 0, 0, 0);
                      const bool live = g < s.ngs;
                      const float s8 = live ? h2f_lo(smw[gg]) * kMfDeq : 0.0f, mn = live ? h2f_hi(smw[gg]) : 0.0f;
#pragma unroll
                      for (int e = 0; e < 4; ++e) am[e] = __builtin_fmaf(s8, d[e], __builtin_fmaf(mn, sx[e], am[e]));
                    }
                  }
                  continue;
                }
                if (q8) {   // lane = (row lane / 4, quarter lane % 4) of each of the slot's 8 groups
                  const int rr = lane >> 2, qq = lane & 3;
                  u32x4 qv[8];
                  float sc[8];
#pragma unroll
                  for (int gl = 0; gl < 8; ++gl) {
                    qv[gl] = *(const u32x4l*)(slot + gl * 1024 + rr * 64 + qq * 16);
                    sc[gl] = h2f_u16(slot + 8192 + gl * 32 + rr * 2);
                  }
                  __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's reads of the slot are done
                  if (lane == 0) ctl_add(lctl + L::CtlRel + q % kRing, 1u);
#pragma unroll
                  for (int gl = 0; gl < 8; ++gl) {
                    const int g = 8 * h + gl;
                    float cf[16];
                    codes16_q8(qv[gl], cf);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                      float d = dot16f_q8(cf, xs + m * xgps * 32 + g * 64 + qq * 16);
                      d += __shfl_xor(d, 1, 64);
                      d += __shfl_xor(d, 2, 64);
                      if (g < s.ngs)
                        acc[m] = __builtin_fmaf(sc[gl], d - 128.0f * (xsum[m * xgps + 2 * g] + xsum[m * xgps + 2 * g + 1]),
                                                acc[m]);
                    }
                  }
                  continue;
                }
                u32x4 qv[8];
                uint32_t sm[8];
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                  qv[kk] = *(const u32x4l*)(slot + (kk * 64 + lane) * 16);
                  sm[kk] = *(const uint32_t*)(slot + 8192 + (kk * 64 + lane) * 4);
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's reads of the slot are done
                if (lane == 0) ctl_add(lctl + L::CtlRel + q % kRing, 1u);
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                  const int g = 32 * h + 4 * kk + (lane >> 4);
                  if (g < s.ngs) {
                    const float s24 = h2f_lo(sm[kk]) * 16777216.0f, mn = h2f_hi(sm[kk]);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                      const float d = dot32(qv[kk], xs + m * xgps * 32 + g * 32);
                      acc[m] = __builtin_fmaf(s24, d, __builtin_fmaf(mn, xsum[m * xgps + g], acc[m]));
                    }
                  }
                }
              }
              if (q8) {
                if ((lane & 3) == 0)
#pragma unroll
                  for (int m = 0; m < M; ++m) wred[(m * 2 + pt) * 64 + r * 16 + (lane >> 2)] = acc[m];
                continue;
              }
              if (M >= 2 && mf) {   // D[m][n] -> wred: x row m in lanes l / 16 == m / 4, weight row n = l % 16
#pragma unroll
                for (int m = 0; m < M; ++m)
                  if ((lane >> 4) == (m >> 2)) wred[(m * 2 + pt) * 64 + r * 16 + (lane & 15)] = am[m & 3];
                continue;
              }
#pragma unroll
              for (int m = 0; m < M; ++m) {
                float v = acc[m];
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                if (lane < 16) wred[(m * 2 + pt) * 64 + r * 16 + lane] = v;
              }
            }
          }
          __builtin_amdgcn_s_waitcnt(0xC07F);
          __builtin_amdgcn_wave_barrier();
          const int rows = s.nrb * kStageRows;   // 16, or 64 for a softcap unit (the whole wave)
          const int n = share_row(p, s, G, j, 0, 0) + lane;
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const float v0 = wred[m * 128 + min(lane, rows - 1)];
            const float v1 = s.parts == 2 ? wred[m * 128 + 64 + min(lane, rows - 1)] : 0.0f;
            if (lane < rows || e.epi == P0_EPI_SOFTCAP) {
              const float yv = (e.coh & 2) ? epilogue<true>(e, s.split, m, n >> 6, n & 63, v0, v1)
                                           : epilogue<false>(e, s.split, m, n >> 6, n & 63, v0, v1);
              if (M == 1 && e.mbxOut && lane < rows) post_mbx(e, s.split, n, yv);
            }
          }
          __builtin_amdgcn_s_waitcnt(0xC07F);
          __builtin_amdgcn_wave_barrier();   // wred is rewritten by this wave's next unit
        }
      }
      // every compute wave's output stores are acknowledged before the flag: no L2 writeback
      __builtin_amdgcn_s_waitcnt(0);
      cbar();
    }
    if (c == 0 && lane < kFlagCopies) st_coh(flags + ((size_t)lane * n_ops + i) * Gp + b, tag);
    q0 += s.nslot;
  }
  if (abandon) {
    if (lane == 0) ctl_add(lctl + L::CtlBar, kBarRelease);   // no other compute wave waits for this one any more
    return;
  }
  // every workgroup has read this run's tag once all have published op 0: store it back for the next run
  if (b == 0 && wait_flags(flags + 0, nullptr) && tc == 0) st_coh(st, tag);
}

chain_kernel_t pipe_chain_kernel(int M, bool q8) {
  switch (M) {
    case 1: return q8 ? q4_chain_pipe_kernel<1, true> : q4_chain_pipe_kernel<1, false>;
    case 2: return q8 ? q4_chain_pipe_kernel<2, true> : q4_chain_pipe_kernel<2, false>;
    case 3: return q8 ? q4_chain_pipe_kernel<3, true> : q4_chain_pipe_kernel<3, false>;
    case 4: return q8 ? q4_chain_pipe_kernel<4, true> : q4_chain_pipe_kernel<4, false>;
    case 5: return q8 ? q4_chain_pipe_kernel<5, true> : q4_chain_pipe_kernel<5, false>;
  }
  return nullptr;
}

}  // namespace p0
