// chain_wide.hip - the pipelined GEMV chain for 6 - 16 x rows in ONE persistent launch: a speculative-decode verify pass
// of M tokens (gemvM over every linear of the step, engine/llm/lops_spec.js:6-8: "each weight record read ONCE" for
// all M rows; the verify costs the reference plans with, engine/llm/spec.js:41-44). The planning is in gemv.hip
// (plan_wide); the wave roles, the loader waves and the slot format are chain_pipe.hip's (chain_common.hpp).
//
// What changes with the row count. Per group of 32 k and 16 weight rows the matrix cores take all M <= 16 x rows in
// one pair of v_mfma_f32_16x16x32_f16 (x' as fp16 hi and lo A operands, the codes as the B operand), so the slot
// arithmetic costs the same at M = 16 as at M = 1. What grows with M is x': its A operands are M x 4 bytes per k, 128
// KB for a 2048-k split at M = 16, which leaves an LDS of 160 KB no room for the weight ring. So here x' never goes to
// LDS. Each compute wave computes with the same 8 groups of every slot of an op (groups 4 c .. 4 c + 3 of each 32-group
// half of the split, c = the compute wave), and holds those groups' A operands and group sums in registers for the
// whole op (96 VGPRs at any M <= 16): a lane (k chunk aw = lane / 16, row lane % 16) keeps the 8 k of its chunk of
// each group. The LDS holds the ring and a double-buffered reduction area; every share is computed by all compute
// waves in rounds of up to 4 16-row parts (one softcap tile, two geglu units, four store units), a round's row sums
// summed over the waves in LDS and its epilogue run while the next round's slots arrive, and each wave hands a slot
// back as soon as it has read its 4 groups' code and scale words.
//
// Where the A operands come from:
//  * the previous op's epilogue staged them (GemvP::stgIn, 2^8 x' split into hi and lo, and the 16-k sums, as in the
//    pipelined kernel): each wave loads its 8 groups straight into registers, 2 x 16 bytes a lane per group;
//  * when the staging marked a half of the wave's groups too large for the fixed 2^8 scale (NaN), the wave takes the
//    fp32 x' values the producer also wrote and splits them with a scale of its own: 2^e with e chosen from the largest
//    |x'| of the wave (that value x 2^e in [2^14, 2^15)), so the hi / lo pair keeps 22 bits of every value near the
//    wave's largest and nothing overflows. The wave's D results are scaled back by 2^-e with the weight scale, one
//    multiply it has anyway;
//  * an op whose x is not the previous op's output (the chain's first op) stages its x' from x (raw or rms prologue)
//    with such a scale.
//    There is no VALU fallback: any finite x' runs on the matrix cores.
#include "chain_common.hpp"

namespace p0 {

constexpr int kWideParts = 4;    // 16-row parts per round
constexpr int kWideMaxM = 16;

template <int MW>   // the largest x row count of the instantiation (8 or 16)
struct WideL {
  static constexpr int RedB = kWideParts * MW * kPC * 16 * 4;       // one reduction buffer: [part][m][wave][16 rows]
  static constexpr int Ring0 = (160 * 1024 - 512 - 2 * RedB) / kSlotB;
  static constexpr int Ring = Ring0 > 12 ? 12 : Ring0;               // slots in the ring
  static constexpr int OffRed = Ring * kSlotB;
  static constexpr int OffCtl = OffRed + 2 * RedB;
  static constexpr int CtlFull = 0, CtlRel = Ring, CtlBar = 2 * Ring, CtlStop = 2 * Ring + 1, CtlGo = 2 * Ring + 2,
                       CtlTag = 2 * Ring + 3, CtlWords = 2 * Ring + 4;
  static constexpr int Lds = OffCtl + CtlWords * 4;
  static_assert(Lds <= 160 * 1024 - 256, "wide chain LDS");
  static_assert(RedB / 4 >= kAuxLdsFloats, "the aux ops' trees use the reduction area");
};

__host__ int wide_lds_bytes(int M) { return M <= 8 ? WideL<8>::Lds : WideL<16>::Lds; }
__host__ int wide_ring_slots(int M) { return M <= 8 ? WideL<8>::Ring : WideL<16>::Ring; }
__host__ int wide_max_m() { return kWideMaxM; }

// the 8 groups of compute wave c: group gi = 4 h + jg of the wave is 32 h + 4 c + jg of the split
__device__ __forceinline__ int wide_group(int c, int gi) { return 32 * (gi >> 2) + 4 * c + (gi & 3); }

// A operands of the wave from the previous op's staging (stg_half_at's layout, 2^8 x', device-coherent 16-byte
// loads: written by other CUs in this run) and the group sums of x row 4 (lane / 16) + i in sx[gi][i] (the two 16-k
// halves added, as stage_stg adds them). Rows >= M read row M - 1 (their D rows are never stored). False in every
// lane if a sum of the wave's groups is NaN: a half the producer marked too large for the 2^8 scale.
__device__ __forceinline__ bool wide_load_staged(const GemvP& p, const Share& s, int M, int c, int lane,
                                                 half8_t (&ahi)[8], half8_t (&alo)[8], f4_t (&sx)[8]) {
  const int aw = lane >> 4, arow = min(lane & 15, M - 1);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)p.stgIn, (short)0, 0x7FFFFFFF, 0x00020000);
  const float* ps = (const float*)(p.stgIn + (int64_t)p.K * M);
  float hs[8][2];
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    const int g = wide_group(c, gi), gg = s.gA + min(g, s.ngs - 1);
    const int at = (((gg * 4 + aw) * 2) * M + arow) * 8;   // halves
    const auto hi = __builtin_amdgcn_raw_buffer_load_b128(sr, at * 2, 0, 16);
    const auto lo = __builtin_amdgcn_raw_buffer_load_b128(sr, (at + M * 8) * 2, 0, 16);
    ahi[gi] = __builtin_bit_cast(half8_t, hi);
    alo[gi] = __builtin_bit_cast(half8_t, lo);
    hs[gi][0] = ldf<true>(&ps[(gg * 2) * M + arow]);
    hs[gi][1] = ldf<true>(&ps[(gg * 2 + 1) * M + arow]);
  }
  bool ok = true;
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    const bool live = wide_group(c, gi) < s.ngs;
    const float gsum = live ? hs[gi][0] + hs[gi][1] : 0.0f;   // the lane's row arow
    ok = ok && gsum == gsum;
    if (!live) ahi[gi] = alo[gi] = half8_t{};
#pragma unroll
    for (int i = 0; i < 4; ++i) sx[gi][i] = __shfl(gsum, 4 * aw + i, 64);
  }
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// The wave's A operands from its 8 groups' x' values v[gi][j] (k 8 (lane / 16) + j of group gi, row lane % 16 or
// M - 1; zero for groups past the split), with the wave's own scale 2^e: the largest |x'| of the wave x 2^e in
// [2^14, 2^15); *deq = 2^-e. Odd k are pre-scaled 1/16, as the B operand's odd codes are 16 q. sx as wide_load_staged.
// fit8: where every |x'| of the wave is below kMfBig, the fixed 2^8 instead, so that the operands, group sums and deq
// equal wide_load_staged's bit for bit (the producer's hi / lo split of 2^8 x', and its sums in the same tree).
// Returns true if the wave's x' exceeds that range or holds a NaN (a half the producer marked, either way).
// Lane exchanges: the two chunk-pair adds through the gfx950 row and half swaps (lane ^ 16, lane ^ 32: VALU moves, no
// LDS round trip; each add takes the same two values as before, in either order), the wave's largest |x'| through
// DPP and the same swaps (a maximum does not depend on the order).
__device__ __forceinline__ bool wide_scale_x(float (&v)[8][8], int lane, half8_t (&ahi)[8], half8_t (&alo)[8],
                                             f4_t (&sx)[8], float& deq, bool fit8) {
  const int aw = lane >> 4;
  auto swap_add = [](float x, bool half) {
    const auto r = half ? __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                        : __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  };
  float mx = 0.0f;
  bool nan = false;
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    const float s8 = ((v[gi][0] + v[gi][1]) + (v[gi][2] + v[gi][3])) + ((v[gi][4] + v[gi][5]) + (v[gi][6] + v[gi][7]));
    const float gsum = swap_add(swap_add(s8, false), true);
    nan = nan || gsum != gsum;
#pragma unroll
    for (int i = 0; i < 4; ++i) sx[gi][i] = __shfl(gsum, 4 * aw + i, 64);
#pragma unroll
    for (int j = 1; j < 8; j += 2) v[gi][j] *= 0.0625f;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, __builtin_fabsf(v[gi][j]));
  }
  mx = fmaxf(mx, dpp_f<0xB1>(mx));    // lane ^ 1
  mx = fmaxf(mx, dpp_f<0x4E>(mx));    // lane ^ 2
  mx = fmaxf(mx, dpp_f<0x141>(mx));   // the other quad of the 8 lanes
  mx = fmaxf(mx, dpp_f<0x140>(mx));   // the other 8 of the 16
  {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
  }
  int E = 15;
  if (mx > 0.0f && mx <= 3.4e38f) (void)__builtin_frexpf(mx, &E);   // mx in [2^(E-1), 2^E)
  const bool big = !(mx < kMfBig) || __builtin_amdgcn_ballot_w64(nan) != 0;
  const int e = fit8 && !big ? 8 : min(60, max(-60, 15 - E));
  const float scale = __builtin_ldexpf(1.0f, e);
  deq = __builtin_ldexpf(1.0f, -e);
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float xs = v[gi][j] * scale;
      hi[j] = (_Float16)xs;
      lo[j] = (_Float16)(xs - (float)hi[j]);
    }
    // positions 0 .. 7 hold k 0, 4, 1, 5, 2, 6, 3, 7 of the chunk (codes_b's order)
    ahi[gi] = half8_t{hi[0], hi[4], hi[1], hi[5], hi[2], hi[6], hi[3], hi[7]};
    alo[gi] = half8_t{lo[0], lo[4], lo[1], lo[5], lo[2], lo[6], lo[3], lo[7]};
  }
  return big;
}

// the wave's x' from x (raw or rms prologue, the prologue's own order x * rstd * nw), every group's loads issued
// before the first is used, then wide_scale_x
template <bool COH>
__device__ __forceinline__ void wide_stage_x(const GemvP& p, const Share& s, int M, int c, int lane, half8_t (&ahi)[8],
                                             half8_t (&alo)[8], f4_t (&sx)[8], float& deq) {
  const int aw = lane >> 4, arow = min(lane & 15, M - 1);
  const bool rms = p.pro == P0_PRO_RMS;
  const bool vec = ((uintptr_t)(p.X + p.rowB) & 15) == 0 && (p.ldx & 3) == 0 &&
                   (!rms || ((uintptr_t)(p.NW + p.nOff) & 15) == 0);
  const float st = rms ? ldf<COH>(&p.ST[p.statOff + arow * p.statLd]) : 1.0f;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)(p.X + p.rowB), (short)0, 0x7FFFFFFF,
                                                                      0x00020000);
  float v[8][8];
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    const int k0 = (s.gA + min(wide_group(c, gi), s.ngs - 1)) * 32 + 8 * aw;   // in bounds also past the split
    if (vec) {
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(xr, (arow * (int)p.ldx + k0) * 4, 0, COH ? 16 : 0);
      const auto b = __builtin_amdgcn_raw_buffer_load_b128(xr, (arow * (int)p.ldx + k0 + 4) * 4, 0, COH ? 16 : 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[gi][j] = __uint_as_float(a[j]);
        v[gi][4 + j] = __uint_as_float(b[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[gi][j] = ldf<COH>(&p.X[arow * p.ldx + p.rowB + k0 + j]);
    }
  }
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    const bool live = wide_group(c, gi) < s.ngs;
    const int k0 = (s.gA + min(wide_group(c, gi), s.ngs - 1)) * 32 + 8 * aw;
    float nw[8];
    if (rms) {
      if (vec) {
        const float4 na = *(const float4*)&p.NW[p.nOff + k0], nb = *(const float4*)&p.NW[p.nOff + k0 + 4];
        nw[0] = na.x; nw[1] = na.y; nw[2] = na.z; nw[3] = na.w;
        nw[4] = nb.x; nw[5] = nb.y; nw[6] = nb.z; nw[7] = nb.w;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) nw[j] = ldf<COH>(&p.NW[p.nOff + k0 + j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[gi][j] = live ? (rms ? v[gi][j] * st * nw[j] : v[gi][j]) : 0.0f;
  }
  (void)wide_scale_x(v, lane, ahi, alo, sx, deq, false);
}

// the wave's x' from the previous op's fp32 staging (stg_f32_at: the prologue's values as the producer computed them,
// device-coherent loads, all in flight together), then wide_scale_x with fit8: for a wave whose staged halves
// overflowed the fixed 2^8 scale, or whose x' overflowed it in the op before (returns wide_scale_x's value)
__device__ __forceinline__ bool wide_stage_f32(const GemvP& p, const Share& s, int M, int c, int lane, half8_t (&ahi)[8],
                                               half8_t (&alo)[8], f4_t (&sx)[8], float& deq) {
  const int aw = lane >> 4, arow = min(lane & 15, M - 1);
  const __amdgpu_buffer_rsrc_t fr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.stgIn + stg_f32_at(M, p.K)), (short)0, 0x7FFFFFFF, 0x00020000);
  float v[8][8];
#pragma unroll
  for (int gi = 0; gi < 8; ++gi) {
    const int k0 = (s.gA + min(wide_group(c, gi), s.ngs - 1)) * 32 + 8 * aw;
    const auto a = __builtin_amdgcn_raw_buffer_load_b128(fr, (arow * p.K + k0) * 4, 0, 16);
    const auto b = __builtin_amdgcn_raw_buffer_load_b128(fr, (arow * p.K + k0 + 4) * 4, 0, 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[gi][j] = __uint_as_float(a[j]);
      v[gi][4 + j] = __uint_as_float(b[j]);
    }
  }
#pragma unroll
  for (int gi = 0; gi < 8; ++gi)
    if (wide_group(c, gi) >= s.ngs)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[gi][j] = 0.0f;
  return wide_scale_x(v, lane, ahi, alo, sx, deq, true);
}

template <int MW>
__global__ __launch_bounds__(64 * kPW) void q4_chain_wide_kernel(const GemvP* __restrict__ ops, int n_ops,
                                                                 unsigned* __restrict__ st, int spin_limit) {
  using L = WideL<MW>;
  constexpr int kRing = L::Ring;
  constexpr int kRedF = L::RedB / 4;
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
  if (wv < kPL) {   // loader waves: every compute wave reads every slot, so a slot is released kPC times
    chain_loader<kRing, false, kPC>(ops, n_ops, st, lds, ctl, L::CtlFull, L::CtlRel, L::CtlStop, b, G, wv, lane);
    return;
  }

  // ---- compute waves (at a higher wave priority than the loaders, as in the pipelined kernel)
  const int c = wv - kPL, tc = tid - 64 * kPL;
  __builtin_amdgcn_s_setprio(1);
  lds_u32* const lctl = (lds_u32*)ctl;
  float* const red0 = (float*)(lds + L::OffRed);
  unsigned gen = 0;
  auto cbar = [&]() { aux_bar(lctl + L::CtlBar, gen, lane); };
  auto give_up = [&]() {   // lane 0 of a wave whose wait gave up: mark the run, stop the loaders and the other waves
    atomicOr(timed_out, 1u);
    ctl_st(lctl + L::CtlStop, 1u);
    ctl_st(lctl + L::CtlGo, 0u);
  };
  auto wait_slot = [&](int q) -> bool {
    for (int spins = 0; ctl_ld(lctl + L::CtlFull + q % kRing) != (unsigned)q + 1; ++spins) {
      if (ctl_ld(lctl + L::CtlStop)) return false;
      if (spins >= spin_limit) {
        if (lane == 0) give_up();
        return false;
      }
      __builtin_amdgcn_s_sleep(0);
    }
    return true;
  };
  // the G flags at f hold this run's tag (wave c == 0 polls); false in every compute thread if the wait gave up
  auto wait_flags = [&](const unsigned* f) -> bool {
    if (c == 0) {
      int go = spin_limit >= 0;
      for (int spins = 0; go && !flags_set(f, G, tag, lane); ++spins) {
        if (spins >= spin_limit || (spins % 64 == 63 && ld_coh(timed_out))) go = 0;
        else __builtin_amdgcn_s_sleep(1);
      }
      if (!go && lane == 0) give_up();
    }
    cbar();
    return ctl_ld(lctl + L::CtlGo) != 0;
  };
  const unsigned* const mine = flags + (size_t)(b % kFlagCopies) * n_ops * Gp;   // this XCD's copy
  const int aw = lane >> 4, n16 = lane & 15;
  int q0 = 0, buf = 0;
  bool abandon = false;
  // this wave's x' exceeded the staging's 2^8 range in its last staged op: it takes the fp32 x' straight away (one
  // round trip instead of two when the next op's x' exceeds it too; the operands are the same either way).
  // st[kCfgPredict] = 0 (p0_chain_tune knob 14): every wave tries the staged halves first.
  const bool predict = st[kCfgPredict] != 0u;
  bool big = false;
  for (int i = 0; i < n_ops; ++i) {
    const GemvP& p = op_at(ops, i);
    if (p.kind != kOpGemv) {   // copy / argmax / rowstats / normadd, as in the pipelined kernel
      if (aux_worker(p, b)) {
        if (p.abefore >= 0 && !wait_flags(mine + (size_t)p.abefore * Gp)) {
          abandon = true;
          break;
        }
        gen = aux_run(&p, b, G, tc, (lds_f32*)red0, lctl + L::CtlBar, gen);
        __builtin_amdgcn_s_waitcnt(0);
        cbar();
      }
      if (c == 0 && lane < kFlagCopies) st_coh(flags + ((size_t)lane * n_ops + i) * Gp + b, tag);
      continue;
    }
    const Share s = share_of<false>(p, b, G);
    if (s.nu > 0) {
      const EpiP e = epi_of(p);
      const int M = p.mrows;
      // op i - 1 complete in every workgroup (its outputs are this op's x; every earlier op is then complete too)
      if (i > 0 && !wait_flags(mine + (size_t)(i - 1) * Gp)) {
        abandon = true;
        break;
      }
      half8_t ahi[8], alo[8];
      f4_t sx[8];
      float deq = kMfDeq;
      if (p.stgIn) {
        if (big || !wide_load_staged(p, s, M, c, lane, ahi, alo, sx))
          big = wide_stage_f32(p, s, M, c, lane, ahi, alo, sx, deq) && predict;
      } else if (p.coh & 1) {
        wide_stage_x<true>(p, s, M, c, lane, ahi, alo, sx, deq);
      } else {
        wide_stage_x<false>(p, s, M, c, lane, ahi, alo, sx, deq);
      }
      const bool stg_rms = p.stgOut && p.stgPro == P0_PRO_RMS;
      const int upr = max(1, kWideParts / (s.nrb * s.parts));   // units per round
      const int S = s.nrb * s.parts * s.nh;                     // slots per unit
      for (int j0 = 0; j0 < s.nu; j0 += upr) {
        const int nur = min(upr, s.nu - j0), npr = nur * s.nrb * s.parts;
        f4_t am[kWideParts];
#pragma unroll
        for (int rp = 0; rp < kWideParts; ++rp) am[rp] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        const int qr0 = q0 + j0 * S;   // the round's slots are consecutive: part rp, half h at qr0 + rp nh + h
#pragma unroll
        for (int rp = 0; rp < kWideParts; ++rp) {
          if (rp >= npr) break;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if (h >= s.nh) break;
            const int q = qr0 + rp * s.nh + h;
            wait_slot(q);
            const uint8_t* slot = lds + (q % kRing) * kSlotB;
            uint32_t cw[4], sm[4];
#pragma unroll
            for (int jg = 0; jg < 4; ++jg) {
              const int gs = 4 * c + jg;
              cw[jg] = *(const uint32_t*)(slot + (gs * 16 + n16) * 16 + aw * 4);
              sm[jg] = *(const uint32_t*)(slot + 8192 + (gs * 16 + n16) * 4);
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's reads of the slot are done
            if (lane == 0) ctl_add(lctl + L::CtlRel + q % kRing, 1u);
#pragma unroll
            for (int jg = 0; jg < 4; ++jg) {
              const int gi = 4 * h + jg;
              const half8_t bq = codes_b(cw[jg]);
              f4_t d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[gi], bq, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
              d = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[gi], bq, d, 0, 0, 0);
              const bool live = wide_group(c, gi) < s.ngs;
              const float s8 = live ? h2f_lo(sm[jg]) * deq : 0.0f, mn = live ? h2f_hi(sm[jg]) : 0.0f;
#pragma unroll
              for (int k = 0; k < 4; ++k) am[rp][k] = __builtin_fmaf(s8, d[k], __builtin_fmaf(mn, sx[gi][k], am[rp][k]));
            }
          }
        }
        // D[m][n]: x row m = 4 (lane / 16) + k, weight row n16 of the part
        float* const red = red0 + buf * kRedF;
#pragma unroll
        for (int rp = 0; rp < kWideParts; ++rp) {
          if (rp >= npr) break;
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (4 * aw + k < MW) red[((rp * MW + 4 * aw + k) * kPC + c) * 16 + n16] = am[rp][k];
        }
        cbar();   // every wave's row sums of the round are in
        if (!ctl_ld(lctl + L::CtlGo)) {   // a wait gave up: no stores
          abandon = true;
          break;
        }
        // epilogue of the round: pair et -> x row m = et / rows, row et % rows of the round (rows a multiple of 16, a
        // softcap round a whole 64-row tile per wave)
        const int rows = nur * s.nrb * kStageRows, npairs = rows * M;
        for (int e0 = 0; e0 < npairs; e0 += kAuxThreads) {
          const int et = e0 + tc;
          if (et - lane >= npairs) break;   // whole waves past the end
          const int ec = min(et, npairs - 1), m = ec / rows, row = ec - m * rows;
          const int jr = row / (s.nrb * kStageRows), rr = row - jr * (s.nrb * kStageRows);
          const int rpg = (jr * s.nrb + (rr >> 4)) * s.parts, r16 = rr & 15;
          float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
          for (int w = 0; w < kPC; ++w) v0 += red[((rpg * MW + m) * kPC + w) * 16 + r16];
          if (s.parts == 2) {
#pragma unroll
            for (int w = 0; w < kPC; ++w) v1 += red[(((rpg + 1) * MW + m) * kPC + w) * 16 + r16];
          }
          const int n = share_row(p, s, G, j0 + jr, 0, 0) + rr;
          if (et >= npairs) continue;   // (a softcap wave is whole: npairs is a multiple of 64 there)
          const float yv = (e.coh & 2) ? epilogue<true>(e, s.split, m, n >> 6, n & 63, v0, v1)
                                       : epilogue<false>(e, s.split, m, n >> 6, n & 63, v0, v1);
          if (p.stgOut) {
            // the next op's x' of (x row m, k = n - stgR0), as the pipelined kernel's producer writes it (2^8 x' as
            // fp16 hi + lo, odd k scaled 1/16; the 16-k group sums in the balanced tree over the 16 consecutive lanes of
            // a 16-row block, NaN marking a half some |x'| of which is too large for the 2^8 scale)
            const int64_t k = (int64_t)n - p.stgR0;
            if (s.split == p.stgSp && k >= 0 && k < p.stgK) {
              const float x = stg_rms ? yv * p.stgST[p.stgStatOff + m * p.stgStatLd] * p.stgNW[p.stgNOff + k] : yv;
              const float xo = (k & 1) ? x * 0.0625f : x;
              const float xs8 = xo * kMfScale;
              const _Float16 hi = (_Float16)xs8, lo = (_Float16)(xs8 - (float)hi);
              _Float16* const sh = (_Float16*)p.stgOut;
              *P0_GLOBAL(_Float16, sh + stg_half_at(M, k, m, 0)) = hi;
              *P0_GLOBAL(_Float16, sh + stg_half_at(M, k, m, 1)) = lo;
              *P0_GLOBAL(float, (float*)p.stgOut + stg_f32_at(M, p.stgK) + (int64_t)m * p.stgK + k) = x;
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
        buf ^= 1;
      }
      if (abandon) break;
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
  if (b == 0 && wait_flags(flags + 0) && tc == 0) st_coh(st, tag);
}

chain_kernel_t wide_chain_kernel(int M) { return M <= 8 ? q4_chain_wide_kernel<8> : q4_chain_wide_kernel<16>; }

}  // namespace p0
