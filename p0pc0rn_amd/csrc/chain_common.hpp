// chain_common.hpp - what the two pipelined chain kernels share (chain_pipe.hip: M <= 5 x rows; chain_wide.hip:
// 6 - 16): the workgroup's wave roles, the LDS control words, a workgroup's share of an op and its slot order, the
// epilogue parameters, and the loader waves that stream the weights into the LDS ring.
#pragma once
#include "chain_aux.hpp"

namespace p0 {

constexpr int kPL = 4;                       // loader waves
constexpr int kPC = 8;                       // compute waves
constexpr int kPW = kPL + kPC;
constexpr int kSlotB = kStageRows * 32 * 20; // 10240: one slot
// chain state words (in the first 128-byte line, after the tag) that the host sets from p0_chain_tune knob 5
constexpr int kCfgLoaders = 4, kCfgDepth = 5, kCfgPredict = 6;

// LDS words seen by the loader waves through inline assembly: the compiler tracks LDS-DMA loads as pending writes to
// LDS and would otherwise wait for all of them (vmcnt(0)) before any LDS access in the loader code, which would
// drain the loads in flight at every ring check.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ unsigned asm_lds_ld(unsigned a) {
  unsigned v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return v;
}
__device__ __forceinline__ void asm_lds_st(unsigned a, unsigned v) {
  asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : : "v"(a), "v"(v) : "memory");
}

// The compute waves' control words, through an LDS-typed pointer: a volatile access through a generic pointer
// compiles to a flat load, which also waits for every outstanding global access of the wave (vmcnt(0)).
__device__ __forceinline__ unsigned ctl_ld(lds_u32* a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void ctl_st(lds_u32* a, unsigned v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void ctl_add(lds_u32* a, unsigned v) {
  __hip_atomic_fetch_add(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// a workgroup's share of one op
struct Share {
  int nu, first, nrb, parts, nh, ngs, split, gA, nslot, spread;
};
template <bool Q8>
__device__ __forceinline__ Share share_of(const GemvP& p, int b, int G) {
  Share s;
  const int pos = stage_pos(b, G);
  s.first = pos >= p.scur ? pos - p.scur : pos - p.scur + G;
  s.nu = s.first < p.su ? (p.su - s.first + G - 1) / G : 0;
  s.nrb = p.snrb;
  s.parts = p.epi == P0_EPI_GEGLU ? 2 : 1;
  s.split = s.first % p.nsplit;   // every unit of a share has this split (the host checks)
  // groups of the split (32 k for q4g32a.t64, 64 k for q8g64s.t64) and slots per 16-row part (32 or 8 groups each)
  const int gsh = Q8 && p.enc == P0_ENC_Q8G64S_T64 ? 6 : 5;
  s.gA = s.split * (p.kPer >> gsh);
  s.ngs = (min(p.K, (s.split + 1) * p.kPer) >> gsh) - s.gA;
  s.nh = gsh == 6 ? (s.ngs + 7) >> 3 : (s.ngs + 31) >> 5;
  s.nslot = s.nu * s.nrb * s.parts * s.nh;
  s.spread = p.sngp;   // the host's choice: 1 = all compute waves on every slot (the share fits the ring), 0 = a wave per unit
  return s;
}
// Slot order of a share. Small shares: unit-major, then block, part, half. Large shares: units in rounds of kPC (unit
// j = kPC R + c goes to compute wave c), and inside a round the waves' slots interleave (slot s of every unit, then
// slot s + 1, ...), so the ring's consecutive slots feed all waves at once.
__device__ __forceinline__ void slot_of(const Share& s, int k, int& j, int& si) {
  const int S = s.nrb * s.parts * s.nh;
  if (s.spread) {
    j = k / S;
    si = k - j * S;
    return;
  }
  const int R = min(k / (kPC * S), (s.nu - 1) / kPC);
  const int nw = min(kPC, s.nu - kPC * R), kr = k - R * kPC * S;
  si = kr / nw;
  j = kPC * R + (kr - si * nw);
}
__device__ __forceinline__ int slot_index(const Share& s, int j, int si) {   // inverse of slot_of
  const int S = s.nrb * s.parts * s.nh;
  if (s.spread) return j * S + si;
  const int R = j / kPC, nw = min(kPC, s.nu - kPC * R);
  return R * kPC * S + si * nw + (j - kPC * R);
}
// The parameters the epilogue and the mailbox post read, loaded at the op's start (while the workgroup waits for the
// op's input) and pinned in registers. Read where they are used, each would be a scalar load that waits for the
// scalar cache, and the epilogue's branches put several such waits in a row on the op's critical path.
struct EpiP {
  float* Y;
  float* MX;
  unsigned long long* mbxOut;
  int64_t ldy, ldm;
  float cap;
  int epi, NT, coh;
};
__device__ __forceinline__ EpiP epi_of(const GemvP& p) {
  EpiP e{p.Y, p.MX, p.mbxOut, p.ldy, p.ldm, p.cap, p.epi, p.NT, p.coh};
  asm volatile("" : "+s"(e.Y), "+s"(e.MX), "+s"(e.mbxOut), "+s"(e.ldy), "+s"(e.ldm), "+s"(e.cap), "+s"(e.epi),
               "+s"(e.NT), "+s"(e.coh));
  return e;
}

// first weight row of part (unit j, block r, part pt) of a share
__device__ __forceinline__ int share_row(const GemvP& p, const Share& s, int G, int j, int r, int pt) {
  return ((s.first + j * G) / p.nsplit * s.nrb + r) * kStageRows + (pt ? p.N : 0);
}

// The loader waves of a chain workgroup (waves wv < kPL): every op's weight share streamed into the ring of kRing
// slots at the start of the workgroup's LDS, with LDS-DMA loads, in the share's slot order (slot_of), ops ahead of the
// compute waves as far as the ring has room. A slot is published (ctl[ctl_full + pos] = q + 1) once the loader's own
// vmcnt says it has landed; its position is reused once the compute waves have released it RelPer times (the waves
// that read it). The loaders never touch activations or flags; they leave when ctl[ctl_stop] is set (a compute wave
// gave up), with no load in flight.
template <int kRing, bool Q8, int RelPer>
__device__ __forceinline__ void chain_loader(const GemvP* __restrict__ ops, int n_ops, const unsigned* __restrict__ st,
                                             uint8_t* lds, unsigned* ctl, int ctl_full, int ctl_rel, int ctl_stop,
                                             int b, int G, int wv, int lane) {
  // st[kCfgLoaders]: loader waves that stream a small share (1 .. kPL; a large share takes all kPL),
  // st[kCfgDepth]: slots in flight per loader (1 or 2)
  const int nls = min(kPL, max(1, (int)st[kCfgLoaders])), depth2 = st[kCfgDepth] >= 2;
  const unsigned a_full = lds_addr(ctl + ctl_full), a_rel = lds_addr(ctl + ctl_rel), a_stop = lds_addr(ctl + ctl_stop);
  int q0 = 0, pend = -1;
  auto publish = [&](int q) { asm_lds_st(a_full + (q % kRing) * 4, (unsigned)q + 1); };
  for (int i = 0; i < n_ops; ++i) {
    const GemvP& p = op_at(ops, i);
    // Touch every 64-byte line of the op's parameters: the op table would otherwise be fetched from memory (the
    // weight stream evicts it from L2 every run) by the compute waves' scalar loads, one miss after another, on the
    // chain's critical path; the loaders run ops ahead, so the lines are in the CU's scalar cache by then.
    {
      const uint32_t* pw = (const uint32_t*)&p;
      uint32_t t = 0;
#pragma unroll
      for (int k = 0; k < (int)(sizeof(GemvP) / 4); k += 16) t ^= pw[k];
      asm volatile("" : : "s"(t));
    }
    const Share s = share_of<Q8>(p, b, G);
    const int nl = s.spread && s.nslot <= kRing ? nls : kPL;   // a share larger than the ring takes every loader
    const int k0 = wv < nl ? ((wv - q0) % nl + nl) % nl : s.nslot;
    for (int k = k0; k < s.nslot; k += nl) {
      const int q = q0 + k, pos = q % kRing;
      if ((int)asm_lds_ld(a_rel + pos * 4) < RelPer * (q / kRing)) {   // the position still holds slot q - kRing
        if (pend >= 0) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          publish(pend);
          pend = -1;
        }
        while ((int)asm_lds_ld(a_rel + pos * 4) < RelPer * (q / kRing)) {
          if (asm_lds_ld(a_stop)) {   // the compute waves gave up: leave, with no load in flight
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            return;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      // slot k of the share: unit j, its slot si = (block r, part pt, half h of 32 groups)
      int j, si;
      slot_of(s, k, j, si);
      const int h = si % s.nh, rest = si / s.nh, pt = rest % s.parts, r = rest / s.parts;
      const int n = share_row(p, s, G, j, r, pt);
      const int r0 = n & 63, glast = s.ngs - 1;
      uint8_t* const slot = lds + pos * kSlotB;
      if (Q8 && p.enc == P0_ENC_Q8G64S_T64) {
        // q8g64s.t64 slot: 16 rows x 8 groups of 64 k. Codes [8 groups][16 rows][64 B] (a group's 16 rows are 1 KB
        // of one record), then scales [8 groups][16 rows][2 B]; the scale load is issued twice so that every slot
        // takes 10 loads, as the vmcnt arithmetic below assumes
        const uint8_t* tb = p.w + ((int64_t)(n >> 6) * p.wG + s.gA) * 4224;
#pragma unroll
        for (int ci = 0; ci < 8; ++ci) {
          const int g = min(8 * h + ci, glast);
          __builtin_amdgcn_global_load_lds((const void*)(tb + (int64_t)g * 4224 + r0 * 64 + lane * 16),
                                           (__attribute__((address_space(3))) void*)(slot + ci * 1024), 16, 0, 0);
        }
        const int g = min(8 * h + ((lane >> 1) & 7), glast);   // lane: group (lane / 2) % 8, half lane % 2
        const uint8_t* src = tb + (int64_t)g * 4224 + 4096 + r0 * 2 + (lane & 1) * 16;
#pragma unroll
        for (int rep = 0; rep < 2; ++rep)
          __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(slot + 8192),
                                           16, 0, 0);
      } else {
      const uint8_t* tb = p.w + ((int64_t)(n >> 6) * p.wG + s.gA) * 1280;
#pragma unroll
      for (int ci = 0; ci < 8; ++ci) {   // codes: 4 groups per load (lane: group 4 ci + lane / 16, row lane % 16)
        const int g = min(32 * h + 4 * ci + (lane >> 4), glast);
        const uint8_t* src = tb + (int64_t)g * 1280 + (r0 + (lane & 15)) * 16;
        __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)(slot + ci * 1024),
                                         16, 0, 0);
      }
#pragma unroll
      for (int si = 0; si < 2; ++si) {   // scale words: 16 groups per load (lane: group 16 si + lane / 4, 4 rows)
        const int g = min(32 * h + 16 * si + (lane >> 2), glast);
        const uint8_t* src = tb + (int64_t)g * 1280 + 1024 + (r0 + 4 * (lane & 3)) * 4;
        __builtin_amdgcn_global_load_lds((const void*)src,
                                         (__attribute__((address_space(3))) void*)(slot + 8192 + si * 1024), 16, 0, 0);
      }
      }
      if (!depth2) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        publish(q);
        continue;
      }
      if (pend >= 0) {   // the previous slot's 10 loads are older than this slot's 10
        asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
        publish(pend);
      }
      pend = q;
    }
    q0 += s.nslot;
  }
  if (pend >= 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    publish(pend);
  }
}

}  // namespace p0
