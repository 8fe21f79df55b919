// chain_aux.hpp - the ops of a pipelined chain that are not GEMVs, so that a whole decode token (the reference's
// per-token command buffer, engine/llm/drunner.js:1-8) is one launch:
//   * copy      runner.copy between buffers (engine/core/gpu.js:237-242, the token's rstd copy into the head's stat
//               slot, engine/llm/gemma4.js:505, and the result copy of DecodeRunner.end, engine/llm/drunner.js:82-90);
//   * argmax    argmax / argmaxM over a softcap GEMV's (max, index) tile pairs (engine/llm/lops.js:416-436,
//               engine/llm/lops_spec.js:327-348);
//   * rowstats  the (mean, rstd) slots an rms prologue reads (engine/ops/misc.js:13-40);
//   * normadd   the split-K sum with the residual update and its rstd (engine/llm/lops.js:143-178).
// The 512 compute threads of a chain workgroup run them. Row ops take one row per workgroup (rows b, b + G, ...); the
// copy deals 2048-word blocks to workgroups in turn. Every sum follows the standalone kernels' order (misc.hip)
// exactly: threads t < 256 sum elements t, t + 256, ... in turn, then the halving tree over the 256 partials, products
// and sums rounded separately. So an op's results in a chain equal the standalone op's bit for bit. All accesses are
// device-coherent: other ops of the chain, on other XCDs, write the inputs and read the outputs.
#pragma once
#include "gemv_kernels.hpp"

namespace p0 {

constexpr int kAuxThreads = 512;                  // compute threads of a pipelined chain workgroup
constexpr int kAuxWaves = kAuxThreads / 64;
constexpr int kAuxCopyWords = 4 * kAuxThreads;    // copy words a workgroup takes per round
constexpr int kAuxLdsFloats = 2 * 256;            // LDS the aux ops use: two tree areas

// does workgroup b take part in aux op p? (the others only publish their flags)
__device__ __forceinline__ bool aux_worker(const GemvP& p, int b) {
  return p.kind == kOpCopy ? (int64_t)b * kAuxCopyWords < p.an : b < p.arows;
}

__device__ __forceinline__ unsigned aux_ldu(const void* a) {
  return __hip_atomic_load(P0_GLOBAL(unsigned, (unsigned*)const_cast<void*>(a)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void aux_stu(void* a, unsigned v) {
  __hip_atomic_store(P0_GLOBAL(unsigned, (unsigned*)a), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float aux_ldf(const float* a) { return __uint_as_float(aux_ldu(a)); }
__device__ __forceinline__ unsigned long long aux_ld2(const float* a) {   // an 8-byte aligned pair of words
  return __hip_atomic_load(P0_GLOBAL(unsigned long long, (unsigned long long*)const_cast<float*>(a)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kAuxBatch = 8;   // loads a thread issues before it uses the first (one memory round trip per batch)
__device__ __forceinline__ void aux_stf(float* a, float v) { aux_stu(a, __float_as_uint(v)); }

// (value, index) with ties to the lower index (engine/llm/lops.js:424). A thread's running best is never NaN (a NaN
// never compares better than the start value), so "better" is a total order on what is combined and any reduction order
// gives the standalone kernel's result.
__device__ __forceinline__ bool aux_better(float v, uint32_t id, float bv, uint32_t bi) {
  return v > bv || (v == bv && id < bi);
}

typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) unsigned lds_u32;

// the barrier of the chain kernel's compute waves: a monotonic LDS counter at ctr, every compute wave adds 1 per
// barrier (gen: this wave's count of the barriers so far, times kAuxWaves). A wave that leaves the kernel after a
// wait gave up adds kBarRelease first (every wave at most once: 8 x 2^26 < 2^32), which ends every barrier wait of
// the workgroup at once: the go word it left on can turn 0 between two waves' reads of it after one barrier, and a
// wave that read 1 must not wait at its next barrier for one that left (the run is void then and stores nothing
// more once the others see the go word)
constexpr unsigned kBarRelease = 1u << 26;
__device__ __forceinline__ void aux_bar(lds_u32* ctr, unsigned& gen, int lane) {
  gen += kAuxWaves;
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's LDS writes are done
  if (lane == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < gen) __builtin_amdgcn_s_sleep(0);
  __builtin_amdgcn_s_waitcnt(0xC07F);
}

// the reference's halving tree over the 256 partials v of threads t < 256 (level s: red[t] += red[t + s], t < s), its
// result in every thread t < 256. One barrier: each of the 4 waves reads the 256 partials and runs the whole tree
// (levels 128 and 64 on the values it read, 32 .. 1 by lane exchanges, each pairing red[t] with red[t + s]).
__device__ __forceinline__ float aux_tree256(float v, lds_f32* area, int tc, lds_u32* ctr, unsigned& gen) {
#pragma clang fp contract(off)
  if (tc < 256) area[tc] = v;
  aux_bar(ctr, gen, tc & 63);
  float r = 0.0f;
  if (tc < 256) {
    const int l = tc & 63;
    r = (area[l] + area[l + 128]) + (area[l + 64] + area[l + 192]);
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) r = r + __shfl_xor(r, s, 64);
    r = __shfl(r, 0, 64);
  }
  return r;
}

__device__ __forceinline__ float aux_rsqrt(float v) { return 1.0f / __builtin_sqrtf(v); }

// aux op p in workgroup b of G, compute thread tc (0 .. 511); lds: kAuxLdsFloats floats of this workgroup's LDS, free
// during the op; ctr / gen: the compute waves' barrier (aux_bar). The caller has waited for op i - 1 in every
// workgroup, and waits for these stores (vmcnt) before it publishes the op. Not inlined: the chain kernels' GEMV code
// keeps its register allocation (inlined, these loops added VGPR spills to the M > 1 kernels). Returns gen.
__device__ __noinline__ unsigned aux_run(const GemvP* pp, int b, int G, int tc, lds_f32* lds, lds_u32* ctr,
                                         unsigned gen) {
#pragma clang fp contract(off)
  const GemvP& p = *pp;
  const int lane = tc & 63, wv = tc >> 6;
  if (p.kind == kOpCopy) {
    for (int64_t base = (int64_t)b * kAuxCopyWords; base < p.an; base += (int64_t)G * kAuxCopyWords) {
      unsigned v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i = base + u * kAuxThreads + tc;
        if (i < p.an) v[u] = aux_ldu(p.asrc + i);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i = base + u * kAuxThreads + tc;
        if (i < p.an) aux_stu(p.adst + i, v[u]);
      }
    }
    return gen;
  }
  int area = 0;   // the two tree areas alternate, so a tree's writes never meet a slower wave's reads of the one before
  for (int64_t r = b; r < p.arows; r += G) {
    if (p.kind == kOpArgmax) {   // engine/llm/lops.js:418-433 (any order gives its result: aux_better)
      const int64_t n = p.acols, base = r * n;
      float bv = -3.4e38f;
      uint32_t bi = 0xFFFFFFFFu;
      for (int64_t i0 = 0; i0 < n; i0 += kAuxBatch * kAuxThreads) {   // every compute thread, a batch of pairs in flight
        unsigned long long pr[kAuxBatch];
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u) {
          const int64_t i = i0 + u * kAuxThreads + tc;
          pr[u] = i < n ? aux_ld2(p.asrc + 2 * (base + i)) : 0xFFFFFFFFFF7FFFFFull;   // (-3.4e38 down, 0xFFFFFFFF)
        }
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u) {
          const float v = __uint_as_float((unsigned)pr[u]);
          const uint32_t id = (uint32_t)(pr[u] >> 32);
          if (aux_better(v, id, bv, bi)) { bv = v; bi = id; }
        }
      }
#pragma unroll
      for (int s = 32; s > 0; s >>= 1) {
        const float ov = __shfl_xor(bv, s, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, s, 64);
        if (aux_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      lds_f32* const ws = lds + area * 256;   // the waves' (value, index) results
      if (lane == 0) {
        ws[2 * wv] = bv;
        ws[2 * wv + 1] = __uint_as_float(bi);
      }
      aux_bar(ctr, gen, lane);
      if (tc == 0) {
        float fv = ws[0];
        uint32_t fi = __float_as_uint(ws[1]);
        for (int w = 1; w < kAuxWaves; ++w)
          if (aux_better(ws[2 * w], __float_as_uint(ws[2 * w + 1]), fv, fi)) { fv = ws[2 * w]; fi = __float_as_uint(ws[2 * w + 1]); }
        aux_stu(p.adst + 2 * r, fi);
        aux_stf(p.adst + 2 * r + 1, fv);
      }
      area ^= 1;
      continue;
    }
    if (p.kind == kOpRowstats) {   // engine/ops/misc.js:17-30
      const float* xr = p.asrc + r * p.ald + p.ac0;
      const int64_t cols = p.acols;
      float mean = 0.0f;
      if (p.amode == 0) {
        float s = 0.0f;
        if (tc < 256)
          for (int64_t i0 = tc; i0 < cols; i0 += kAuxBatch * 256) {
            float v[kAuxBatch];
#pragma unroll
            for (int u = 0; u < kAuxBatch; ++u) v[u] = i0 + u * 256 < cols ? aux_ldf(xr + i0 + u * 256) : 0.0f;
#pragma unroll
            for (int u = 0; u < kAuxBatch; ++u)
              if (i0 + u * 256 < cols) s = s + v[u];
          }
        mean = aux_tree256(s, lds + area * 256, tc, ctr, gen) / (float)cols;
        area ^= 1;
      }
      float q = 0.0f;
      if (tc < 256)
        for (int64_t i0 = tc; i0 < cols; i0 += kAuxBatch * 256) {
          float v[kAuxBatch];
#pragma unroll
          for (int u = 0; u < kAuxBatch; ++u) v[u] = i0 + u * 256 < cols ? aux_ldf(xr + i0 + u * 256) : 0.0f;
#pragma unroll
          for (int u = 0; u < kAuxBatch; ++u)
            if (i0 + u * 256 < cols) {
              const float d = v[u] - mean;
              q = q + d * d;
            }
        }
      const float var = aux_tree256(q, lds + area * 256, tc, ctr, gen) / (float)cols;
      area ^= 1;
      if (tc == 0) {
        aux_stf(p.adst + (p.astOff + r) * 2, mean);
        aux_stf(p.adst + (p.astOff + r) * 2 + 1, aux_rsqrt(var + p.aeps));
      }
      continue;
    }
    // normadd, engine/llm/lops.js:153-170: the t sums are added again in the second pass (the same order, the same
    // bits) instead of being kept in LDS
    const int64_t D = p.acols, xb = r * D;
    // t of elements i0 + 256 u (u < kAuxBatch, those < D): the partials added in j order, a batch of loads per j
    auto tsum = [&](int64_t i0, float (&t)[kAuxBatch]) {
#pragma unroll
      for (int u = 0; u < kAuxBatch; ++u) t[u] = 0.0f;
      for (int64_t j = 0; j < p.an; ++j) {
        float v[kAuxBatch];
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u)
          v[u] = i0 + u * 256 < D ? aux_ldf(p.asrc + j * p.aldp + xb + i0 + u * 256) : 0.0f;
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u) t[u] = t[u] + v[u];
      }
    };
    float s = 0.0f;
    if (tc < 256)
      for (int64_t i0 = tc; i0 < D; i0 += kAuxBatch * 256) {
        float t[kAuxBatch];
        tsum(i0, t);
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u)
          if (i0 + u * 256 < D) s = s + t[u] * t[u];
      }
    const float rs = aux_rsqrt(aux_tree256(s, lds + area * 256, tc, ctr, gen) / (float)D + p.aeps);
    area ^= 1;
    float s2 = 0.0f;
    if (tc < 256)
      for (int64_t i0 = tc; i0 < D; i0 += kAuxBatch * 256) {
        float t[kAuxBatch], xv[kAuxBatch], wv8[kAuxBatch];
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u) {
          const bool in = i0 + u * 256 < D;
          xv[u] = in ? aux_ldf(p.adst + xb + i0 + u * 256) : 0.0f;
          wv8[u] = in && p.amode == 0 ? aux_ldf(p.aw + p.awOff + i0 + u * 256) : 0.0f;
        }
        tsum(i0, t);
#pragma unroll
        for (int u = 0; u < kAuxBatch; ++u) {
          if (i0 + u * 256 >= D) continue;
          float x = xv[u];
          if (p.amode == 0) x = (x + t[u] * rs * wv8[u]) * p.ascale;
          else x = t[u];
          aux_stf(p.adst + xb + i0 + u * 256, x);
          s2 = s2 + x * x;
        }
      }
    const float r2 = aux_tree256(s2, lds + area * 256, tc, ctr, gen);
    area ^= 1;
    if (tc == 0) aux_stf(p.ast + p.astOff + r, aux_rsqrt(r2 / (float)D + p.aeps));
  }
  return gen;
}

}  // namespace p0
