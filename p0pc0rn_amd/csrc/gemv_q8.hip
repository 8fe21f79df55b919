// gemv_q8.hip - the q8g64s.t64 GEMV (M = 1, gemv) and GEMV-M (M <= 16, gemvM) on gfx950: the reference's other weight
// encoding on the same call surface (engine/llm/lops.js:74-80, engine/llm/lops_spec.js:165), with the same prologues,
// epilogues and split semantics as the q4 kernels (gemv_kernels.hpp).
//
// Data layout (packQ8, engine/kcheck.js:39-52): a weight W[N][K] is a sequence of 4224-byte records, record (tile, g)
// = rows 64 tile .. + 63, k = 64 g .. + 63, tile-major. Bytes [64 r, 64 r + 64) are row r's 64 signed codes in k order;
// bytes 4096 + 2 r hold its fp16 scale. The weight is q s (exact in fp32).
//
// Mapping: a workgroup of 4 waves owns one 64-row tile (a geglu: the gate tile and its up tile) and one split; lane =
// row. Wave v takes the groups v, v + 4, ... of the split: per group a lane loads its row's 64 code bytes (four
// 16-byte loads, the wave's 4 KB contiguous) and its scale. x' = prologue(x) is staged in LDS 1024 k at a time with
// the sums of its 64-groups. The codes are biased by 128 (a XOR of the sign bits), so each byte converts with one
// unsigned-byte convert: sum (q + 128) x' - 128 sum x' = sum q x'. The waves' sums are added in wave order (LDS), so the
// result does not depend on timing.
#include "gemv_kernels.hpp"

namespace p0 {

constexpr int kQ8Waves = 4, kQ8Threads = 64 * kQ8Waves, kQ8Chunk = 1024, kQ8CG = kQ8Chunk / 64;
// the M = 1 kernel: 16 waves, 2 groups per wave and round, splits of at most 3072 k
constexpr int kQ81Waves = 16, kQ81Threads = 64 * kQ81Waves, kQ81G = 2, kQ81MaxK = 3072;

size_t q8_lds_bytes(int M) {   // x' chunk, group sums, and the cross-wave reduction [wave][tile][m][lane]
  return (size_t)M * (kQ8Chunk + kQ8CG) * sizeof(float) + (size_t)kQ8Waves * 2 * M * 64 * sizeof(float);
}

// MT: the compile-time row count (1), or 0 = p.mrows rows (at most 16)
template <int MT>
__global__ __launch_bounds__(kQ8Threads) void q8_gemv_kernel(GemvP p) {
  constexpr int MM = MT ? MT : 16;
  const int M = MT ? MT : p.mrows;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* xs = smem;                           // [M][kQ8Chunk]
  float* xsum = xs + M * kQ8Chunk;            // [M][kQ8CG]
  float* red = xsum + M * kQ8CG;              // [wave][T][M][64]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const bool pair = p.epi == P0_EPI_GEGLU;
  const int T = pair ? 2 : 1;
  const int tile0 = blockIdx.x, split = blockIdx.y;
  const int64_t tiles[2] = {tile0, tile0 + (pair ? p.NT : 0)};
  const int k0s = split * p.kPer, k1s = min(p.K, k0s + p.kPer);

  float acc[2][MM];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[t][m] = 0.0f;

  for (int c0 = k0s; c0 < k1s; c0 += kQ8Chunk) {
    const int c1 = min(k1s, c0 + kQ8Chunk), ng = (c1 - c0) >> 6;
    __syncthreads();   // the previous chunk's x' is no longer read
    for (int i = tid; i < M * kQ8Chunk; i += kQ8Threads) {
      const int m = i / kQ8Chunk, kl = i - m * kQ8Chunk;
      xs[i] = c0 + kl < c1 ? prologue<false>(p, m, c0 + kl) : 0.0f;
    }
    __syncthreads();
    for (int i = tid; i < M * kQ8CG; i += kQ8Threads) {   // group sums in k order
      const int m = i / kQ8CG, gl = i - m * kQ8CG;
      float s = 0.0f;
      for (int j = 0; j < 64; ++j) s += xs[m * kQ8Chunk + gl * 64 + j];
      xsum[i] = s;
    }
    __syncthreads();
    for (int gl = wv; gl < ng; gl += kQ8Waves) {
      const int g = (c0 >> 6) + gl;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t >= T) break;
        const uint8_t* rec = p.w + (tiles[t] * p.wG + g) * 4224;
        u32x4 q[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = *P0_GLOBAL(const u32x4, rec + lane * 64 + j * 16);
        const uint32_t sw = *P0_GLOBAL(const uint32_t, rec + 4096 + (lane & ~1) * 2);
        const float s = (lane & 1) ? h2f_hi(sw) : h2f_lo(sw);
        float d[MM];
#pragma unroll
        for (int m = 0; m < MM; ++m) d[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t wd[4] = {q[j].x ^ 0x80808080u, q[j].y ^ 0x80808080u, q[j].z ^ 0x80808080u, q[j].w ^ 0x80808080u};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float b0 = (float)(wd[e] & 0xFFu), b1 = (float)((wd[e] >> 8) & 0xFFu);
            const float b2 = (float)((wd[e] >> 16) & 0xFFu), b3 = (float)(wd[e] >> 24);
            const int kk = gl * 64 + j * 16 + e * 4;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
              if (m >= M) break;
              const float4 x4 = *(const float4*)(xs + m * kQ8Chunk + kk);
              d[m] = __builtin_fmaf(b0, x4.x, __builtin_fmaf(b1, x4.y, __builtin_fmaf(b2, x4.z, __builtin_fmaf(b3, x4.w, d[m]))));
            }
          }
        }
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          if (m >= M) break;
          acc[t][m] = __builtin_fmaf(s, d[m] - 128.0f * xsum[m * kQ8CG + gl], acc[t][m]);
        }
      }
    }
  }

  // the waves' sums, added in wave order
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int m = 0; m < MM; ++m)
      if (t < T && m < M) red[((wv * 2 + t) * M + m) * 64 + lane] = acc[t][m];
  __syncthreads();
  if (wv != 0) return;
  for (int m = 0; m < M; ++m) {
    float tot[2] = {0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t >= T) break;
      float v = red[((0 * 2 + t) * M + m) * 64 + lane];
#pragma unroll
      for (int w = 1; w < kQ8Waves; ++w) v += red[((w * 2 + t) * M + m) * 64 + lane];
      tot[t] = v;
    }
    epilogue<false>(p, split, m, tile0, lane, tot[0], tot[1]);
  }
}

// M = 1 (gemv, the decode case): a workgroup of 16 waves per (64-row tile, split), every wave's record loads issued
// before the input is staged. Wave w takes groups w and 16 + w of each round of 32 (a geglu, two tiles: group w of
// each round of 16), so a split's records (at most 48 groups of 3072 k) are in flight in one to three rounds, the
// first round's latency overlapping the x' staging; the kernel above, 4 waves that load their groups one after another, spends a memory round trip per group.
// The group sums add the 64 x' of a group in k order; the waves' sums are added in wave order (deterministic).
// With p.nks > 1 a split's groups are cut into p.nks slices of consecutive groups, one workgroup each (blockIdx.y =
// split * nks + slice); wave 0 writes the slice's row sums to the uncached split-K workspace with device-scope stores
// and counts the arrival, and the last workgroup of the (split, tile) adds the slices' partials in slice order and
// runs the epilogue (the GEMV's split-K protocol, gemv_item).
template <int T>   // 2: a geglu (the gate tile and its up tile), else 1
__global__ __launch_bounds__(kQ81Threads) void q8_gemv1_kernel(GemvP p) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* xs = smem;                       // [kQ81MaxK] x' of the split
  float* xsum = xs + kQ81MaxK;            // [kQ81MaxK / 64] its group sums
  float* red = xsum + kQ81MaxK / 64;      // [wave][tile][64 rows]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int tile0 = blockIdx.x, split = (int)blockIdx.y / p.nks, ks = (int)blockIdx.y - split * p.nks;
  const int64_t tiles[2] = {tile0, tile0 + (T == 2 ? p.NT : 0)};
  // this workgroup's slice of the split: groups [gs0, gs0 + ng) (p.gps groups of 64 k a slice)
  const int sk0 = split * p.kPer, sk1 = min(p.K, sk0 + p.kPer);
  const int gs0 = (sk0 >> 6) + ks * p.gps, gs1 = min(sk1 >> 6, gs0 + p.gps);
  const int k0s = gs0 * 64, k1s = gs1 * 64, ng = gs1 - gs0, g0 = gs0;
  constexpr int GW = kQ81G / T;   // groups per wave and round (the registers of 2 tile-groups)
  float acc[2] = {0.0f, 0.0f};
  for (int r0 = 0; r0 < ng; r0 += kQ81Waves * GW) {
    u32x4 q[GW][T][4];
    uint32_t sw[GW][T];
#pragma unroll
    for (int b = 0; b < GW; ++b) {
      const int gl = min(r0 + b * kQ81Waves + wv, ng - 1);   // past the split: its last group again (unused)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint8_t* rec = p.w + (tiles[t] * p.wG + g0 + gl) * 4224;
#pragma unroll
        for (int j = 0; j < 4; ++j) q[b][t][j] = *P0_GLOBAL(const u32x4, rec + lane * 64 + j * 16);
        sw[b][t] = *P0_GLOBAL(const uint32_t, rec + 4096 + (lane & ~1) * 2);
      }
    }
    if (r0 == 0) {   // x' of the split while the first round's records are in flight, then its group sums
      for (int i = tid; i < k1s - k0s; i += kQ81Threads) xs[i] = prologue<false>(p, 0, k0s + i);
      __syncthreads();
      for (int gl = tid; gl < ng; gl += kQ81Threads) {
        float s = 0.0f;
        for (int j = 0; j < 64; ++j) s += xs[gl * 64 + j];
        xsum[gl] = s;
      }
      __syncthreads();
    }
#pragma unroll
    for (int b = 0; b < GW; ++b) {
      const int gl = r0 + b * kQ81Waves + wv;
      if (gl >= ng) break;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float s = (lane & 1) ? h2f_hi(sw[b][t]) : h2f_lo(sw[b][t]);
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t wd[4] = {q[b][t][j].x ^ 0x80808080u, q[b][t][j].y ^ 0x80808080u, q[b][t][j].z ^ 0x80808080u,
                                  q[b][t][j].w ^ 0x80808080u};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float b0 = (float)(wd[e] & 0xFFu), b1 = (float)((wd[e] >> 8) & 0xFFu);
            const float b2 = (float)((wd[e] >> 16) & 0xFFu), b3 = (float)(wd[e] >> 24);
            const float4 x4 = *(const float4*)(xs + gl * 64 + j * 16 + e * 4);
            d = __builtin_fmaf(b0, x4.x, __builtin_fmaf(b1, x4.y, __builtin_fmaf(b2, x4.z, __builtin_fmaf(b3, x4.w, d))));
          }
        }
        acc[t] = __builtin_fmaf(s, d - 128.0f * xsum[gl], acc[t]);
      }
    }
  }
  // the waves' sums, added in wave order
#pragma unroll
  for (int t = 0; t < 2; ++t)
    if (t < T) red[(wv * 2 + t) * 64 + lane] = acc[t];
  __syncthreads();
  if (wv != 0) return;
  float tot[2] = {0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (t >= T) break;
    float v = red[t * 64 + lane];
    for (int w = 1; w < kQ81Waves; ++w) v += red[(w * 2 + t) * 64 + lane];
    tot[t] = v;
  }
  if (p.nks > 1) {
    // rows of the (split, slice) partials: the tile's 64 rows, and for a geglu its up rows at N + ...
    const size_t base = (size_t)blockIdx.y * p.rowsTot;
#pragma unroll
    for (int t = 0; t < T; ++t) stf<true>(&p.part[base + (t ? p.N : 0) + tile0 * 64 + lane], tot[t]);
    __builtin_amdgcn_s_waitcnt(0);   // the partials (uncached memory) are written before the arrival count
    unsigned last = 0;
    if (lane == 0) {
      auto* c = P0_GLOBAL(unsigned, p.cnt + (size_t)split * p.NT + tile0);
      last = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(p.nks - 1);
      if (last) __hip_atomic_exchange(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // leave it at zero
    }
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    // the slices' partials, loaded 8 slices at a time and added in slice order
    const size_t sbase = (size_t)split * p.nks * p.rowsTot;
    float sum[2] = {0.0f, 0.0f};
    for (int s0 = 0; s0 < p.nks; s0 += 8) {
      float v[8][2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sl = min(s0 + j, p.nks - 1);   // past the last slice: re-read it (in bounds, not added)
#pragma unroll
        for (int t = 0; t < T; ++t) v[j][t] = ldf<true>(&p.part[sbase + (size_t)sl * p.rowsTot + (t ? p.N : 0) + tile0 * 64 + lane]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < p.nks) {
#pragma unroll
          for (int t = 0; t < T; ++t) sum[t] += v[j][t];
        }
    }
    tot[0] = sum[0];
    tot[1] = sum[1];
  }
  epilogue<false>(p, split, 0, tile0, lane, tot[0], tot[1]);
}

q8_kernel_t q8_kernel(int M) { return M == 1 ? q8_gemv_kernel<1> : q8_gemv_kernel<0>; }
q8_kernel_t q8_gemv1(bool geglu) { return geglu ? q8_gemv1_kernel<2> : q8_gemv1_kernel<1>; }
size_t q8_gemv1_lds_bytes() { return (kQ81MaxK + kQ81MaxK / 64 + kQ81Waves * 2 * 64) * sizeof(float); }

}  // namespace p0
