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

q8_kernel_t q8_kernel(int M) { return M == 1 ? q8_gemv_kernel<1> : q8_gemv_kernel<0>; }

}  // namespace p0
