// util.hip - bit-exact q4g32a.t64 dequant and the synthetic-data fillers.
#include "common.hpp"

namespace p0 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// One thread per (row, code word): the 8 weights k = 32 g + 8 w .. + 7 of row n.
// fl32(q * s + m) as engine/kcheck.js:32 / engine/core/store.js:291 compute it (q * s is exact in f32, so the fused and
// unfused forms round the same), and fl16 of that as the GEMM tile (engine/ops/gemm.js:147-148).
__global__ void q4_dequant_kernel(const uint8_t* __restrict__ w, int64_t wG, int64_t N, int64_t K, float* __restrict__ o32,
                                  uint16_t* __restrict__ o16) {
  const int64_t words = N * (K / 8);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = i / (K / 8), kw = i - n * (K / 8), g = kw >> 2, wd = kw & 3;
    const uint8_t* rec = w + ((n >> 6) * wG + g) * 1280;
    const int r = (int)(n & 63);
    const uint32_t q = *(const uint32_t*)(rec + r * 16 + wd * 4);
    const h2_t sm = __builtin_bit_cast(h2_t, *(const uint32_t*)(rec + 1024 + r * 4));
    const float s = (float)sm.x, m = (float)sm.y;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = (float)((q >> (4 * j)) & 15u) * s + m;
      const int64_t o = n * K + kw * 8 + j;
      if (o32) o32[o] = v;
      if (o16) o16[o] = __builtin_bit_cast(uint16_t, (_Float16)v);
    }
  }
}

// The PCG RXS-M-XS hash (Jarzynski & Olano, JCGT 2020), as the reference's GPU filler (engine/tune/autotune.js:76).
__device__ __forceinline__ uint32_t hash32(uint32_t x) {
  uint32_t v = x * 747796405u + 2891336453u;
  uint32_t w = ((v >> ((v >> 28) + 4u)) ^ v) * 277803737u;
  return (w >> 22) ^ w;
}
__device__ __forceinline__ double u01(uint32_t h) { return ((double)(h >> 8) + 0.5) * (1.0 / 16777216.0); }
__device__ __forceinline__ double hnorm(uint32_t idx, uint32_t seed) {   // Box-Muller in float64
  const double a = u01(hash32((2u * idx) ^ seed)), b = u01(hash32((2u * idx + 1u) ^ seed ^ 0x9E3779B9u));
  return sqrt(-2.0 * log(a)) * cos(6.283185307179586 * b);
}

// One thread per u32 of a record: words 0..255 = codes (uniform nibbles), 256..319 = f16(|z| sigma) | f16(-8 s) << 16
__global__ void fill_q4_sym_kernel(uint32_t* __restrict__ w, int64_t nrec, uint32_t seed, float sigma) {
  const int64_t words = nrec * 320;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rc = i / 320;
    const int j = (int)(i - rc * 320);
    uint32_t v;
    if (j < 256) {
      v = hash32((uint32_t)(rc * 256 + j) ^ seed);
    } else {
      const double z = hnorm((uint32_t)(rc * 64 + (j - 256)), seed ^ 0x5bd1e995u);
      const _Float16 sh = (_Float16)(float)(fabs(z) * (double)sigma);
      const _Float16 mh = (_Float16)(-8.0f * (float)sh);
      v = (uint32_t)__builtin_bit_cast(uint16_t, sh) | ((uint32_t)__builtin_bit_cast(uint16_t, mh) << 16);
    }
    w[i] = v;
  }
}

__global__ void fill_randn_kernel(void* __restrict__ dst, int64_t n, uint32_t seed, float sigma, int as_f16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const _Float16 h = (_Float16)(float)(hnorm((uint32_t)i, seed) * (double)sigma);
    if (as_f16) ((uint16_t*)dst)[i] = __builtin_bit_cast(uint16_t, h);
    else ((float*)dst)[i] = (float)h;
  }
}

static unsigned grid_for(int64_t work) {
  int64_t b = (work + 255) / 256;
  return (unsigned)(b > 16384 ? 16384 : (b < 1 ? 1 : b));
}

}  // namespace p0

using namespace p0;

extern "C" int p0_q4_dequant(const void* w, int64_t w_off, int64_t N, int64_t K, float* out32, uint16_t* out16) {
  if (N <= 0 || N % 64) { set_error("dequant: N %% 64"); return P0_EINVAL; }
  if (K <= 0 || K % 32) { set_error("dequant: K must be a multiple of 32"); return P0_EINVAL; }
  if (w_off % 4) { set_error("dequant: weight offset"); return P0_EINVAL; }
  if (!w || (!out32 && !out16)) { set_error("dequant: missing buffer"); return P0_EINVAL; }
  if (int r = require_open("dequant")) return r;
  hipLaunchKernelGGL(q4_dequant_kernel, dim3(grid_for(N * K / 8)), dim3(256), 0, ctx().cur, (const uint8_t*)w + w_off, K / 32,
                     N, K, out32, out16);
  P0_LAUNCHED("dequant");
  return P0_OK;
}

extern "C" int p0_fill_q4_sym(void* w, int64_t w_off, int64_t N, int64_t K, uint32_t seed, float sigma) {
  if (N <= 0 || N % 64 || K <= 0 || K % 32) { set_error("fill_q4_sym: N %% 64 and K %% 32 required"); return P0_EINVAL; }
  if (w_off % 4) { set_error("fill_q4_sym: weight offset"); return P0_EINVAL; }
  if (!w) { set_error("fill_q4_sym: missing buffer"); return P0_EINVAL; }
  if (int r = require_open("fill_q4_sym")) return r;
  const int64_t nrec = (N / 64) * (K / 32);
  hipLaunchKernelGGL(fill_q4_sym_kernel, dim3(grid_for(nrec * 320)), dim3(256), 0, ctx().cur,
                     (uint32_t*)((uint8_t*)w + w_off), nrec, seed, sigma);
  P0_LAUNCHED("fill_q4_sym");
  return P0_OK;
}

// The dense fp16 matrix-core rate this chip sustains: every wave of one 8-wave workgroup per CU runs `iters` rounds of
// 4 independent v_mfma_f32_32x32x16_f16 chains (no memory traffic; the sum goes to `sink` only on a value it never
// takes, so the arithmetic stays live). The measured peak that bench.py reports beside the spec-sheet one.
__global__ __launch_bounds__(512) void mfma_probe_kernel(int64_t iters, float* sink) {
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  const int lane = threadIdx.x & 63;
  half8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (_Float16)(0.125f * (float)((lane + j) & 7));
    b[j] = (_Float16)(0.0625f * (float)((lane * 3 + j) & 7));
  }
  f32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[c][e] = 0.0f;
  for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[c][e];
  if (s == -1.0f) sink[blockIdx.x] = s;
}

extern "C" int p0_probe_mfma(int64_t iters, float* sink, double* flops_out) {
  if (iters <= 0 || !sink) { set_error("probe_mfma: iters > 0 and a sink buffer of one float per CU required"); return P0_EINVAL; }
  if (int r = require_open("probe_mfma")) return r;
  const int grid = ctx().cu_count > 0 ? ctx().cu_count : 1;
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(grid), dim3(512), 0, ctx().cur, iters, sink);
  P0_LAUNCHED("probe_mfma");
  if (flops_out) *flops_out = (double)grid * 8 * 4 * 32768.0 * (double)iters;
  return P0_OK;
}

// the HBM read rate: a grid-stride stream of 16-byte loads over the buffer, XOR-folded per thread; the sink is written
// only on a fold value the caller's data does not give (the loads cannot be dropped)
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* __restrict__ p, int64_t n, uint32_t* sink) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (; i < n; i += stride) {
    const uint4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

extern "C" int p0_probe_read(const void* buf, int64_t bytes, uint32_t* sink) {
  if (!buf || !sink || bytes <= 0 || bytes % 16) {
    set_error("probe_read: a buffer of a positive multiple of 16 bytes and a sink word required");
    return P0_EINVAL;
  }
  if (int r = require_open("probe_read")) return r;
  hipLaunchKernelGGL(read_probe_kernel, dim3(2048), dim3(256), 0, ctx().cur, (const uint4*)buf, bytes / 16, sink);
  P0_LAUNCHED("probe_read");
  return P0_OK;
}

extern "C" int p0_fill_randn(void* dst, int64_t off_bytes, int64_t n, uint32_t seed, float sigma, int32_t as_f16) {
  if (!dst || n < 0 || off_bytes % (as_f16 ? 2 : 4)) { set_error("fill_randn: bad destination"); return P0_EINVAL; }
  if (int r = require_open("fill_randn")) return r;
  if (!n) return P0_OK;
  hipLaunchKernelGGL(fill_randn_kernel, dim3(grid_for(n)), dim3(256), 0, ctx().cur, (void*)((uint8_t*)dst + off_bytes), n, seed,
                     sigma, as_f16);
  P0_LAUNCHED("fill_randn");
  return P0_OK;
}
