// misc.hip - the GEMV's producer and consumers in a decode step: row statistics (the rstd slot an rms prologue reads),
// the split-K sum with the residual RMS update (normadd), and the argmax over the per-tile maxima a softcap GEMV
// writes. One workgroup of 256 threads per row, summing in the reference's order (thread t takes elements t, t + 256,
// ... in turn, then a halving tree over the 256 partials), so the fp32 sums equal the reference's, bit for bit.
#include "common.hpp"

// no FMA contraction: every a + b * c rounds the product and the sum separately, as the CPU restatement does, so the
// device sums and the oracle's agree bit for bit
#pragma clang fp contract(off)

namespace p0 {

constexpr int kRowThreads = 256;

// the reference's halving tree over red[0..255] (engine/ops/misc.js:20-23, engine/llm/lops.js:158-159): level s adds
// red[t + s] into red[t] for t < s; every thread gets red[0]
__device__ __forceinline__ float tree256(float v, float* red) {
  const int t = threadIdx.x;
  red[t] = v;
  __syncthreads();
#pragma unroll
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s) red[t] = red[t] + red[t + s];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float rsqrt_exact(float v) { return 1.0f / __builtin_sqrtf(v); }

// engine/ops/misc.js:17-30
__global__ __launch_bounds__(kRowThreads) void rowstats_kernel(const float* __restrict__ x, int64_t ld, int64_t c0,
                                                              int64_t rows, int64_t cols, int mode, float eps,
                                                              float* __restrict__ st, int64_t st_off) {
  __shared__ float red[kRowThreads];
  const int t = threadIdx.x;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* xr = x + row * ld + c0;
    float mean = 0.0f;
    if (mode == 0) {
      float s = 0.0f;
      for (int64_t i = t; i < cols; i += kRowThreads) s = s + xr[i];
      mean = tree256(s, red) / (float)cols;
    }
    float q = 0.0f;
    for (int64_t i = t; i < cols; i += kRowThreads) {
      const float d = xr[i] - mean;
      q = q + d * d;
    }
    const float var = tree256(q, red) / (float)cols;
    if (t == 0) {
      st[(st_off + row) * 2] = mean;
      st[(st_off + row) * 2 + 1] = rsqrt_exact(var + eps);
    }
  }
}

// engine/llm/lops.js:153-170; the t sums of a row live in LDS (dynamic: D floats)
__global__ __launch_bounds__(kRowThreads) void normadd_kernel(const float* __restrict__ T, int64_t nsrc, int64_t ldp,
                                                             const float* __restrict__ W, int64_t woff,
                                                             float* __restrict__ X, float* __restrict__ ST,
                                                             int64_t stoff, int64_t D, float eps, float scale,
                                                             int mode) {
  __shared__ float red[kRowThreads];
  extern __shared__ float tv[];
  const int t = threadIdx.x;
  const int64_t m = blockIdx.x, xb = m * D;
  float s = 0.0f;
  for (int64_t i = t; i < D; i += kRowThreads) {
    float v = 0.0f;
    for (int64_t j = 0; j < nsrc; ++j) v = v + T[j * ldp + xb + i];
    tv[i] = v;
    s = s + v * v;
  }
  const float rs = rsqrt_exact(tree256(s, red) / (float)D + eps);
  float s2 = 0.0f;
  for (int64_t i = t; i < D; i += kRowThreads) {
    float xv = X[xb + i];
    if (mode == 0) xv = (xv + tv[i] * rs * W[woff + i]) * scale;
    else xv = tv[i];
    X[xb + i] = xv;
    s2 = s2 + xv * xv;
  }
  const float r2 = tree256(s2, red);
  if (t == 0) ST[stoff + m] = rsqrt_exact(r2 / (float)D + eps);
}

// engine/llm/lops.js:418-433, engine/llm/lops_spec.js:329-343: (value, index) with ties to the lower index
__device__ __forceinline__ bool better(float v, uint32_t id, float bv, uint32_t bi) {
  return v > bv || (v == bv && id < bi);
}
__global__ __launch_bounds__(kRowThreads) void argmax_kernel(const float* __restrict__ MX, int64_t n,
                                                            uint32_t* __restrict__ out) {
  __shared__ float rv[kRowThreads];
  __shared__ uint32_t ri[kRowThreads];
  const int t = threadIdx.x;
  const int64_t b = (int64_t)blockIdx.x * n;
  float bv = -3.4e38f;
  uint32_t bi = 0xFFFFFFFFu;
  for (int64_t i = t; i < n; i += kRowThreads) {
    const float v = MX[2 * (b + i)];
    const uint32_t id = __float_as_uint(MX[2 * (b + i) + 1]);
    if (better(v, id, bv, bi)) { bv = v; bi = id; }
  }
  rv[t] = bv;
  ri[t] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (t < s && better(rv[t + s], ri[t + s], rv[t], ri[t])) { rv[t] = rv[t + s]; ri[t] = ri[t + s]; }
    __syncthreads();
  }
  if (t == 0) {
    out[2 * blockIdx.x] = ri[0];
    out[2 * blockIdx.x + 1] = __float_as_uint(rv[0]);
  }
}

// normadd's LDS allowance (one row of up to 150 KB), set once at p0_open
int misc_init() {
  P0_HIP(hipFuncSetAttribute((const void*)normadd_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024),
         "p0_open: normadd");
  return P0_OK;
}

}  // namespace p0

using namespace p0;

extern "C" int p0_rowstats(const p0_rowstats_args_t* a) {
  if (!a) { set_error("rowstats: no arguments"); return P0_EINVAL; }
  if (a->rows < 0 || a->cols <= 0) { set_error("rowstats: rows %lld, cols %lld", (long long)a->rows, (long long)a->cols); return P0_EINVAL; }
  if (a->mode != 0 && a->mode != 1) { set_error("rowstats: mode %d", (int)a->mode); return P0_EINVAL; }
  if (!a->x || !a->st) { set_error("rowstats: missing x or st buffer"); return P0_EINVAL; }
  if (a->x_off % 4) { set_error("rowstats: x offset"); return P0_EINVAL; }
  if (int r = require_open("rowstats")) return r;
  if (a->rows == 0) return P0_OK;
  const int64_t ld = a->x_ld ? a->x_ld : a->cols;
  if (building_chain())   // a chain op (chain_aux.hpp): the same sums in the same order
    return chain_add_rowstats((const float*)((const uint8_t*)a->x + a->x_off), ld, a->x_c0, a->rows, a->cols,
                              (int)a->mode, a->eps, a->st, a->st_off);
  const unsigned grid = (unsigned)(a->rows < 65536 * 4 ? a->rows : 65536 * 4);
  hipLaunchKernelGGL(rowstats_kernel, dim3(grid), dim3(kRowThreads), 0, ctx().cur,
                     (const float*)((const uint8_t*)a->x + a->x_off), ld, a->x_c0, a->rows, a->cols, (int)a->mode,
                     a->eps, a->st, a->st_off);
  P0_LAUNCHED("rowstats");
  return P0_OK;
}

extern "C" int p0_normadd(const p0_normadd_args_t* a) {
  if (!a) { set_error("normadd: no arguments"); return P0_EINVAL; }
  const int64_t D = a->D, M = a->M ? a->M : 1;
  if (D <= 0 || M < 0) { set_error("normadd: D %lld, M %lld", (long long)D, (long long)M); return P0_EINVAL; }
  if (a->mode != 0 && a->mode != 1) { set_error("normadd: mode %d", (int)a->mode); return P0_EINVAL; }
  if (!a->t || !a->x || !a->st || (a->mode == 0 && !a->w)) { set_error("normadd: missing t, w, x or st buffer"); return P0_EINVAL; }
  if (D * (int64_t)sizeof(float) > 150 * 1024) { set_error("normadd: D %lld exceeds this build's row buffer", (long long)D); return P0_EINVAL; }
  if (int r = require_open("normadd")) return r;
  const int64_t nsrc = a->t_n ? a->t_n : 1, ldp = a->t_ld ? a->t_ld : D * M;
  const float eps = a->eps != 0.0f ? a->eps : 1e-6f;
  if (building_chain())
    return chain_add_normadd(a->t, nsrc, ldp, a->w, a->w_off, a->x, a->st, a->st_off, D, M, eps, a->scale, (int)a->mode);
  const size_t lds = (size_t)D * sizeof(float);
  hipLaunchKernelGGL(normadd_kernel, dim3((unsigned)M), dim3(kRowThreads), lds, ctx().cur, a->t, nsrc, ldp, a->w,
                     a->w_off, a->x, a->st, a->st_off, D, eps, a->scale, (int)a->mode);
  P0_LAUNCHED("normadd");
  return P0_OK;
}

extern "C" int p0_argmaxM(const float* mx, int64_t n, int64_t M, uint32_t* out) {
  if (!mx || !out) { set_error("argmax: missing mx or out buffer"); return P0_EINVAL; }
  if (n < 0 || M < 1) { set_error("argmax: n %lld, M %lld", (long long)n, (long long)M); return P0_EINVAL; }
  if (int r = require_open("argmax")) return r;
  if (building_chain()) return chain_add_argmax(mx, n, M, out);
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)M), dim3(kRowThreads), 0, ctx().cur, mx, n, out);
  P0_LAUNCHED("argmax");
  return P0_OK;
}

extern "C" int p0_argmax(const float* mx, int64_t n, uint32_t* out) { return p0_argmaxM(mx, n, 1, out); }
