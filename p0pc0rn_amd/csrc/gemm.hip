// gemm.hip - q4g32a.t64 dequant-GEMM on gfx950 MFMA: Y[m, n] = sum_k X'[m, k] * fl16(fl32(q s + m))[n, k].
//
// Replaces the WebGPU dispatch of gemm (engine/ops/gemm.js:255-322) for the q4 encoding, with its prologues
// f16 | lnmod | rms (engine/ops/gemm.js:55-63; plus bf16 activations converted to fp16) and epilogues
// f16 | f32 | resadd | swiglu | bias (engine/ops/gemm.js:187-211).
//
// Mapping: a workgroup of 4 waves owns a BM x BN output tile; per 32-k step (one q4 group, the reference's BK) it stages
// the prologue-applied fp16 X tile and the dequantised fp16 W tile in LDS, then each wave runs 32x32x16 fp16 MFMAs
// over its (BM/2) x (BN/2) sub-tile with fp32 accumulators. The W tile value is fl16(fl32(q * s + m)), the
// reference's own fp16 tile rounding (engine/ops/gemm.js:147-148), so the only difference from the reference is the
// fp32 summation order inside the MFMA.
#include "common.hpp"

namespace p0 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));

struct GemmP {
  const uint8_t* w; int64_t wG; int64_t Nw;
  const uint8_t* x; int64_t ldx, kx0; int xmode;
  int M, N, K;
  int64_t wr0, wr1, wk0;
  int epi;
  uint8_t* y; int64_t ldy, ny0;
  const float* ev; int64_t evOff;
  const float* st; int64_t stOff;
  const float* pv; int64_t pvOff; uint32_t pvShift;   // shift base = (pv_off + pv_stride) mod 2^32
  const float* bv; int64_t bvOff, bvUp;
  int act, store, res;
};

constexpr int BM = 128, BN = 128, BK = 32, LDK = BK + 8;   // LDS row stride 40 halves (80 B)

__device__ __forceinline__ _Float16 to_h(float v) { return (_Float16)v; }   // RNE

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// 8 prologue-applied fp16 values of X row `row`, k = k0 + 8 c .. + 7 (engine/ops/gemm.js:55-63)
__device__ __forceinline__ half8 xload8(const GemmP& p, int row, int k) {
  half8 h;
  const int64_t idx = (int64_t)row * p.ldx + p.kx0 + k;
  if (p.xmode == P0_XMODE_F16 || p.xmode == P0_XMODE_BF16) {
    const uint16_t* src = (const uint16_t*)p.x + idx;
    uint16_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = src[j];
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = p.xmode == P0_XMODE_F16 ? __builtin_bit_cast(_Float16, v[j]) : to_h(bf16_to_f32(v[j]));
  } else {
    const float* src = (const float*)p.x + idx;
    const float* s = p.st + (p.stOff + row) * 2;
    const float mean = s[0], rstd = s[1];
    const int64_t kk = p.kx0 + k;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float xv = src[j];
      float t;
      if (p.xmode == P0_XMODE_LNMOD) t = (xv - mean) * rstd * (1.0f + p.pv[p.pvOff + kk + j]) + p.pv[(int64_t)p.pvShift + kk + j];
      else t = xv * rstd * p.pv[p.pvOff + kk + j];
      h[j] = to_h(t);
    }
  }
  return h;
}

// weight row of ws column n (engine/ops/gemm.js:94-97)
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

__global__ __launch_bounds__(256) void q4_gemm_kernel(GemmP p) {
  __shared__ _Float16 xs[BM * LDK];
  __shared__ _Float16 ws[BN * LDK];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // staging assignments: X: thread -> (row tid / 2, 16 k from (tid & 1) * 16); W: thread -> (row tid / 2, words 2 (tid & 1) .. +1)
  const int sr = tid >> 1, sc = tid & 1;
  const int xrow = min(m0 + sr, p.M - 1);   // rows past M repeat the last row (engine/ops/gemm.js:132-133); never stored
  const int ncol = n0 + sr;
  const bool wvalid = ncol < p.N;
  const int64_t wr = wvalid ? wrow(p, ncol) : 0;
  const uint8_t* wrec_row = p.w + (wr >> 6) * p.wG * 1280 + (wr & 63) * 16;
  const uint8_t* wsm_row = p.w + (wr >> 6) * p.wG * 1280 + 1024 + (wr & 63) * 4;

  for (int k0 = 0; k0 < p.K; k0 += BK) {
    // ---- X tile (prologue applied, fp16)
    {
      const half8 a = xload8(p, xrow, k0 + sc * 16), b = xload8(p, xrow, k0 + sc * 16 + 8);
      *(half8*)&xs[sr * LDK + sc * 16] = a;
      *(half8*)&xs[sr * LDK + sc * 16 + 8] = b;
    }
    // ---- W tile: two code words of one row -> 16 fp16 weights
    {
      const int64_t gi = (p.wk0 + k0) >> 5;
      half8 o0, o1;
      if (wvalid) {
        const uint32_t* q = (const uint32_t*)(wrec_row + gi * 1280) + sc * 2;
        const h2_t sm = __builtin_bit_cast(h2_t, *(const uint32_t*)(wsm_row + gi * 1280));
        const float s = (float)sm.x, mn = (float)sm.y;
        const uint32_t q0 = q[0], q1 = q[1];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          o0[j] = to_h((float)((q0 >> (4 * j)) & 15u) * s + mn);
          o1[j] = to_h((float)((q1 >> (4 * j)) & 15u) * s + mn);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) { o0[j] = (_Float16)0.0f; o1[j] = (_Float16)0.0f; }
      }
      *(half8*)&ws[sr * LDK + sc * 16] = o0;
      *(half8*)&ws[sr * LDK + sc * 16 + 8] = o1;
    }
    __syncthreads();
    // ---- MFMA: 2 k-steps of 16, 2 x 2 blocks of 32 x 32 per wave
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        av[i] = *(const half8*)&xs[(wm * 64 + i * 32 + (lane & 31)) * LDK + kk + (lane >> 5) * 8];
        bv[i] = *(const half8*)&ws[(wn * 64 + i * 32 + (lane & 31)) * LDK + kk + (lane >> 5) * 8];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // ---- epilogue: acc[i][j][e] is row 8 (e / 4) + 4 (lane / 32) + e % 4, column lane % 32 of block (i, j)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int n = n0 + wn * 64 + j * 32 + (lane & 31);
        const float a = acc[i][j][e];
        const float up = __shfl_xor(a, 1, 64);   // swiglu: the odd column (up) of an even column's pair
        if (m >= p.M || n >= p.N) continue;
        const int64_t o = (int64_t)m * p.ldy + p.ny0;
        if (p.epi == P0_GEPI_F16) {
          ((_Float16*)p.y)[o + n] = to_h(a);
        } else if (p.epi == P0_GEPI_F32) {
          ((float*)p.y)[o + n] = a;
        } else if (p.epi == P0_GEPI_RESADD) {
          const float g = p.ev ? p.ev[p.evOff + n] : 1.0f, b = p.bv ? p.bv[p.bvOff + n] : 0.0f;
          float* yp = (float*)p.y + o + n;
          *yp = p.store ? g * (a + b) : *yp + g * (a + b);
        } else if (p.epi == P0_GEPI_BIAS) {
          _Float16* yp = (_Float16*)p.y + o + n;
          float r = a + p.ev[p.evOff + n];
          if (p.res) r += (float)*yp;
          *yp = to_h(r);
        } else if (!(n & 1)) {   // swiglu: gate = even column, up = the next one (engine/ops/gemm.js:200-206)
          const int jn = n >> 1;
          const float gB = p.bv ? p.bv[p.bvOff + jn] : 0.0f, uB = p.bv ? p.bv[p.bvOff + p.bvUp + jn] : 0.0f;
          ((_Float16*)p.y)[o + jn] = to_h(act_f(p, a + gB) * (up + uB));
        }
      }
}

static const char* gepi_name(int e) {
  switch (e) {
    case P0_GEPI_F16: return "f16";
    case P0_GEPI_F32: return "f32";
    case P0_GEPI_RESADD: return "resadd";
    case P0_GEPI_SWIGLU: return "swiglu";
    case P0_GEPI_BIAS: return "bias";
  }
  return "?";
}

}  // namespace p0

using namespace p0;

extern "C" int p0_q4_gemm(const p0_gemm_args_t* a, double* flops_out) {
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
  if (a->x_mode < P0_XMODE_F16 || a->x_mode > P0_XMODE_BF16) { set_error("gemm: x mode %d", a->x_mode); return P0_EINVAL; }
  if (a->epi < P0_GEPI_F16 || a->epi > P0_GEPI_BIAS) { set_error("gemm: epilogue %d", a->epi); return P0_EINVAL; }
  if (a->epi == P0_GEPI_SWIGLU && (N & 1)) { set_error("gemm: swiglu needs an even N"); return P0_EINVAL; }
  if (!a->w || !a->x || !a->y) { set_error("gemm: missing w, x or y buffer"); return P0_EINVAL; }
  if ((a->x_mode == P0_XMODE_LNMOD || a->x_mode == P0_XMODE_RMS) && (!a->stats || !a->pv)) {
    set_error("gemm: %s needs stats and pv", a->x_mode == P0_XMODE_LNMOD ? "lnmod" : "rms"); return P0_EINVAL;
  }
  if (a->epi == P0_GEPI_BIAS && !a->ev) { set_error("gemm: bias needs ev"); return P0_EINVAL; }
  if (int r = require_open("gemm")) return r;

  GemmP p{};
  p.w = (const uint8_t*)a->w + a->w_off;
  p.wG = a->w_cols / 32;
  p.Nw = a->w_rows;
  p.x = (const uint8_t*)a->x + a->x_off;
  p.ldx = a->x_ld ? a->x_ld : K;
  p.kx0 = a->x_k0;
  p.xmode = a->x_mode;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.wr0 = a->wr0; p.wr1 = a->wr1; p.wk0 = a->wk0;
  p.epi = a->epi;
  p.y = (uint8_t*)a->y + a->y_off;
  p.ldy = a->y_ld ? a->y_ld : N;
  p.ny0 = a->y_n0;
  p.ev = a->ev; p.evOff = a->ev_off;
  p.st = a->stats; p.stOff = a->stats_off;
  p.pv = a->pv; p.pvOff = a->pv_off; p.pvShift = (uint32_t)(a->pv_off + a->pv_stride);
  p.bv = a->bv; p.bvOff = a->bv_off; p.bvUp = a->bv_up;
  p.act = a->act; p.store = a->store; p.res = a->res;
  (void)gepi_name;
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  hipLaunchKernelGGL(q4_gemm_kernel, grid, dim3(256), 0, ctx().cur, p);
  P0_LAUNCHED("gemm");
  if (flops_out) *flops_out = 2.0 * (double)M * (double)N * (double)K;
  return P0_OK;
}
