// gemv.hip - q4g32a.t64 GEMV (M = 1) and GEMV-M (M <= 16) for gfx950.
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
#include "common.hpp"

namespace p0 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
// 4-byte alignment is all a record base guarantees (weight offsets are multiples of 4, engine/llm/lops.js:124);
// global_load_dwordx4 needs only dword alignment, so one 16-byte load per lane serves both cases
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));

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
  float* part; unsigned* cnt;
};

__device__ __forceinline__ float gelu_tanh(float v) {   // engine/llm/lops.js:26
  float t = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  t = fminf(15.0f, fmaxf(-15.0f, t));
  return v * 0.5f * (1.0f + tanhf(t));
}

// prologue value x'[m][k] (engine/llm/lops.js:50-57, engine/llm/lops_spec.js:61-64)
__device__ __forceinline__ float prologue(const GemvP& p, int m, int k) {
  if (p.pro == P0_PRO_RAW) return p.X[m * p.ldx + p.rowB + k];
  if (p.pro == P0_PRO_RMS) return p.X[m * p.ldx + p.rowB + k] * p.ST[p.statOff + m * p.statLd] * p.NW[p.nOff + k];
  float s = 0.0f;
  for (int j = 0; j < p.nsrc; ++j) s += p.X[j * p.ldp + m * p.ldx + k];
  if (p.pro == P0_PRO_SUM) return s;
  return gelu_tanh(s) * p.EV[p.evOff + m * p.evLd + k];
}

struct Rec {
  u32x4 q;
  uint32_t sm;
};

__device__ __forceinline__ Rec load_rec(const GemvP& p, int64_t tile, int g, int lane) {
  const uint8_t* rec = p.w + (int64_t)__builtin_amdgcn_readfirstlane((int)((tile * p.wG + g) >> 0)) * 1280;
  Rec r;
  r.q = __builtin_nontemporal_load((const u32x4*)(rec + lane * 16));
  r.sm = __builtin_nontemporal_load((const uint32_t*)(rec + 1024 + lane * 4));
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

// the epilogue of one wave for x row m: tot0 = row sums of tile0 (gate tile for a geglu), tot1 = the up tile's
__device__ __forceinline__ void epilogue(const GemvP& p, int split, int m, int tile0, int lane, float tot0, float tot1) {
  const int n = tile0 * 64 + lane;
  if (p.epi == P0_EPI_STORE) {
    p.Y[split * p.ldy + m * p.ldm + n] = tot0;
  } else if (p.epi == P0_EPI_GEGLU) {
    p.Y[m * p.ldm + n] = gelu_tanh(tot0) * tot1;
  } else {
    float v = p.cap * tanhf(fminf(15.0f, fmaxf(-15.0f, tot0 / p.cap)));
    p.Y[m * p.ldm + n] = v;
    int r = lane;
    wave_argmax(v, r);
    if (lane == 0) {
      const int o = (m * p.NT + tile0) * 2;
      p.MX[o] = v;
      p.MX[o + 1] = __int_as_float(tile0 * 64 + r);
    }
  }
}

// MODE 0: one tile per wave; MODE 1: two tiles per wave; MODE 2: geglu (gate tile + its up tile N/64 tiles later).
// A workgroup = tgw tile slots x kw waves per slot; it owns the K-slice [g0, g1) of one split, and the kw waves of a
// slot take contiguous shares of it, reduced through LDS in wave order.
template <int M, int MODE>
__global__ __launch_bounds__(512) void q4_gemv_kernel(GemvP p) {
  constexpr int T = MODE == 0 ? 1 : 2;
  constexpr int TPW = MODE == 1 ? 2 : 1;   // distinct output tiles per wave
  extern __shared__ __attribute__((aligned(16))) float smem[];   // 16-byte aligned: ds_read_b128 of x
  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform indices live in SGPRs: record addresses become a scalar base plus the lane's constant 16-byte offset
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kwv = wv % p.kw, tw = wv / p.kw;
  const int KL = p.gps * 32;
  float* xs = smem;                    // [M][KL]   x' of the slice, odd k scaled 1/16
  float* xsum = smem + M * KL;         // [M][gps]  group sums of x'
  float* red = xsum + M * p.gps;       // [waves][T][64] in-workgroup reduction
  __shared__ int s_last;

  const int split = blockIdx.y / p.nks, ks = blockIdx.y - split * p.nks;
  const int k0s = split * p.kPer, k1s = min(p.K, k0s + p.kPer);
  const int gs0 = k0s >> 5, gs1 = k1s >> 5;
  const int g0 = min(gs1, gs0 + ks * p.gps), g1 = min(gs1, g0 + p.gps);
  const int sub = (g1 - g0 + p.kw - 1) / p.kw;
  const int wg0 = min(g1, g0 + kwv * sub), wg1 = min(g1, wg0 + sub);   // this wave's share

  // tiles of this wave
  const int slot = blockIdx.x * p.tgw + tw;
  int tile[T];
  if (MODE == 2) {
    tile[0] = slot;
    tile[T - 1] = slot + p.NT;
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) tile[t] = slot * TPW + t;
  }
  const bool active = tile[0] < p.NT;

  // ---- prologue: x'[m][k] for the workgroup's K-slice -> LDS (odd k scaled 1/16), then per-group sums of x'
  const int kb = g0 * 32, ke = g1 * 32;
  for (int idx = tid; idx < M * KL; idx += blockDim.x) {
    const int m = idx / KL, kl = idx - m * KL, k = kb + kl;
    float v = k < ke ? prologue(p, m, k) : 0.0f;
    xs[idx] = (k & 1) ? v * 0.0625f : v;
  }
  __syncthreads();
  for (int idx = tid; idx < M * p.gps; idx += blockDim.x) {
    const int m = idx / p.gps, gl = idx - m * p.gps;
    const float* xp = xs + m * KL + gl * 32;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) s += xp[i] + xp[i + 1] * 16.0f;
    xsum[idx] = s;
  }
  __syncthreads();

  // ---- stream the records of the wave's share
  float acc[T][M];
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
  // Chunks of D groups: all D (x T) records of a chunk are issued, then consumed in order. No load is carried across
  // the loop's back edge, so the compiler's wait counts stay exact (each consume waits for its own record only; a
  // rotating pipeline carried across the back edge made the counts collapse to near-full drains). The latency at
  // the start of each chunk is hidden by the other resident waves. Loads past the share's end re-read its last group
  // (in bounds, value unused), so every load is unconditional.
  constexpr int D = MODE == 0 ? 8 : 4;
  // a wave's second tile past N (odd tile count, MODE 1) re-reads its first tile; its results are never stored
  auto tl = [&](int t) -> int64_t { return (MODE == 1 && tile[t] >= p.NT) ? tile[0] : tile[t]; };
  if (active) {
    const int glast = wg1 - 1;
    for (int c0 = wg0; c0 < wg1; c0 += D) {
      Rec r[D][T];
#pragma unroll
      for (int i = 0; i < D; ++i)
#pragma unroll
        for (int t = 0; t < T; ++t) r[i][t] = load_rec(p, tl(t), min(c0 + i, glast), lane);
#pragma unroll
      for (int i = 0; i < D; ++i)
        if (c0 + i < wg1) consume(r[i], c0 + i);
    }
  }

  // ---- the kw waves of a slot: sum their shares in wave order into wave kwv == 0
  if (p.kw > 1) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      __syncthreads();
#pragma unroll
      for (int t = 0; t < T; ++t) red[(wv * T + t) * 64 + lane] = acc[t][m];
      __syncthreads();
      if (kwv == 0) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float s = 0.0f;
          for (int j = 0; j < p.kw; ++j) s += red[((wv + j) * T + t) * 64 + lane];
          acc[t][m] = s;
        }
      }
    }
  }

  // ---- one workgroup per split: the epilogue straight from registers
  if (p.nks == 1) {
    if (!active || kwv != 0) return;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if (MODE == 2) {
        epilogue(p, split, m, tile[0], lane, acc[0][m], acc[T - 1][m]);
      } else {
#pragma unroll
        for (int t = 0; t < T; ++t)
          if (tile[t] < p.NT) epilogue(p, split, m, tile[t], lane, acc[t][m], 0.0f);
      }
    }
    return;
  }

  // ---- several workgroups per split: partials -> workspace; the last workgroup of (split, tile block) to arrive
  // reduces them in K-slice order. One thread fences for the workgroup (a device-scope release / acquire writes back
  // / invalidates the whole L2 of the XCD, so it is done once, after the barrier that orders every wave's stores).
  const size_t sliceBase = (size_t)(split * p.nks) * M * p.rowsTot;
  const bool owner = active && kwv == 0;
  if (owner) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int row = (MODE == 2 && t == 1) ? p.N + tile[0] * 64 + lane : tile[t] * 64 + lane;
      if (MODE != 1 || tile[t] < p.NT) {
#pragma unroll
        for (int m = 0; m < M; ++m) p.part[sliceBase + ((size_t)ks * M + m) * p.rowsTot + row] = acc[t][m];
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    __threadfence();   // release: the workgroup's partials reach memory before the arrival count
    unsigned* c = p.cnt + (size_t)split * p.ntb + blockIdx.x;
    const unsigned prev = atomicAdd(c, 1u);
    const int last = prev == (unsigned)(p.nks - 1);
    if (last) {
      atomicExch(c, 0u);   // leave the counter at zero for the next call
      __threadfence();     // acquire: every other workgroup's partials
    }
    s_last = last;
  }
  __syncthreads();
  if (!s_last || !owner) return;

#pragma unroll
  for (int m = 0; m < M; ++m) {
    float tot[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      tot[t] = 0.0f;
      const int row = (MODE == 2 && t == 1) ? p.N + tile[0] * 64 + lane : tile[t] * 64 + lane;
      if (MODE != 1 || tile[t] < p.NT) {
        for (int s = 0; s < p.nks; ++s) tot[t] += p.part[sliceBase + ((size_t)s * M + m) * p.rowsTot + row];
      }
    }
    if (MODE == 2) {
      epilogue(p, split, m, tile[0], lane, tot[0], tot[T - 1]);
    } else {
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (tile[t] < p.NT) epilogue(p, split, m, tile[t], lane, tot[t], 0.0f);
    }
  }
}

// ------------------------------------------------------------------------------------------------ launch
typedef void (*gemv_kernel_t)(GemvP);

template <int M>
static gemv_kernel_t pick_m(int mode) {
  if (mode == 0) return q4_gemv_kernel<M, 0>;
  if (mode == 1) return q4_gemv_kernel<M, 1>;
  return q4_gemv_kernel<M, 2>;
}

static gemv_kernel_t pick(int M, int mode) {
  switch (M) {
    case 1: return pick_m<1>(mode);
    case 2: return pick_m<2>(mode);
    case 3: return pick_m<3>(mode);
    case 4: return pick_m<4>(mode);
    case 5: return pick_m<5>(mode);
    case 6: return pick_m<6>(mode);
    case 7: return pick_m<7>(mode);
    case 8: return pick_m<8>(mode);
    case 9: return pick_m<9>(mode);
    case 10: return pick_m<10>(mode);
    case 11: return pick_m<11>(mode);
    case 12: return pick_m<12>(mode);
    case 13: return pick_m<13>(mode);
    case 14: return pick_m<14>(mode);
    case 15: return pick_m<15>(mode);
    case 16: return pick_m<16>(mode);
  }
  return nullptr;
}

// tuning knobs (the analogue of the reference's per-device picks, engine/llm/lopsx.js:317-321)
static int g_target_waves = 2048;       // waves a call aims for before it splits K
static int g_two_tiles_min_nt = 1024;   // output tiles from which a wave streams two tiles
static int g_min_gpw = 2;               // fewest q4 groups a wave streams when K is split
static int g_max_kw = 4;                // most waves that share one tile slot's K-slice inside a workgroup

struct Plan {
  int mode, gps, nks, kw, tgw, ntb, rowsTot, waves;
  size_t lds;
};

static Plan plan(int M, int NT, int epi, int nsplit, int kPer) {
  Plan pl{};
  pl.mode = epi == P0_EPI_GEGLU ? 2 : (NT >= g_two_tiles_min_nt ? 1 : 0);
  const int T = pl.mode == 0 ? 1 : 2;
  const int slots = pl.mode == 1 ? (NT + 1) / 2 : NT;
  pl.rowsTot = (epi == P0_EPI_GEGLU ? 2 : 1) * NT * 64;
  const int Gs = kPer / 32;
  // K shares per slot and split: enough waves for the chip, but at least g_min_gpw groups each
  int kws = (g_target_waves + slots * nsplit - 1) / (slots * nsplit);
  const int kws_max = Gs / g_min_gpw > 1 ? Gs / g_min_gpw : 1;
  if (kws > kws_max) kws = kws_max;
  if (kws < 1) kws = 1;
  pl.kw = kws < g_max_kw ? kws : g_max_kw;
  pl.tgw = pl.kw >= 4 ? 1 : 4 / pl.kw;                 // 4 waves per workgroup unless kw is larger
  if (pl.tgw > slots) pl.tgw = slots;
  pl.waves = pl.tgw * pl.kw;
  int nks = (kws + pl.kw - 1) / pl.kw;
  int gps = (Gs + nks - 1) / nks;
  // LDS: x' and its group sums for the slice, plus the reduction rows
  const size_t red = (size_t)pl.waves * T * 64 * sizeof(float);
  int maxGps = (int)((48 * 1024 - red) / ((size_t)M * 33 * sizeof(float)));
  if (maxGps < 1) maxGps = 1;
  if (gps > maxGps) gps = maxGps;
  for (;;) {   // the partials must fit the workspace: coarser slices until they do
    nks = (Gs + gps - 1) / gps;
    if (nks == 1 || (size_t)nsplit * nks * M * pl.rowsTot <= ctx().part_floats || gps >= maxGps) break;
    gps = gps * 2 > maxGps ? maxGps : gps * 2;
  }
  pl.gps = gps;
  pl.nks = nks;
  pl.ntb = (slots + pl.tgw - 1) / pl.tgw;
  pl.lds = (size_t)M * gps * 33 * sizeof(float) + red;
  return pl;
}

static int launch(GemvP& p, int M, const char* op) {
  const Plan pl = plan(M, p.NT, p.epi, p.nsplit, p.kPer);
  if (pl.nks > 1 && (size_t)p.nsplit * pl.nks * M * pl.rowsTot > ctx().part_floats) {
    set_error("%s: split-K partials exceed the workspace (M %d, N %d, K %d)", op, M, p.N, p.K);
    return P0_EINVAL;
  }
  if ((size_t)p.nsplit * pl.ntb > ctx().n_counters) {
    set_error("%s: too many tile blocks for the workspace counters", op);
    return P0_EINVAL;
  }
  p.gps = pl.gps;
  p.nks = pl.nks;
  p.kw = pl.kw;
  p.tgw = pl.tgw;
  p.ntb = pl.ntb;
  p.rowsTot = pl.rowsTot;
  p.part = ctx().part;
  p.cnt = ctx().counters;
  gemv_kernel_t k = pick(M, pl.mode);
  dim3 grid((unsigned)pl.ntb, (unsigned)(p.nsplit * pl.nks));
  hipLaunchKernelGGL(k, grid, dim3(64 * pl.waves), pl.lds, ctx().cur, p);
  P0_LAUNCHED(op);
  return P0_OK;
}

static int check_enc(int32_t enc, const char* op) {
  if (enc == P0_ENC_Q4G32A_T64) return P0_OK;
  if (enc == P0_ENC_Q8G64S_T64) set_error("%s: encoding q8g64s.t64 is not supported by this build", op);
  else set_error("%s: encoding %d", op, (int)enc);
  return P0_EINVAL;
}

static const char* epi_name(int e) { return e == P0_EPI_GEGLU ? "geglu" : e == P0_EPI_SOFTCAP ? "softcap" : "store"; }

}  // namespace p0

using namespace p0;

extern "C" int p0_q4_gemv(const p0_gemv_args_t* a, int32_t* nsplit_out) {
  if (!a) { set_error("gemv: no arguments"); return P0_EINVAL; }
  if (int r = check_enc(a->w_enc, "gemv")) return r;
  const int64_t K = a->K, N = a->N;
  // engine/llm/lops.js:116-124, in the reference's order
  const int64_t kch = (!a->kPer && K > 2048) ? (K + 255) / 256 * 256 : 2048;
  if (kch > 3072) { set_error("gemv: K %lld needs a kPer", (long long)K); return P0_EINVAL; }
  const int64_t kPer = a->kPer ? (a->kPer < kch ? a->kPer : kch) : (K < kch ? K : kch);
  if (kPer <= 0 || kPer % 32) { set_error("gemv: kPer must be a multiple of 32"); return P0_EINVAL; }
  const int64_t nsplit = (K + kPer - 1) / kPer;
  if (a->epi != P0_EPI_STORE && nsplit > 1) { set_error("gemv: %s needs one split", epi_name(a->epi)); return P0_EINVAL; }
  if (N % 64) { set_error("gemv: N %% 64"); return P0_EINVAL; }
  if (a->w_off % 4) { set_error("gemv: weight offset"); return P0_EINVAL; }
  // this build's additional guards (the reference would read undefined memory here)
  if (K <= 0 || K % 32) { set_error("gemv: K must be a multiple of 32"); return P0_EINVAL; }
  if (N <= 0) { set_error("gemv: N must be positive"); return P0_EINVAL; }
  if (a->w_cols < K) { set_error("gemv: weight has %lld columns < K %lld", (long long)a->w_cols, (long long)K); return P0_EINVAL; }
  if (a->pro < P0_PRO_RAW || a->pro > P0_PRO_PLEG) { set_error("gemv: prologue %d", a->pro); return P0_EINVAL; }
  if (a->epi < P0_EPI_STORE || a->epi > P0_EPI_SOFTCAP) { set_error("gemv: epilogue %d", a->epi); return P0_EINVAL; }
  if (!a->w || !a->x || !a->y) { set_error("gemv: missing w, x or y buffer"); return P0_EINVAL; }
  if (a->pro == P0_PRO_RMS && (!a->norm || !(a->epi == P0_EPI_SOFTCAP ? a->mx : a->stat))) {
    set_error("gemv: rms needs norm and stat buffers"); return P0_EINVAL;
  }
  if (a->pro == P0_PRO_PLEG && !a->ev) { set_error("gemv: pleg needs an ev buffer"); return P0_EINVAL; }
  if (a->epi == P0_EPI_SOFTCAP && !a->mx) { set_error("gemv: softcap needs an mx buffer"); return P0_EINVAL; }
  if (int r = require_open("gemv")) return r;

  GemvP p{};
  p.w = (const uint8_t*)a->w + a->w_off;
  p.wG = a->w_cols / 32;
  p.N = (int)N; p.K = (int)K; p.kPer = (int)kPer; p.nsplit = (int)nsplit; p.NT = (int)(N / 64);
  p.pro = a->pro; p.epi = a->epi;
  p.X = a->x; p.ldx = 0; p.rowB = a->x_rowB;
  p.ST = a->epi == P0_EPI_SOFTCAP ? a->mx : a->stat;   // the rms rstd slot lives in mx for a softcap (lops.js:125)
  p.statOff = a->stat_off; p.statLd = 0;
  p.NW = a->norm; p.nOff = a->norm_off;
  p.nsrc = (int)a->src_n; p.ldp = a->src_ld;
  p.EV = a->ev; p.evOff = a->ev_off; p.evLd = 0;
  p.Y = a->y; p.ldy = a->ldy ? a->ldy : N; p.ldm = 0;
  p.MX = a->mx; p.cap = a->cap != 0.0f ? a->cap : 30.0f;
  if (int r = launch(p, 1, "gemv")) return r;
  if (nsplit_out) *nsplit_out = (int32_t)nsplit;
  return P0_OK;
}

extern "C" int p0_q4_gemvM(const p0_gemvm_args_t* a, int32_t* nsplit_out) {
  if (!a) { set_error("gemvM: no arguments"); return P0_EINVAL; }
  if (int r = check_enc(a->w_enc, "gemvM")) return r;
  const int64_t K = a->K, N = a->N, M = a->M;
  if (a->pro != P0_PRO_RAW && a->pro != P0_PRO_RMS && a->pro != P0_PRO_PLEG) {   // lops_spec.js:64
    set_error("gemvM: prologue %s", a->pro == P0_PRO_SUM ? "sum" : "?"); return P0_EINVAL;
  }
  if (M < 1 || M > 16) { set_error("gemvM: M %lld (this build: 1..16)", (long long)M); return P0_EINVAL; }
  // engine/llm/lops_spec.js:170-173, in the reference's order
  const int64_t kPer = a->kPer ? (a->kPer < 2048 ? a->kPer : 2048) : K;
  if (kPer <= 0 || kPer % 32) { set_error("gemvM: kPer must be a multiple of 32"); return P0_EINVAL; }
  const int64_t nsplit = (K + kPer - 1) / kPer;
  if (a->epi != P0_EPI_STORE && nsplit > 1) { set_error("gemvM: %s needs one split", epi_name(a->epi)); return P0_EINVAL; }
  if (N % 64) { set_error("gemvM: N %% 64"); return P0_EINVAL; }
  if (a->w_off % 4) { set_error("gemvM: weight offset"); return P0_EINVAL; }
  if (K <= 0 || K % 32) { set_error("gemvM: K must be a multiple of 32"); return P0_EINVAL; }
  if (N <= 0) { set_error("gemvM: N must be positive"); return P0_EINVAL; }
  if (a->w_cols < K) { set_error("gemvM: weight has %lld columns < K %lld", (long long)a->w_cols, (long long)K); return P0_EINVAL; }
  if (a->epi < P0_EPI_STORE || a->epi > P0_EPI_SOFTCAP) { set_error("gemvM: epilogue %d", a->epi); return P0_EINVAL; }
  if (!a->w || !a->x || !a->y) { set_error("gemvM: missing w, x or y buffer"); return P0_EINVAL; }
  if (a->pro == P0_PRO_RMS && (!a->norm || !a->stat)) { set_error("gemvM: rms needs norm and stat buffers"); return P0_EINVAL; }
  if (a->pro == P0_PRO_PLEG && !a->ev) { set_error("gemvM: pleg needs an ev buffer"); return P0_EINVAL; }
  if (a->epi == P0_EPI_SOFTCAP && !a->mx) { set_error("gemvM: softcap needs an mx buffer"); return P0_EINVAL; }
  if (int r = require_open("gemvM")) return r;

  GemvP p{};
  p.w = (const uint8_t*)a->w + a->w_off;
  p.wG = a->w_cols / 32;
  p.N = (int)N; p.K = (int)K; p.kPer = (int)kPer; p.nsplit = (int)nsplit; p.NT = (int)(N / 64);
  p.pro = a->pro; p.epi = a->epi;
  p.X = a->x; p.ldx = a->x_ldx ? a->x_ldx : K; p.rowB = a->x_rowB;
  p.ST = a->stat; p.statOff = a->stat_off; p.statLd = a->stat_ld ? a->stat_ld : 2;
  p.NW = a->norm; p.nOff = a->norm_off;
  p.nsrc = a->src_n ? (int)a->src_n : 1; p.ldp = a->src_ld;
  p.EV = a->ev; p.evOff = a->ev_off; p.evLd = a->ev_ld;
  p.ldm = a->y_ldm ? a->y_ldm : N;
  p.Y = a->y; p.ldy = a->y_ldy ? a->y_ldy : M * p.ldm;
  p.MX = a->mx; p.cap = a->cap != 0.0f ? a->cap : 30.0f;
  if (int r = launch(p, (int)M, "gemvM")) return r;
  if (nsplit_out) *nsplit_out = (int32_t)nsplit;
  return P0_OK;
}

// tuning knobs (benchmark sweeps): 0 = target waves before K is split, 1 = tile count from which a wave takes two
// tiles, 2 = fewest groups per wave, 3 = most waves per tile slot in a workgroup. Returns the previous value.
extern "C" int p0_gemv_tune(int knob, int value) {
  int* t = knob == 0 ? &g_target_waves : knob == 1 ? &g_two_tiles_min_nt : knob == 2 ? &g_min_gpw
         : knob == 3 ? &g_max_kw : nullptr;
  if (!t) return -1;
  const int old = *t;
  if (value > 0) *t = knob == 3 && value > 8 ? 8 : value;
  return old;
}
