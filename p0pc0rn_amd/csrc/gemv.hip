// gemv.hip - host side of the q4g32a.t64 GEMV (M = 1), GEMV-M (M <= 16) and GEMV chains: validation, planning,
// launch and the C entry points.
//
// Replaces the WebGPU dispatch of gemv (engine/llm/lops.js:108-141) and gemvM (engine/llm/lops_spec.js:159-191) with
// the same arguments, the same split semantics (nsplit partial rows Y[split * ldy + m * ldm + n]) and the same errors.
// The kernels and their mapping onto MI355X are described in gemv_kernels.hpp.
#include "chain_aux.hpp"

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace p0 {
// ------------------------------------------------------------------------------------------------ launch
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
static int g_max_kw = 16;               // most waves that share one tile slot's K-slice inside a workgroup
static int g_mf_min_m = 2;              // fewest x rows a standalone GEMV-M runs on MFMA (17: never)
static int g_q8_slices = 0;             // q8g64s.t64 GEMV at M = 1: K-slices per split across workgroups (0: planned)
static int g_pipe_mf_min_m = 3;         // fewest x rows a pipelined chain does its slot arithmetic on MFMA (6: never)

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
  // K shares per slot and split: enough waves for the chip, but at least g_min_gpw groups each. A geglu slot streams
  // the gate and the up tile and counts twice at M = 1 and from M = 12 on; at M = 2-8 the extra K-slices' partials cost
  // more than the parallelism gains (measured on the E2B gate_up: 14-20 us per launch against 20-26)
  const int work = pl.mode == 2 && (M == 1 || M >= 12) ? 2 * g_target_waves : g_target_waves;
  int kws = (work + slots * nsplit - 1) / (slots * nsplit);
  // 12-16 x rows over several kPer splits (the E2B down projection): the splits already give the chip its workgroups,
  // and K-slices would multiply the partials of every row; two waves per slot, K in one workgroup per split
  // (measured at M = 12 / 16: 25-26 us per launch against 31-32)
  if (M >= 12 && nsplit >= 4 && kws > 2) kws = 2;
  const int kws_max = Gs / g_min_gpw > 1 ? Gs / g_min_gpw : 1;
  if (kws > kws_max) kws = kws_max;
  if (kws < 1) kws = 1;
  const bool mf = M >= 2 && M >= g_mf_min_m;   // the MFMA kernel (512 threads)
  const int max_kw = M <= 2 && !mf ? g_max_kw : (g_max_kw < 8 ? g_max_kw : 8);   // the kernel's launch bound
  pl.kw = kws < max_kw ? kws : max_kw;
  // one tile per slot whose K is split across workgroups anyway: at most 8 waves per slot, so that twice the
  // workgroups (each with half the records to issue and dot) share it
  if (pl.mode == 0 && kws > pl.kw && pl.kw > 8) pl.kw = 8;
  pl.tgw = pl.kw >= 4 ? 1 : 4 / pl.kw;                 // 4 waves per workgroup unless kw is larger
  if (pl.tgw > slots) pl.tgw = slots;
  pl.waves = pl.tgw * pl.kw;
  int nks = (kws + pl.kw - 1) / pl.kw;
  int gps = (Gs + nks - 1) / nks;
  // LDS: x' and its group sums for the slice, plus the reduction rows. M >= 2 runs on MFMA (gemv_item): its group
  // sums take 16 entries per group (a 16-row A operand) when M < 16
  const size_t red = (size_t)pl.waves * T * 64 * sizeof(float);
  const int XS = mf && M < 16 ? 16 : M;
  int maxGps = (int)((48 * 1024 - red) / ((size_t)M * 32 * sizeof(float) + (size_t)XS * sizeof(float)));
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
  pl.lds = (size_t)M * gps * 32 * sizeof(float) + (size_t)XS * gps * sizeof(float) + red;
  return pl;
}

// ---- chain building: between p0_chain_begin and p0_chain_end, gemv / gemvM calls append planned ops instead of
// launching. A chain runs with W waves per workgroup (16 for M = 1, else 8) and G = CUs x (1 or 2) workgroups.
static chain_kernel_t pick_chain(int M, int W) {
  switch (M) {
    case 1: return pick_chain_m<1>(W);
    case 2: return pick_chain_m<2>(W);
    case 3: return pick_chain_m<3>(W);
    case 4: return pick_chain_m<4>(W);
    case 5: return pick_chain_m<5>(W);
    case 6: return pick_chain_m<6>(W);
    case 7: return pick_chain_m<7>(W);
    case 8: return pick_chain_m<8>(W);
    case 9: return pick_chain_m<9>(W);
    case 10: return pick_chain_m<10>(W);
    case 11: return pick_chain_m<11>(W);
    case 12: return pick_chain_m<12>(W);
    case 13: return pick_chain_m<13>(W);
    case 14: return pick_chain_m<14>(W);
    case 15: return pick_chain_m<15>(W);
    case 16: return pick_chain_m<16>(W);
  }
  return nullptr;
}

static int g_chain_waves = 16;          // waves per chain workgroup for M = 1 (8 or 16)
static int g_chain_split_gpw = 16;      // a wave share above this many groups splits K across workgroups
static int g_chain_spin = 1 << 22;      // polls before a chain wait gives up (about 0.3 s)
static int g_chain_force_give_up = 0;   // tests: every wait gives up at once
static int g_chain_stage = 1;           // staged ops (weights copied to LDS before the wait) where they fit
static int g_chain_mbx = 1;             // pipelined chains: mailbox hand-offs where an op reads the previous op's output
static int g_chain_stg = 1;             // pipelined M > 1 chains: x' staged by the previous op where possible
static int g_chain_pipe_m = 1;          // gemvM chains (M <= 5) on the pipelined kernel (1) or the general one (0)
static int g_pipe_loaders = 2;          // pipelined chain: loader waves that stream
static int g_pipe_depth = 2;            // pipelined M = 1 chain: slots in flight per loader wave
static int g_pipe_depth_m = 1;          // pipelined M > 1 chain: the same (measured: 1 is 1-2.5% faster at M = 2-5)
static int g_chain_wide = 1;            // chains of 6-16 rows in one pass of the wide kernel (1) or as row groups (0)
static int g_wide_depth = 2;            // wide chain: slots in flight per loader wave (measured: 2 is 2% faster at M >= 12)
static int g_wide_predict = 1;          // wide chain: a wave whose x' overflowed the 2^8 staging takes fp32 x' next op
static constexpr size_t kChainLds = 64 * 1024;
static constexpr size_t kChainLdsMax = 160 * 1024 - 256;   // gfx950: LDS per CU, less the kernel's static LDS

struct ChainBuild {
  int M = 0, W = 0, G = 0;
  bool q8 = false;     // holds q8g64s.t64 ops (the pipelined kernel only)
  bool aux = false;    // holds copy / argmax / rowstats / normadd ops (the pipelined kernel only)
  size_t lds = 0;
  std::vector<GemvP> ops;
  std::string error;   // the first failed append (reported again by p0_chain_end)
};
struct ChainExec {
  int pipe_cfg[3];   // pipelined chains: loader waves, slots in flight per loader (0: another kernel), wide: predict
  GemvP* ops;
  unsigned* st;
  size_t st_words;
  int n_ops, M, W, grid;
  size_t lds;
  chain_kernel_t kernel;
  int mailboxes;     // ops that take their input from a mailbox
  int staged;        // ops that take their x' staged by the previous op
  Keep dev;          // owns ops and st (a recording that captured a run of the chain holds it too)
  // a gemvM chain of more rows than the pipelined kernel holds, run as pipelined passes over row groups (one chain
  // each, launched back to back; see build_row_groups); empty for a chain of one launch
  std::vector<ChainExec*> parts;
};
static ChainBuild* g_chain = nullptr;
bool building_chain() { return g_chain != nullptr; }
static std::map<unsigned*, size_t> g_state_bytes;   // sizes of the uncached state blocks

// Chain state (completion flags and the run tag) lives in uncached device memory: a flag store and the polls of
// other workgroups then go straight to memory, which halves the hand-off latency against cached device memory
// (measured on MI355X, cross-XCD round trip 0.69 us vs 1.14 us). Uncached memory that a kernel has read is never
// freed while the process runs (allocations made after such a free have been seen holding wrong values), so freed
// chains return their state blocks to this pool, which later chains reuse.
static std::vector<std::pair<unsigned*, size_t>> g_state_pool;   // free blocks (pointer, bytes)
static hipError_t state_alloc(unsigned** out, size_t bytes) {
  size_t best = (size_t)-1;
  for (size_t i = 0; i < g_state_pool.size(); ++i)
    if (g_state_pool[i].second >= bytes && (best == (size_t)-1 || g_state_pool[i].second < g_state_pool[best].second))
      best = i;
  if (best != (size_t)-1) {
    *out = g_state_pool[best].first;
    g_state_pool.erase(g_state_pool.begin() + (long)best);
    return hipSuccess;
  }
  bytes = (bytes + 65535) & ~(size_t)65535;
  hipError_t e = hipExtMallocWithFlags((void**)out, bytes, hipDeviceMallocUncached);
  if (e == hipSuccess) g_state_bytes[*out] = bytes;
  return e;
}
static void state_free(unsigned* p) {
  if (p) g_state_pool.emplace_back(p, g_state_bytes[p]);
}

// Device-coherent accesses of the ops of a chain (GemvP::coh). Op i reads its inputs with coherent loads when an
// earlier op writes into them, and writes its outputs with coherent stores when a later op reads them or another op
// writes the same lines (plain stores of two ops to one line from two XCDs would sit in two L2 caches, written back
// in no set order). Everything else takes plain, L2-cached accesses. Spans are compared as whole 128-byte lines.
struct Span { uintptr_t a, b; };
static Span span_of(const float* base, int64_t lo, int64_t hi) {   // floats [lo, hi) of base, widened to lines
  const uintptr_t a = (uintptr_t)(base + lo), b = (uintptr_t)(base + hi);
  return {a & ~(uintptr_t)127, (b + 127) & ~(uintptr_t)127};
}
static void op_spans(const GemvP& p, int M, std::vector<Span>& rd, std::vector<Span>& wr) {
  const int64_t m1 = M - 1;
  switch (p.kind) {   // ops that are not GEMVs: what they read first, then the rest (chain_aux.hpp)
    case kOpCopy:
      rd.push_back(span_of(p.asrc, 0, p.an));
      wr.push_back(span_of(p.adst, 0, p.an));
      return;
    case kOpArgmax:
      rd.push_back(span_of(p.asrc, 0, p.arows * p.acols * 2));
      wr.push_back(span_of(p.adst, 0, p.arows * 2));
      return;
    case kOpRowstats:
      rd.push_back(span_of(p.asrc, p.ac0, (p.arows - 1) * p.ald + p.ac0 + p.acols));
      wr.push_back(span_of(p.adst, p.astOff * 2, (p.astOff + p.arows) * 2));
      return;
    case kOpNormadd:
      rd.push_back(span_of(p.asrc, 0, (p.an - 1) * p.aldp + p.arows * p.acols));
      if (p.amode == 0) rd.push_back(span_of(p.aw, p.awOff, p.awOff + p.acols));
      rd.push_back(span_of(p.adst, 0, p.arows * p.acols));
      wr.push_back(span_of(p.adst, 0, p.arows * p.acols));
      wr.push_back(span_of(p.ast, p.astOff, p.astOff + p.arows));
      return;
  }
  if (p.pro == P0_PRO_RAW || p.pro == P0_PRO_RMS) rd.push_back(span_of(p.X, p.rowB, m1 * p.ldx + p.rowB + p.K));
  else rd.push_back(span_of(p.X, 0, (int64_t)(p.nsrc - 1) * p.ldp + m1 * p.ldx + p.K));   // X[j ldp + m ldx + k]
  if (p.pro == P0_PRO_RMS) {
    rd.push_back(span_of(p.ST, p.statOff, p.statOff + m1 * p.statLd + 1));
    rd.push_back(span_of(p.NW, p.nOff, p.nOff + p.K));
  }
  if (p.pro == P0_PRO_PLEG) rd.push_back(span_of(p.EV, p.evOff, p.evOff + m1 * p.evLd + p.K));
  if (p.epi == P0_EPI_STORE) wr.push_back(span_of(p.Y, 0, (int64_t)(p.nsplit - 1) * p.ldy + m1 * p.ldm + p.N));
  else wr.push_back(span_of(p.Y, 0, m1 * p.ldm + p.N));
  if (p.epi == P0_EPI_SOFTCAP) wr.push_back(span_of(p.MX, 0, (int64_t)M * p.NT * 2));
}
static void mark_coherence(std::vector<GemvP>& ops, int M) {
  const size_t n = ops.size();
  std::vector<std::vector<Span>> rd(n), wr(n);
  for (size_t i = 0; i < n; ++i) op_spans(ops[i], M, rd[i], wr[i]);
  auto meet = [](const std::vector<Span>& x, const std::vector<Span>& y) {
    for (const Span& a : x)
      for (const Span& b : y)
        if (a.a < b.b && b.a < a.b) return true;
    return false;
  };
  for (size_t i = 0; i < n; ++i) {
    int c = 0;
    for (size_t j = 0; j < n; ++j) {
      if (j < i && meet(rd[i], wr[j])) c |= 1;
      if (j > i && meet(wr[i], rd[j])) c |= 2;
      if (j != i && meet(wr[i], wr[j])) c |= 2;
    }
    ops[i].coh = c;
  }
}

// Mailbox hand-offs of a pipelined M = 1 chain. Op i takes its x from op i - 1's mailbox (one 64-bit word per output
// element of op i - 1, at the element's float offset from op i - 1's Y: run tag << 32 | the value's bits) when
//  * op i's prologue is raw or rms and its x, [rowB, rowB + K) of X, lies inside one split of op i - 1's store or geglu
//    output (op i - 1's element f = split * ldy + n, n < N);
//  * op i reads nothing else that an op of the chain writes (rms: the rstd slot and the norm weights), and op i and op
//    i - 1 write nothing in common.
// The mailbox words op i reads say that exactly those elements of op i - 1 are written (read-after-write), and nothing
// about the other workgroups: a workgroup that produced none of them may still be in an earlier op, reading or writing
// a buffer that op i writes. Every workgroup publishes its completion flag of every op after its own stores of that
// op, so op j's flags from all workgroups mean every op up to j is complete everywhere. An op whose outputs overlap
// what an op before i - 1 reads or writes (GemvP::wback 2) therefore waits for op i - 2's flags before it writes them
// (by then normally long set; the flags are loaded at the op's start, so the check costs no round trip of its own), and
// one whose outputs overlap what op i - 1 reads (wback 1) for op i - 1's. An op that waits for flags at its start (no
// mailbox) sees every earlier op complete in the flags of op i - 1.
static size_t plan_mailboxes(std::vector<GemvP>& ops, std::vector<int64_t>& mb_out, std::vector<int64_t>& mb_in) {
  const size_t n = ops.size();
  mb_out.assign(n, -1);
  mb_in.assign(n, -1);
  std::vector<std::vector<Span>> rd(n), wr(n);
  for (size_t i = 0; i < n; ++i) op_spans(ops[i], 1, rd[i], wr[i]);
  auto meet = [](const std::vector<Span>& x, const std::vector<Span>& y) {
    for (const Span& a : x)
      for (const Span& b : y)
        if (a.a < b.b && b.a < a.b) return true;
    return false;
  };
  size_t words = 0;
  for (size_t i = 1; i < n; ++i) {
    const GemvP& pr = ops[i - 1];
    GemvP& c = ops[i];
    if (pr.kind != kOpGemv || c.kind != kOpGemv) continue;
    if (pr.epi != P0_EPI_STORE && pr.epi != P0_EPI_GEGLU) continue;
    if (c.pro != P0_PRO_RAW && c.pro != P0_PRO_RMS) continue;
    const intptr_t d = (intptr_t)(const void*)(c.X + c.rowB) - (intptr_t)(const void*)pr.Y;
    if (d < 0 || d % 4) continue;
    const int64_t f = d / 4, ld = pr.nsplit > 1 ? pr.ldy : (int64_t)pr.N;
    const int64_t sp = f / ld, r = f % ld;
    if (sp >= pr.nsplit || r + c.K > pr.N) continue;
    if (c.pro == P0_PRO_RMS) {   // the rstd slot and the norm weights: inputs of the chain, not written by its ops
      std::vector<Span> extra{rd[i].begin() + 1, rd[i].end()};
      bool written = false;
      for (size_t j = 0; j < n && !written; ++j) written = meet(extra, wr[j]);
      if (written) continue;
    }
    if (meet(wr[i], wr[i - 1])) continue;
    if (mb_out[i - 1] < 0) {
      mb_out[i - 1] = (int64_t)words;
      words += 2 * (size_t)((pr.nsplit - 1) * ld + pr.N);
    }
    mb_in[i] = mb_out[i - 1] + 2 * f;
    if (meet(wr[i], rd[i - 1])) c.wback = 1;
    for (size_t j = 0; j + 1 < i && !c.wback; ++j)
      if (meet(wr[i], rd[j]) || meet(wr[i], wr[j])) c.wback = 2;
  }
  return words;
}

// The waits of a pipelined chain's copy / argmax / rowstats / normadd ops (GemvP::abefore). Their workers wait for the
// completion flags of the latest earlier op that writes what the op reads or touches what it writes (on 128-byte
// lines), not for op i - 1's: an op with no such predecessor (a copy of a chain input into a slot no earlier op
// touches) starts at once. An op that workgroup 0 runs alone right after another op that workgroup 0 ran alone needs
// nothing of that op (the workgroup ran it) and nothing the earlier op's own wait covered already (the argmax's result
// copy after the argmax). Every other op still sees every earlier op complete before it writes (flags, or GemvP::wback).
static void plan_aux_waits(std::vector<GemvP>& ops, int M) {
  const size_t n = ops.size();
  std::vector<std::vector<Span>> rd(n), wr(n);
  for (size_t i = 0; i < n; ++i) op_spans(ops[i], M, rd[i], wr[i]);
  auto meet = [](const std::vector<Span>& x, const std::vector<Span>& y) {
    for (const Span& a : x)
      for (const Span& b : y)
        if (a.a < b.b && b.a < a.b) return true;
    return false;
  };
  auto hazard = [&](size_t i, size_t j) { return meet(rd[i], wr[j]) || meet(wr[i], rd[j]) || meet(wr[i], wr[j]); };
  auto last_hazard = [&](size_t i, size_t below) {   // the latest op j < below that op i conflicts with, or -1
    for (size_t j = below; j-- > 0;)
      if (hazard(i, j)) return (int)j;
    return -1;
  };
  auto alone = [](const GemvP& p) {   // run by workgroup 0 alone (aux_worker)
    return p.kind != kOpGemv && (p.kind == kOpCopy ? p.an <= kAuxCopyWords : p.arows <= 1);
  };
  std::vector<int> covered(n, -1);   // aux op i: every op up to covered[i] was complete everywhere when i ran
  for (size_t i = 0; i < n; ++i) {
    GemvP& p = ops[i];
    if (p.kind == kOpGemv) continue;
    int J = last_hazard(i, i);
    const bool after_alone = i > 0 && alone(ops[i - 1]) && alone(p);
    if (after_alone && J == (int)i - 1) {
      const int J2 = last_hazard(i, i - 1);
      J = J2 <= covered[i - 1] ? -1 : J2;
    }
    p.abefore = J;
    covered[i] = std::max(J, after_alone ? covered[i - 1] : -1);
  }
}

// Producer-staged x' of a pipelined M > 1 chain on the matrix cores. Op i takes its x' as op i - 1 wrote it (GemvP::stgIn,
// laid out by stg_half_at) when op i's prologue is raw or rms, its arithmetic runs on the matrix cores, its x lies inside
// one split of op i - 1's store or geglu output at an offset that is a multiple of 32 rows, with the rows of x at op i -
// 1's row stride, and nothing in the chain writes its rms inputs (rstd slots, norm weights); op i - 1 must be a spread
// share (its epilogue gives each thread one output row). The staged words are written before op i - 1's completion
// flags, which op i waits for as before, and the values are those stage_rows computes from op i - 1's outputs, bit for
// bit. Returns the words to add to the chain state; stg_out / stg_in get each op's offset in them (-1: none).
static size_t plan_staging(std::vector<GemvP>& ops, int M, std::vector<int64_t>& stg_out, std::vector<int64_t>& stg_in) {
  const size_t n = ops.size();
  stg_out.assign(n, -1);
  stg_in.assign(n, -1);
  std::vector<std::vector<Span>> rd(n), wr(n);
  for (size_t i = 0; i < n; ++i) op_spans(ops[i], M, rd[i], wr[i]);
  auto meet = [](const std::vector<Span>& x, const std::vector<Span>& y) {
    for (const Span& a : x)
      for (const Span& b : y)
        if (a.a < b.b && b.a < a.b) return true;
    return false;
  };
  size_t words = 0;
  for (size_t i = 1; i < n; ++i) {
    GemvP& pr = ops[i - 1];
    const GemvP& c = ops[i];
    if (pr.kind != kOpGemv || c.kind != kOpGemv) continue;
    if (!c.mf || c.enc != P0_ENC_Q4G32A_T64 || !pr.sngp) continue;
    if (pr.epi != P0_EPI_STORE && pr.epi != P0_EPI_GEGLU) continue;
    if (c.pro != P0_PRO_RAW && c.pro != P0_PRO_RMS) continue;
    const intptr_t d = (intptr_t)(const void*)(c.X + c.rowB) - (intptr_t)(const void*)pr.Y;
    if (d < 0 || d % 4) continue;
    const int64_t f = d / 4, ld = pr.nsplit > 1 ? pr.ldy : (int64_t)pr.N;
    const int64_t sp = f / ld, r = f % ld;
    if (sp >= pr.nsplit || r + c.K > pr.N || r % 32 || (M > 1 && c.ldx != pr.ldm)) continue;
    if (c.pro == P0_PRO_RMS) {
      std::vector<Span> extra{rd[i].begin() + 1, rd[i].end()};
      bool written = false;
      for (size_t j = 0; j < n && !written; ++j) written = meet(extra, wr[j]);
      if (written) continue;
    }
    stg_out[i - 1] = stg_in[i] = (int64_t)words;
    words += (size_t)((stg_words(M, c.K) + 63) & ~(int64_t)63);
    pr.stgR0 = r;
    pr.stgK = c.K;
    pr.stgSp = (int)sp;
    pr.stgPro = c.pro;
    pr.stgST = c.ST; pr.stgStatOff = c.statOff; pr.stgStatLd = c.statLd;
    pr.stgNW = c.NW; pr.stgNOff = c.nOff;
  }
  return words;
}

// plan of one op inside a chain: all W waves of a workgroup busy (tgw = W / kw), one K-slice per split unless the op
// leaves half the grid idle AND a wave's share would exceed g_chain_split_gpw groups
static Plan plan_chain(int M, int NT, int epi, int nsplit, int kPer, int W, int G) {
  Plan pl{};
  pl.mode = epi == P0_EPI_GEGLU ? 2 : (NT >= g_two_tiles_min_nt ? 1 : 0);
  const int T = pl.mode == 0 ? 1 : 2;
  const int slots = pl.mode == 1 ? (NT + 1) / 2 : NT;
  pl.rowsTot = (epi == P0_EPI_GEGLU ? 2 : 1) * NT * 64;
  const int Gs = kPer / 32;
  int kws = (G * W + slots * nsplit - 1) / (slots * nsplit);
  const int kws_max = Gs / g_min_gpw > 1 ? Gs / g_min_gpw : 1;
  if (kws > kws_max) kws = kws_max;
  int kw = 1;
  while (kw * 2 <= kws && kw * 2 <= W) kw *= 2;
  pl.kw = kw;
  pl.tgw = W / kw;
  pl.waves = W;
  pl.ntb = (slots + pl.tgw - 1) / pl.tgw;
  int nks = 1;
  auto gpw = [&](int n) { return ((Gs + n - 1) / n + kw - 1) / kw; };
  while (gpw(nks) > g_chain_split_gpw && pl.ntb * nsplit * nks * 2 <= G) nks *= 2;
  const size_t red = (size_t)W * T * 64 * sizeof(float);
  const int maxGps = (int)((kChainLds - red) / ((size_t)M * 33 * sizeof(float)));
  int gps = (Gs + nks - 1) / nks;
  if (gps > maxGps) gps = maxGps;
  pl.gps = gps;
  pl.nks = (Gs + gps - 1) / gps;
  pl.lds = (size_t)M * gps * 33 * sizeof(float) + red;
  return pl;
}

// Staged plan of a chain op (mode 3, staged_op in gemv_kernels.hpp) on G workgroups of W waves: units of 16 rows (64
// for a softcap, whose tile maximum needs a whole tile; a geglu unit also holds the up rows) x one split, dealt to
// workgroup positions from `cur` on. Returns the LDS bytes the op needs, or 0 (the op stays a streamed op) when a
// workgroup's share does not fit the LDS, the weights are not 16-byte aligned (LDS-DMA loads), or a workgroup would
// get units of two splits.
static size_t plan_staged(GemvP& p, int M, int W, int G, int& cur) {
  if ((uintptr_t)p.w & 15) return 0;
  const int nrb = p.epi == P0_EPI_SOFTCAP ? 4 : 1, parts = p.epi == P0_EPI_GEGLU ? 2 : 1;
  const int64_t U = (int64_t)(p.N / (kStageRows * nrb)) * p.nsplit;
  if (U > G && G % p.nsplit) return 0;
  const int numax = (int)((U + G - 1) / G);
  const int ngp = (p.kPer / 32 + 15) / 16 * 16;
  const int64_t nrp = (int64_t)numax * nrb * parts;
  const size_t xs = (size_t)M * ngp * 33;                      // floats: x' and its group sums
  const size_t red = (size_t)nrp * M * W * 16;                 // floats: the per-wave row sums
  const size_t woff = ((xs + red) * sizeof(float) + 1023) & ~(size_t)1023;
  const size_t need = woff + (size_t)nrp * ngp * 320;
  if (need > kChainLdsMax) return 0;
  p.mode = 3;
  p.su = (int)U;
  p.scur = cur;
  p.snrb = nrb;
  p.sngp = ngp;
  p.sred = (int)xs;
  p.swoff = (int)woff;
  cur = (int)((cur + U) % G);
  return need;
}

// Plan of an M = 1 chain for the pipelined kernel (chain_pipe.hip) on G workgroups: every op's rows are dealt as
// units of 16 rows (64 for a softcap, a geglu unit with its up rows) x one split to workgroup positions, continuing
// where the previous op stopped so each workgroup streams about the same bytes over a step. A share of at most a
// ring's worth of slots (and few enough rows) is computed by all compute waves together, a larger one by one wave per
// unit. Returns false (the chain then runs on q4_gemv_chain_kernel) when the weights are not 16-byte aligned
// (LDS-DMA loads), a workgroup would get units of two splits, or (M > 1) a split exceeds 2048 k.
static bool plan_pipe(std::vector<GemvP>& ops, int G, int M) {
  int cur = 0;
  for (GemvP& p : ops) {
    if (p.kind != kOpGemv) {   // no units: every workgroup's share is empty
      p.su = 0;
      p.scur = cur;
      continue;
    }
    if ((uintptr_t)p.w & 15) return false;
    if (M > 1 && p.kPer > 2048) return false;
    const int nrb = p.epi == P0_EPI_SOFTCAP ? 4 : 1, parts = p.epi == P0_EPI_GEGLU ? 2 : 1;
    const int64_t U = (int64_t)(p.N / (kStageRows * nrb)) * p.nsplit;
    if (U > G && G % p.nsplit) return false;
    const int64_t numax = (U + G - 1) / G;
    const int nh = p.enc == P0_ENC_Q8G64S_T64 ? (p.kPer / 64 + 7) / 8 : (p.kPer / 32 + 31) / 32;   // slots per part
    const int64_t nrp = numax * nrb * parts;
    // (a spread share's epilogue gives each of the 512 compute threads one (row, x row) pair)
    const bool spread = nrp * nh <= pipe_ring_slots(M) && nrp <= pipe_spread_parts(M) && numax * nrb * kStageRows * M <= 512;
    p.su = (int)U;
    p.scur = cur;
    p.snrb = nrb;
    p.sngp = spread ? 1 : 0;
    cur = (int)((cur + U) % G);
  }
  return true;
}

// Plan of a chain of 6 - 16 rows for the wide pipelined kernel (chain_wide.hip) on G workgroups: the pipelined
// kernel's units and positions, every share computed by all compute waves (in rounds of at most 4 16-row parts).
// Returns false (row-group passes, or the general kernel, take the chain) when an op is q8, has a prologue other than
// raw or rms, a split of more than 2048 k, weights not 16-byte aligned (LDS-DMA loads), or a workgroup would get units
// of two splits.
static bool plan_wide(std::vector<GemvP>& ops, int G) {
  int cur = 0;
  for (GemvP& p : ops) {
    if (p.kind != kOpGemv) {
      p.su = 0;
      p.scur = cur;
      continue;
    }
    if ((uintptr_t)p.w & 15) return false;
    if (p.enc != P0_ENC_Q4G32A_T64 || p.kPer > 2048 || (p.pro != P0_PRO_RAW && p.pro != P0_PRO_RMS)) return false;
    const int nrb = p.epi == P0_EPI_SOFTCAP ? 4 : 1;
    const int64_t U = (int64_t)(p.N / (kStageRows * nrb)) * p.nsplit;
    if (U > G && G % p.nsplit) return false;
    p.su = (int)U;
    p.scur = cur;
    p.snrb = nrb;
    p.sngp = 1;
    p.mf = 1;
    cur = (int)((cur + U) % G);
  }
  return true;
}

// the q8 kernels' LDS allowance, set once at p0_open (never lazily, e.g. while the stream is being captured)
int gemv_init() {
  for (int M : {1, 2})
    P0_HIP(hipFuncSetAttribute((const void*)q8_kernel(M), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)q8_lds_bytes(16)), "p0_open: gemv");
  return P0_OK;
}

// q8g64s.t64: one workgroup per (64-row tile, split), gemv_q8.hip
static int launch_q8(GemvP& p, int M, const char* op) {
  // q8_gemv1_kernel: 16 waves per (tile, split), for splits of 1024-3072 k (16-48 groups; a split of 4 groups, the
  // E2B pleg projection's 256 k, runs faster on the 4-wave kernel: 3.9 against 4.9 us)
  if (M == 1 && p.kPer >= 1024 && p.kPer <= 3072) {
    // K-slices across workgroups (p.nks) when the tiles and splits leave most CUs idle: up to ~192 workgroups, at
    // least 8 groups (512 k) a slice (measured at the E2B 8-bit shapes: 6.2-9.3 us per launch against 6.9-10.9 with
    // one workgroup per split; p0_gemv_tune knob 5 sets the count)
    const int gsplit = p.kPer / 64;
    const int wgs = p.NT * p.nsplit;
    int nks = g_q8_slices > 0 ? g_q8_slices : std::min(std::max(gsplit / 8, 1), (192 + wgs - 1) / wgs);
    if (nks > gsplit) nks = gsplit;
    p.gps = (gsplit + nks - 1) / nks;
    p.nks = (gsplit + p.gps - 1) / p.gps;   // every slice holds at least one group
    p.rowsTot = (p.epi == P0_EPI_GEGLU ? 2 : 1) * p.NT * 64;
    p.part = ctx().part;
    p.cnt = ctx().counters;
    if (p.nks > 1 && ((size_t)p.nsplit * p.nks * p.rowsTot > ctx().part_floats ||
                      (size_t)p.nsplit * p.NT > ctx().n_counters)) {
      p.nks = 1;
      p.gps = gsplit;
    }
    hipLaunchKernelGGL(q8_gemv1(p.epi == P0_EPI_GEGLU), dim3((unsigned)p.NT, (unsigned)(p.nsplit * p.nks)), dim3(1024),
                       q8_gemv1_lds_bytes(), ctx().cur, p);
    P0_LAUNCHED(op);
    return P0_OK;
  }
  q8_kernel_t k = q8_kernel(M);
  const size_t lds = q8_lds_bytes(M);
  hipLaunchKernelGGL(k, dim3((unsigned)p.NT, (unsigned)p.nsplit), dim3(256), lds, ctx().cur, p);
  P0_LAUNCHED(op);
  return P0_OK;
}

static int launch(GemvP& p, int M, const char* op) {
  ChainBuild* cb = g_chain;
  if (p.enc == P0_ENC_Q8G64S_T64 && !cb) return launch_q8(p, M, op);
  if (cb && cb->M == 0) {   // the chain's first GEMV fixes M and the workgroup shape
    cb->M = M;
    cb->W = M == 1 ? g_chain_waves : 8;
    cb->G = ctx().cu_count * (cb->W == 16 ? 1 : 2);
  }
  if (cb && M != cb->M) {
    set_error("%s: a chain holds ops of one M (chain M %d, this op %d)", op, cb->M, M);
    if (cb->error.empty()) cb->error = p0_last_error();
    return P0_EINVAL;
  }
  if (cb && p.enc == P0_ENC_Q8G64S_T64) {
    // q8g64s.t64 ops run only on the pipelined kernel (p0_chain_end refuses a chain that cannot take them)
    p.coh = 0;
    cb->ops.push_back(p);
    cb->q8 = true;
    return P0_OK;
  }
  const Plan pl = cb ? plan_chain(M, p.NT, p.epi, p.nsplit, p.kPer, cb->W, cb->G) : plan(M, p.NT, p.epi, p.nsplit, p.kPer);
  if (pl.nks > 1 && (size_t)p.nsplit * pl.nks * M * pl.rowsTot > ctx().part_floats) {
    set_error("%s: split-K partials exceed the workspace (M %d, N %d, K %d)", op, M, p.N, p.K);
    if (cb && cb->error.empty()) cb->error = p0_last_error();
    return P0_EINVAL;
  }
  if ((size_t)p.nsplit * pl.ntb > ctx().n_counters) {
    set_error("%s: too many tile blocks for the workspace counters", op);
    if (cb && cb->error.empty()) cb->error = p0_last_error();
    return P0_EINVAL;
  }
  p.gps = pl.gps;
  p.nks = pl.nks;
  p.kw = pl.kw;
  p.tgw = pl.tgw;
  p.ntb = pl.ntb;
  p.rowsTot = pl.rowsTot;
  p.mode = pl.mode;
  p.part = ctx().part;
  p.cnt = ctx().counters;
  p.coh = 0;   // chains: set for the whole chain by p0_chain_end
  p.mf = !cb && M >= 2 && M >= g_mf_min_m;   // must agree with plan()'s LDS layout
  if (cb) {
    cb->ops.push_back(p);
    if (pl.lds > cb->lds) cb->lds = pl.lds;
    return P0_OK;
  }
  gemv_kernel_t k = pick(M, pl.mode + (p.mf ? 3 : 0));
  dim3 grid((unsigned)pl.ntb, (unsigned)(p.nsplit * pl.nks));
  hipLaunchKernelGGL(k, grid, dim3(64 * pl.waves), pl.lds, ctx().cur, p);
  P0_LAUNCHED(op);
  return P0_OK;
}

// ---- ops that are not GEMVs, appended to the chain being built instead of launched (p0_copy, p0_argmax / p0_argmaxM,
// p0_rowstats, p0_normadd; chain_aux.hpp runs them). The callers have validated the arguments. Such an op has no units
// (su = 0), so no workgroup streams weights for it; only the pipelined kernel runs it (p0_chain_end refuses others).
static int add_aux(GemvP& p) {
  ChainBuild* cb = g_chain;
  p.nsplit = 1;   // share_of's arithmetic on an empty share
  p.kPer = p.K = 32;
  p.snrb = p.sngp = 1;
  p.enc = P0_ENC_Q4G32A_T64;
  cb->ops.push_back(p);
  cb->aux = true;
  return P0_OK;
}
int chain_add_copy(const void* src, void* dst, int64_t words) {
  GemvP p{};
  p.kind = kOpCopy;
  p.asrc = (const float*)src;
  p.adst = (float*)dst;
  p.an = words;
  return add_aux(p);
}
int chain_add_argmax(const float* mx, int64_t n, int64_t M, uint32_t* out) {
  GemvP p{};
  p.kind = kOpArgmax;
  p.asrc = mx;
  p.adst = (float*)out;
  p.acols = n;
  p.arows = M;
  return add_aux(p);
}
int chain_add_rowstats(const float* x, int64_t ld, int64_t c0, int64_t rows, int64_t cols, int mode, float eps,
                       float* st, int64_t st_off) {
  GemvP p{};
  p.kind = kOpRowstats;
  p.asrc = x;
  p.ald = ld;
  p.ac0 = c0;
  p.arows = rows;
  p.acols = cols;
  p.amode = mode;
  p.aeps = eps;
  p.adst = st;
  p.astOff = st_off;
  return add_aux(p);
}
int chain_add_normadd(const float* t, int64_t nsrc, int64_t ldp, const float* w, int64_t w_off, float* x, float* st,
                      int64_t st_off, int64_t D, int64_t M, float eps, float scale, int mode) {
  GemvP p{};
  p.kind = kOpNormadd;
  p.asrc = t;
  p.an = nsrc;
  p.aldp = ldp;
  p.aw = w;
  p.awOff = w_off;
  p.adst = x;
  p.ast = st;
  p.astOff = st_off;
  p.acols = D;
  p.arows = M;
  p.aeps = eps;
  p.ascale = scale;
  p.amode = mode;
  return add_aux(p);
}

// engine/llm/lops.js:113-114: q4g32a.t64 (groups of 32 k) and q8g64s.t64 (groups of 64 k)
static int check_enc(int32_t enc, const char* op) {
  if (enc == P0_ENC_Q4G32A_T64 || enc == P0_ENC_Q8G64S_T64) return P0_OK;
  set_error("%s: encoding %d", op, (int)enc);
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
  const int64_t G = a->w_enc == P0_ENC_Q8G64S_T64 ? 64 : 32;
  if (kPer <= 0 || kPer % G) { set_error("gemv: kPer must be a multiple of %lld", (long long)G); return P0_EINVAL; }
  const int64_t nsplit = (K + kPer - 1) / kPer;
  if (a->epi != P0_EPI_STORE && nsplit > 1) { set_error("gemv: %s needs one split", epi_name(a->epi)); return P0_EINVAL; }
  if (N % 64) { set_error("gemv: N %% 64"); return P0_EINVAL; }
  if (a->w_off % 4) { set_error("gemv: weight offset"); return P0_EINVAL; }
  // this build's additional guards (the reference would read undefined memory here)
  if (K <= 0 || K % G) { set_error("gemv: K must be a multiple of %lld", (long long)G); return P0_EINVAL; }
  if (N <= 0) { set_error("gemv: N must be positive"); return P0_EINVAL; }
  if (a->w_cols < K) { set_error("gemv: weight has %lld columns < K %lld", (long long)a->w_cols, (long long)K); return P0_EINVAL; }
  if (a->w_rows < (a->epi == P0_EPI_GEGLU ? 2 * N : N)) {   // a geglu reads the up rows at N .. 2N - 1
    set_error("gemv: weight has %lld rows < %s %lld", (long long)a->w_rows, a->epi == P0_EPI_GEGLU ? "2N" : "N",
              (long long)(a->epi == P0_EPI_GEGLU ? 2 * N : N));
    return P0_EINVAL;
  }
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
  p.wG = a->w_cols / G;
  p.enc = a->w_enc;
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
  p.mrows = 1;
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
  const int64_t G = a->w_enc == P0_ENC_Q8G64S_T64 ? 64 : 32;
  if (kPer <= 0 || kPer % G) { set_error("gemvM: kPer must be a multiple of %lld", (long long)G); return P0_EINVAL; }
  const int64_t nsplit = (K + kPer - 1) / kPer;
  if (a->epi != P0_EPI_STORE && nsplit > 1) { set_error("gemvM: %s needs one split", epi_name(a->epi)); return P0_EINVAL; }
  if (N % 64) { set_error("gemvM: N %% 64"); return P0_EINVAL; }
  if (a->w_off % 4) { set_error("gemvM: weight offset"); return P0_EINVAL; }
  if (K <= 0 || K % G) { set_error("gemvM: K must be a multiple of %lld", (long long)G); return P0_EINVAL; }
  if (N <= 0) { set_error("gemvM: N must be positive"); return P0_EINVAL; }
  if (a->w_cols < K) { set_error("gemvM: weight has %lld columns < K %lld", (long long)a->w_cols, (long long)K); return P0_EINVAL; }
  if (a->w_rows < (a->epi == P0_EPI_GEGLU ? 2 * N : N)) {
    set_error("gemvM: weight has %lld rows < %s %lld", (long long)a->w_rows, a->epi == P0_EPI_GEGLU ? "2N" : "N",
              (long long)(a->epi == P0_EPI_GEGLU ? 2 * N : N));
    return P0_EINVAL;
  }
  if (a->epi < P0_EPI_STORE || a->epi > P0_EPI_SOFTCAP) { set_error("gemvM: epilogue %d", a->epi); return P0_EINVAL; }
  if (!a->w || !a->x || !a->y) { set_error("gemvM: missing w, x or y buffer"); return P0_EINVAL; }
  if (a->pro == P0_PRO_RMS && (!a->norm || !a->stat)) { set_error("gemvM: rms needs norm and stat buffers"); return P0_EINVAL; }
  if (a->pro == P0_PRO_PLEG && !a->ev) { set_error("gemvM: pleg needs an ev buffer"); return P0_EINVAL; }
  if (a->epi == P0_EPI_SOFTCAP && !a->mx) { set_error("gemvM: softcap needs an mx buffer"); return P0_EINVAL; }
  if (int r = require_open("gemvM")) return r;

  GemvP p{};
  p.w = (const uint8_t*)a->w + a->w_off;
  p.wG = a->w_cols / G;
  p.enc = a->w_enc;
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
  p.mrows = (int)M;
  if (int r = launch(p, (int)M, "gemvM")) return r;
  if (nsplit_out) *nsplit_out = (int32_t)nsplit;
  return P0_OK;
}

// tuning knobs (benchmark sweeps): 0 = target waves before K is split, 1 = tile count from which a wave takes two
// tiles, 2 = fewest groups per wave, 3 = most waves per tile slot in a workgroup. Returns the previous value.
extern "C" int p0_gemv_tune(int knob, int value) {
  int* t = knob == 0 ? &g_target_waves : knob == 1 ? &g_two_tiles_min_nt : knob == 2 ? &g_min_gpw
         : knob == 3 ? &g_max_kw : knob == 4 ? &g_mf_min_m : knob == 5 ? &g_q8_slices : nullptr;
  if (!t) return -1;
  const int old = *t;
  if (value > 0) *t = knob == 3 && value > 16 ? 16 : value;
  else if (knob == 5 && value < 0) *t = 0;   // the planned slice count again
  return old;
}

// ---- chains (engine/llm/drunner.js:1-8, 83-101: a decode token's dispatches recorded once, submitted per token)
extern "C" int p0_chain_begin(void) {
  if (int r = require_open("p0_chain_begin")) return r;
  if (g_chain) { set_error("p0_chain_begin: a chain is already being built"); return P0_EINVAL; }
  g_chain = new ChainBuild();
  return P0_OK;
}

static int build_exec(ChainBuild* cb, bool pipe_only, ChainExec** out);

// The rows of a gemvM chain are independent: row m of an op reads row m of its x (its rstd slot, its pleg row) and
// writes row m of its outputs, so a chain of more rows than the pipelined kernel holds can run as pipelined passes
// over row groups, each pass the whole chain for its rows, one after another on the stream. That holds for the buffers
// as the caller laid them out only if no byte that one row group writes is read or written by another group: checked
// here on exact byte spans (rows of one buffer may share cache lines; the passes do not overlap in time), with the
// weights and norm weights, which every row reads, counted for every group. gs: the groups' first rows, then M.
struct RowSpan {
  uintptr_t a, b;
  int g;
  bool w;
};
static bool rows_independent(const std::vector<GemvP>& ops, const std::vector<int>& gs) {
  const int ng = (int)gs.size() - 1;
  std::vector<RowSpan> sp;
  auto add = [&](const void* base, int64_t lo, int64_t hi, int g, bool w) {   // bytes [lo, hi) of base
    sp.push_back({(uintptr_t)base + (uintptr_t)lo, (uintptr_t)base + (uintptr_t)hi, g, w});
  };
  const int64_t M = gs[ng];
  for (const GemvP& p : ops) {
    if (p.kind != kOpGemv) {   // row-wise only with one row per x row: argmax, rowstats, normadd over the chain's M
      if (p.kind == kOpCopy || p.arows != M) return false;
      for (int g = 0; g < ng; ++g) {
        if (p.kind == kOpNormadd && p.amode == 0) add(p.aw, p.awOff * 4, (p.awOff + p.acols) * 4, g, false);
        for (int64_t m = gs[g]; m < gs[g + 1]; ++m) {
          if (p.kind == kOpArgmax) {
            add(p.asrc, m * p.acols * 8, (m + 1) * p.acols * 8, g, false);
            add(p.adst, m * 8, (m + 1) * 8, g, true);
          } else if (p.kind == kOpRowstats) {
            add(p.asrc, (m * p.ald + p.ac0) * 4, (m * p.ald + p.ac0 + p.acols) * 4, g, false);
            add(p.adst, (p.astOff + m) * 8, (p.astOff + m + 1) * 8, g, true);
          } else {
            for (int64_t j = 0; j < p.an; ++j)
              add(p.asrc, (j * p.aldp + m * p.acols) * 4, (j * p.aldp + (m + 1) * p.acols) * 4, g, false);
            add(p.adst, m * p.acols * 4, (m + 1) * p.acols * 4, g, true);
            add(p.ast, (p.astOff + m) * 4, (p.astOff + m + 1) * 4, g, true);
          }
        }
      }
      continue;
    }
    const int64_t rows = p.epi == P0_EPI_GEGLU ? 2 * (int64_t)p.N : p.N;
    const int64_t wbytes = (rows + 63) / 64 * p.wG * 1280;
    for (int g = 0; g < ng; ++g) {
      add(p.w, 0, wbytes, g, false);
      if (p.pro == P0_PRO_RMS) add(p.NW, p.nOff * 4, (p.nOff + p.K) * 4, g, false);
      for (int64_t m = gs[g]; m < gs[g + 1]; ++m) {
        if (p.pro == P0_PRO_RAW || p.pro == P0_PRO_RMS) {
          add(p.X, (m * p.ldx + p.rowB) * 4, (m * p.ldx + p.rowB + p.K) * 4, g, false);
        } else {
          for (int64_t j = 0; j < p.nsrc; ++j) add(p.X, (j * p.ldp + m * p.ldx) * 4, (j * p.ldp + m * p.ldx + p.K) * 4, g, false);
        }
        if (p.pro == P0_PRO_RMS) add(p.ST, (p.statOff + m * p.statLd) * 4, (p.statOff + m * p.statLd + 1) * 4, g, false);
        if (p.pro == P0_PRO_PLEG) add(p.EV, (p.evOff + m * p.evLd) * 4, (p.evOff + m * p.evLd + p.K) * 4, g, false);
        const int64_t ns = p.epi == P0_EPI_STORE ? p.nsplit : 1;
        for (int64_t sp0 = 0; sp0 < ns; ++sp0) add(p.Y, (sp0 * p.ldy + m * p.ldm) * 4, (sp0 * p.ldy + m * p.ldm + p.N) * 4, g, true);
        if (p.epi == P0_EPI_SOFTCAP) add(p.MX, m * p.NT * 8, (m + 1) * p.NT * 8, g, true);
      }
    }
  }
  // in order of their first byte, a span meets an earlier one of another group iff it starts before that one ends
  std::sort(sp.begin(), sp.end(), [](const RowSpan& x, const RowSpan& y) { return x.a < y.a; });
  std::vector<uintptr_t> end_w(ng, 0), end_any(ng, 0);
  for (const RowSpan& x : sp) {
    for (int h = 0; h < ng; ++h)
      if (h != x.g && (end_w[h] > x.a || (x.w && end_any[h] > x.a))) return false;
    end_any[x.g] = std::max(end_any[x.g], x.b);
    if (x.w) end_w[x.g] = std::max(end_w[x.g], x.b);
  }
  return true;
}

// A chain of M > pipe_max_m() rows (at most 16) as ceil(M / pipe_max_m()) pipelined passes of near-equal row groups
// (8 = 4 + 4, 16 = 4 x 4): each group's ops are the chain's with their row bases moved to the group's first row. *out
// stays null (the general kernel takes the chain) when the rows are not independent or a group cannot be planned.
static int build_row_groups(const ChainBuild* cb, ChainExec** out) {
  *out = nullptr;
  const int M = cb->M, ng = (M + pipe_max_m() - 1) / pipe_max_m();
  std::vector<int> gs(ng + 1, 0);
  for (int g = 0; g < ng; ++g) gs[g + 1] = gs[g] + M / ng + (g < M % ng ? 1 : 0);
  if (!rows_independent(cb->ops, gs)) return P0_OK;
  std::vector<ChainExec*> parts;
  auto drop = [&]() {
    for (ChainExec* e : parts) delete e;
  };
  for (int g = 0; g < ng; ++g) {
    ChainBuild sub;
    sub.M = gs[g + 1] - gs[g];
    sub.W = cb->W;
    sub.G = cb->G;
    sub.lds = cb->lds;
    sub.aux = cb->aux;
    sub.q8 = cb->q8;   // the kernel instantiation that carries the q8 code
    const int64_t m0 = gs[g];
    for (GemvP p : cb->ops) {
      if (p.kind != kOpGemv) {   // argmax / rowstats / normadd over the chain's rows (rows_independent checked)
        if (p.kind == kOpArgmax) {
          p.asrc += m0 * p.acols * 2;
          p.adst += m0 * 2;
        } else if (p.kind == kOpRowstats) {
          p.asrc += m0 * p.ald;
          p.astOff += m0;
        } else {
          p.asrc += m0 * p.acols;
          p.adst += m0 * p.acols;
          p.astOff += m0;
        }
        p.arows = sub.M;
        sub.ops.push_back(p);
        continue;
      }
      p.X += m0 * p.ldx;
      if (p.pro == P0_PRO_RMS) p.statOff += m0 * p.statLd;
      if (p.pro == P0_PRO_PLEG) p.evOff += m0 * p.evLd;
      p.Y += m0 * p.ldm;
      if (p.epi == P0_EPI_SOFTCAP) p.MX += m0 * p.NT * 2;
      p.mrows = sub.M;
      sub.ops.push_back(p);
    }
    ChainExec* e = nullptr;
    if (int r = build_exec(&sub, true, &e)) {
      drop();
      return r;
    }
    if (!e) {
      drop();
      return P0_OK;
    }
    parts.push_back(e);
  }
  auto* ex = new ChainExec{};
  ex->n_ops = (int)cb->ops.size();
  ex->M = M;
  ex->W = parts[0]->W;
  ex->grid = parts[0]->grid;
  ex->lds = parts[0]->lds;
  for (ChainExec* e : parts) ex->staged += e->staged;
  ex->parts = parts;
  *out = ex;
  return P0_OK;
}

extern "C" int p0_chain_end(void** out) {
  ChainBuild* cb = g_chain;
  g_chain = nullptr;
  if (out) *out = nullptr;
  if (!cb) { set_error("p0_chain_end: no chain is being built"); return P0_EINVAL; }
  std::unique_ptr<ChainBuild> hold(cb);
  if (int r = require_open("p0_chain_end")) return r;
  if (!cb->error.empty()) { set_error("p0_chain_end: %s", cb->error.c_str()); return P0_EINVAL; }
  if (cb->ops.empty()) { set_error("p0_chain_end: the chain holds no ops"); return P0_EINVAL; }
  if (!out) { set_error("p0_chain_end: no output"); return P0_EINVAL; }
  if (cb->M == 0) {   // no GEMV (only copy / argmax / rowstats / normadd ops): the M = 1 kernel runs them
    cb->M = 1;
    cb->W = g_chain_waves;
    cb->G = ctx().cu_count * (cb->W == 16 ? 1 : 2);
  }
  ChainExec* ex = nullptr;
  if (cb->M > pipe_max_m()) {   // one pass of the wide kernel, else passes over row groups, else the general kernel
    if (int r = build_exec(cb, true, &ex)) return r;
    if (!ex && g_chain_stage && g_chain_pipe_m)
      if (int r = build_row_groups(cb, &ex)) return r;
  }
  if (!ex) {
    if (int r = build_exec(cb, false, &ex)) return r;
  }
  *out = ex;
  return P0_OK;
}

// One launch for the chain cb: the pipelined kernel where every op can be planned for it, else the general chain
// kernel; with pipe_only, *out stays null instead of taking the general kernel.
static int build_exec(ChainBuild* cb, bool pipe_only, ChainExec** out) {
  *out = nullptr;
  chain_kernel_t k = pick_chain(cb->M, cb->W);
  int per_cu = 0;
  P0_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k, 64 * cb->W, cb->lds), "p0_chain_end");
  if (per_cu < 1) { set_error("p0_chain_end: a chain workgroup does not fit a CU"); return P0_EINVAL; }
  int grid = ctx().cu_count * per_cu;
  if (grid > cb->G) grid = cb->G;   // the plans were made for G workgroups; never more than are resident
  if (grid > kChainMaxGrid) grid = kChainMaxGrid;
  size_t lds = cb->lds;
  if (g_chain_stage && cb->M != 1 && !pipe_only) {
    // staged ops are dealt over exactly `grid` workgroups, so the grid must stay resident with their LDS: plan, check
    // the occupancy, and plan again on a smaller grid if it shrank
    std::vector<GemvP> staged;
    for (int pass = 0; pass < 3; ++pass) {
      staged = cb->ops;
      int cur = 0;
      size_t need = 0;
      for (GemvP& p : staged) {
        const size_t b = plan_staged(p, cb->M, cb->W, grid, cur);
        if (b > need) need = b;
      }
      if (need == 0) break;
      const size_t tot = need > cb->lds ? need : cb->lds;
      P0_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kChainLdsMax),
             "p0_chain_end");
      int pc = 0;
      P0_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, (const void*)k, 64 * cb->W, tot), "p0_chain_end");
      if (pc >= 1 && ctx().cu_count * pc >= grid) {
        cb->ops = staged;
        lds = tot;
        break;
      }
      if (pc < 1) break;
      grid = ctx().cu_count * pc;
    }
  }
  // 6 - 16 rows (2 - 16 with knob 12 = 2): the wide pipelined kernel, one workgroup per CU, when every op can be
  // planned for it
  bool pipe = false;
  const int wide_min = g_chain_wide >= 2 ? 2 : pipe_max_m() + 1;
  if (cb->M >= wide_min && cb->M <= wide_max_m() && g_chain_stage && g_chain_wide && !cb->q8) {
    chain_kernel_t wk = wide_chain_kernel(cb->M);
    const int wlds = wide_lds_bytes(cb->M);
    P0_HIP(hipFuncSetAttribute((const void*)wk, hipFuncAttributeMaxDynamicSharedMemorySize, wlds), "p0_chain_end");
    int pc = 0;
    P0_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, (const void*)wk, 64 * pipe_waves(), wlds), "p0_chain_end");
    std::vector<GemvP> planned = cb->ops;
    if (pc >= 1 && plan_wide(planned, ctx().cu_count)) {
      cb->ops = planned;
      k = wk;
      cb->W = pipe_waves();
      grid = ctx().cu_count;
      lds = wlds;
      pipe = true;
    }
  }
  // M <= pipe_max_m(): the pipelined kernel, one workgroup per CU, when every op can be planned for it
  if (!pipe && cb->M <= pipe_max_m() && g_chain_stage && (cb->M == 1 || g_chain_pipe_m)) {
    chain_kernel_t pk = pipe_chain_kernel(cb->M, cb->q8);
    const int plds = pipe_lds_bytes(cb->M);
    P0_HIP(hipFuncSetAttribute((const void*)pk, hipFuncAttributeMaxDynamicSharedMemorySize, plds), "p0_chain_end");
    int pc = 0;
    P0_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, (const void*)pk, 64 * pipe_waves(), plds), "p0_chain_end");
    std::vector<GemvP> planned = cb->ops;
    if (pc >= 1 && plan_pipe(planned, ctx().cu_count, cb->M)) {
      for (GemvP& o : planned) o.mf = cb->M >= 2 && cb->M >= g_pipe_mf_min_m;
      cb->ops = planned;
      k = pk;
      cb->W = pipe_waves();
      grid = ctx().cu_count;
      lds = plds;
      pipe = true;
    }
  }
  if (pipe_only && !pipe) return P0_OK;
  if (cb->aux && !pipe) {
    set_error("p0_chain_end: copy, argmax, rowstats and normadd ops join only pipelined chains (M <= 5 or rows that "
              "share no memory, 16-byte aligned weights, splits of at most 2048 k for M > 1, knobs 4 and 8 on)");
    return P0_EINVAL;
  }
  if (cb->q8 && !pipe) {
    set_error("p0_chain_end: q8g64s.t64 ops join only pipelined chains (M <= 5 or rows that share no memory, "
              "16-byte aligned weights, splits of at most 2048 k for M > 1, knobs 4 and 8 on)");
    return P0_EINVAL;
  }
  mark_coherence(cb->ops, cb->M);
  if (cb->aux) plan_aux_waits(cb->ops, cb->M);
  std::vector<int64_t> mb_out, mb_in;
  size_t mb_words = pipe && cb->M == 1 && g_chain_mbx ? plan_mailboxes(cb->ops, mb_out, mb_in) : 0;
  std::vector<int64_t> stg_out, stg_in;
  size_t stg_base = 0;
  if (pipe && cb->M > 1 && g_chain_stg) {
    stg_base = (mb_words + 63) & ~(size_t)63;
    const size_t w = plan_staging(cb->ops, cb->M, stg_out, stg_in);
    if (w) mb_words = stg_base + w;   // the staged x' follows the mailboxes (none at M > 1) in the chain state
  }
  auto* ex = new ChainExec{};
  ex->n_ops = (int)cb->ops.size();
  ex->M = cb->M;
  ex->W = cb->W;
  ex->grid = grid;
  ex->lds = lds;
  ex->kernel = k;
  if (pipe) {
    ex->pipe_cfg[0] = g_pipe_loaders;
    ex->pipe_cfg[1] = k == wide_chain_kernel(cb->M) ? g_wide_depth : cb->M > 1 ? g_pipe_depth_m : g_pipe_depth;
    ex->pipe_cfg[2] = g_wide_predict;
  }
  // chain state: last tag, timed out, the workgroups' lines and the completion counters (one 128-byte line each)
  const size_t mb_base = (chain_state_words((int)cb->ops.size(), grid) + 63) & ~(size_t)63;   // 256-byte aligned
  const size_t words = mb_words ? mb_base + mb_words : chain_state_words((int)cb->ops.size(), grid);
  const size_t ob = cb->ops.size() * sizeof(GemvP), sb = words * sizeof(unsigned);
  ex->st_words = words;
  hipError_t e = hipMalloc((void**)&ex->ops, ob);
  if (e == hipSuccess) e = state_alloc(&ex->st, sb);
  if (e == hipSuccess && mb_words) {
    for (size_t i = 0; i < cb->ops.size(); ++i) {
      if (!mb_out.empty() && mb_out[i] >= 0) cb->ops[i].mbxOut = (unsigned long long*)(ex->st + mb_base + mb_out[i]);
      if (!mb_in.empty() && mb_in[i] >= 0) cb->ops[i].mbxIn = (const unsigned long long*)(ex->st + mb_base + mb_in[i]);
      if (!mb_in.empty() && mb_in[i] >= 0) ++ex->mailboxes;
      if (!stg_out.empty() && stg_out[i] >= 0) cb->ops[i].stgOut = ex->st + mb_base + stg_base + stg_out[i];
      if (!stg_in.empty() && stg_in[i] >= 0) cb->ops[i].stgIn = ex->st + mb_base + stg_base + stg_in[i];
      if (!stg_in.empty() && stg_in[i] >= 0) ++ex->staged;
    }
  }
  if (e == hipSuccess) e = hipMemcpy(ex->ops, cb->ops.data(), ob, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(ex->st, 0, sb);
  if (e == hipSuccess && ex->pipe_cfg[0])
    e = hipMemcpy(ex->st + pipe_cfg_word(), ex->pipe_cfg, sizeof ex->pipe_cfg, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(ex->ops);   // (the first error is the one reported)
    state_free(ex->st);
    delete ex;
    return fail_hip(e, "p0_chain_end");
  }
  {
    GemvP* ops_mem = ex->ops;
    unsigned* st_mem = ex->st;
    ex->dev = Keep(ops_mem, [st_mem](void* q) {
      (void)hipFree(q);
      state_free(st_mem);
    });
  }
  *out = ex;
  return P0_OK;
}

extern "C" int p0_chain_run(void* chain) {
  if (int r = require_open("p0_chain_run")) return r;
  if (!chain) { set_error("p0_chain_run: no chain"); return P0_EINVAL; }
  if (g_chain) { set_error("p0_chain_run: a chain is being built"); return P0_EINVAL; }
  auto* ex = (ChainExec*)chain;
  const size_t np = ex->parts.size();
  for (size_t i = 0; i < (np ? np : 1); ++i) {   // row-group passes in order, each after the one before on the stream
    ChainExec* e = np ? ex->parts[i] : ex;
    hipLaunchKernelGGL(e->kernel, dim3((unsigned)e->grid), dim3(64 * e->W), e->lds, ctx().cur, e->ops, e->n_ops,
                       e->st, g_chain_force_give_up ? -1 : g_chain_spin);
    P0_LAUNCHED("p0_chain_run");
    keep_for_recording(e->dev);
  }
  return P0_OK;
}

extern "C" int p0_chain_status(void* chain, int32_t* timed_out) {
  if (int r = require_open("p0_chain_status")) return r;
  if (!chain || !timed_out) { set_error("p0_chain_status: no chain or output"); return P0_EINVAL; }
  auto* ex = (ChainExec*)chain;
  P0_HIP(hipStreamSynchronize(ctx().cur), "p0_chain_status");
  unsigned any = 0;
  const size_t np = ex->parts.size();
  for (size_t i = 0; i < (np ? np : 1); ++i) {   // every row-group pass reports and resets its own state
    ChainExec* e = np ? ex->parts[i] : ex;
    unsigned v = 0;
    P0_HIP(hipMemcpy(&v, e->st + kCtrStride, sizeof v, hipMemcpyDeviceToHost), "p0_chain_status");
    if (v) {
      // an abandoned run can leave split-K arrival counters mid-way: clear them, and the chain state with them
      P0_HIP(hipMemset(e->st, 0, e->st_words * sizeof(unsigned)), "p0_chain_status");
      if (e->pipe_cfg[0])
        P0_HIP(hipMemcpy(e->st + pipe_cfg_word(), e->pipe_cfg, sizeof e->pipe_cfg, hipMemcpyHostToDevice),
               "p0_chain_status");
      P0_HIP(hipMemset(ctx().counters, 0, ctx().n_counters * sizeof(unsigned)), "p0_chain_status");
      P0_HIP(hipDeviceSynchronize(), "p0_chain_status");
      any = 1;
    }
  }
  *timed_out = any ? 1 : 0;
  return P0_OK;
}

extern "C" int p0_chain_info(void* chain, p0_chain_info_t* out) {
  if (!chain || !out) { set_error("p0_chain_info: no chain or output"); return P0_EINVAL; }
  auto* ex = (ChainExec*)chain;
  out->n_ops = ex->n_ops;
  out->m = ex->M;
  out->workgroups = ex->grid;
  out->waves_per_workgroup = ex->W;
  out->lds_bytes = (int64_t)ex->lds;
  out->mailboxes = ex->mailboxes;
  out->staged = ex->staged;
  out->passes = ex->parts.empty() ? 1 : (int32_t)ex->parts.size();
  return P0_OK;
}

extern "C" int p0_chain_free(void* chain) {
  if (!chain) return P0_OK;
  auto* ex = (ChainExec*)chain;
  if (ctx().device >= 0) (void)hipStreamSynchronize(ctx().cur);   // (freeing proceeds whatever it reports)
  for (ChainExec* e : ex->parts) delete e;
  delete ex;   // the op table and state go once no recording that ran the chain holds them
  return P0_OK;
}

// chain knobs: 0 = waves per workgroup for M = 1 (8 or 16), 1 = largest wave share (groups) before K is split
// across workgroups, 2 = polls before a wait gives up, 3 = 1: every wait gives up at once (tests), 4 = staged ops
// (1, the default) or none (0), 5 / 6 = loader waves / slots in flight of the pipelined kernel, 7 = mailbox hand-offs
// in pipelined chains (1, the default) or none (0), 8 = gemvM chains of M <= 5 on the pipelined kernel (1, the
// default) or the general one (0). Returns the previous value; a value < 0 only reads (knobs 3, 4, 7 and 8 also
// take 0).
extern "C" int p0_chain_tune(int knob, int value) {
  if (knob == 12) {
    const int old = g_chain_wide;
    if (value >= 0) g_chain_wide = value > 2 ? 2 : value;
    return old;
  }
  if (knob == 14) {
    const int old = g_wide_predict;
    if (value >= 0) g_wide_predict = value ? 1 : 0;
    return old;
  }
  if (knob == 9) {
    const int old = g_pipe_mf_min_m;
    if (value > 0) g_pipe_mf_min_m = value;
    return old;
  }
  if (knob == 10) {
    const int old = g_chain_stg;
    if (value >= 0) g_chain_stg = value ? 1 : 0;
    return old;
  }
  if (knob == 7 || knob == 8) {
    int* t = knob == 7 ? &g_chain_mbx : &g_chain_pipe_m;
    const int old = *t;
    if (value >= 0) *t = value ? 1 : 0;
    return old;
  }
  if (knob == 3) {
    const int old = g_chain_force_give_up;
    if (value >= 0) g_chain_force_give_up = value ? 1 : 0;
    return old;
  }
  if (knob == 4) {
    const int old = g_chain_stage;
    if (value >= 0) g_chain_stage = value ? 1 : 0;
    return old;
  }
  if (knob == 5 || knob == 6 || knob == 11 || knob == 13) {
    int* t = knob == 5 ? &g_pipe_loaders : knob == 6 ? &g_pipe_depth : knob == 11 ? &g_pipe_depth_m : &g_wide_depth;
    const int old = *t;
    if (value > 0) *t = knob == 5 ? (value > 4 ? 4 : value) : (value >= 2 ? 2 : 1);
    return old;
  }
  int* t = knob == 0 ? &g_chain_waves : knob == 1 ? &g_chain_split_gpw : knob == 2 ? &g_chain_spin : nullptr;
  if (!t) return -1;
  const int old = *t;
  if (value > 0) *t = knob == 0 ? (value >= 16 ? 16 : 8) : value;
  return old;
}
