// gemm.mjs - gemm(gpu, a): Y[m, n] = sum_k X'[m, k] W[n, k] with q4g32a.t64 weights dequantised inside the kernel
// (engine/ops/gemm.js:255-322), on the MI355X library's MFMA kernel. Same argument object and return value (2 M N K).
// Prologues f16 | lnmod | rms (+ bf16 activations); epilogues f16 | f32 | resadd | swiglu | bias | heads.
// Not part of this build, and refused with an Error: the conv / conv3 prologues and the onormgate epilogue (they run
// on f16-weight GEMMs in the reference, off the q4 path), and acc: 'f16' (the reference's fp16-partial-sum mode for its
// autotuner): this build always accumulates in fp32.
'use strict';
import { native } from '../native.mjs';
import { ENC, addr, within } from '../llm/lops.mjs';

export const DEFAULT_TILE = { BM: 256, BN: 256 };
const XMODE = { f16: 0, lnmod: 1, rms: 2, bf16: 3 };
const GEPI = { f16: 0, f32: 1, resadd: 2, swiglu: 3, bias: 4, heads: 5 };
const ACT = { silu: 0, gelu: 1 };
const ROPE = { inter: 0, half: 1 };

/** a = { w: {buf, off, enc, rows (Nw), cols (Ktot)}, x: {buf, off (bytes), ld, k0, mode}, M, N, K, wr0, wr1, wk0, epi,
 *        y: {buf, off (bytes), ld, n0}, ev: {buf, off (floats)}, stats: {buf, off (rows)}, pv: {buf, off, stride},
 *        bv: {buf, off, up}, act, store, res,
 *        heads: {Ltot, Hq, Hkv, rowOff, eps, ropeMode: 'inter' | 'half', rope: {buf}} (epi 'heads') }  ->  2 M N K
 *  Every view on a buffer handle that knows its size is checked against it before the call (WebGPU bound-checks its
 *  bindings; a HIP kernel reading past an allocation would fault). */
export function gemm(gpu, a) {
  const enc = ENC[a.w.enc];
  if (!enc || enc !== ENC['q4g32a.t64']) throw new Error('gemm: unsupported weight encoding ' + a.w.enc);
  if (a.conv) throw new Error('gemm: the conv prologues are not part of this build');
  const acc = a.acc || (gpu && gpu.tune && gpu.tune.acc) || 'f32';
  if (acc !== 'f32') throw new Error('gemm: acc ' + acc + ' is not part of this build (it accumulates in fp32)');
  const mode = (a.x && a.x.mode) || 'f16', epi = a.epi || 'f16';
  if (!(mode in XMODE)) throw new Error('gemm: x mode ' + mode);
  if (!(epi in GEPI)) throw new Error('gemm: epilogue ' + epi + ' is not part of this build');
  const M = a.M, N = a.N, K = a.K, h = a.heads || {};
  if (K % 32) throw new Error('gemm: K must be a multiple of 32');   // engine/ops/gemm.js:278
  if (epi === 'heads' && !((h.ropeMode || 'inter') in ROPE)) throw new Error('gemm: heads ropeMode ' + h.ropeMode);
  // the extent of every view the call reads or writes (bytes past the view's buffer start)
  const xs = mode === 'lnmod' || mode === 'rms' ? 4 : 2, ldx = a.x.ld || K, ldy = a.y.ld || N;
  within('gemm', 'w', a.w.buf, (a.w.off || 0) + (a.w.rows / 64) * (a.w.cols / 32) * 1280);
  within('gemm', 'x', a.x.buf, (a.x.off || 0) + ((M - 1) * ldx + (a.x.k0 || 0) + K) * xs);
  if (epi === 'heads') {
    within('gemm', 'y', a.y.buf, (a.y.off || 0) + ((N / 128 - 1) * h.Ltot + (h.rowOff || 0) + M) * 256);
    if (h.rope) within('gemm', 'heads.rope', h.rope.buf, ((h.rowOff || 0) + M) * 512);
    if (a.ev) within('gemm', 'ev', a.ev.buf, ((a.ev.off || 0) + 256) * 4);
  } else {
    const ys = epi === 'f32' || epi === 'resadd' ? 4 : 2, ny = epi === 'swiglu' ? N / 2 : N;
    within('gemm', 'y', a.y.buf, (a.y.off || 0) + ((M - 1) * ldy + (a.y.n0 || 0) + ny) * ys);
    if (a.ev) within('gemm', 'ev', a.ev.buf, ((a.ev.off || 0) + N) * 4);
  }
  if (a.stats) within('gemm', 'stats', a.stats.buf, ((a.stats.off || 0) + M) * 8);
  if (a.pv) {
    const k1 = (a.x.k0 || 0) + K;
    within('gemm', 'pv', a.pv.buf, ((a.pv.off || 0) + k1) * 4);
    if (mode === 'lnmod') within('gemm', 'pv', a.pv.buf, ((((a.pv.off || 0) + (a.pv.stride || 0)) >>> 0) + k1) * 4);
  }
  if (a.bv) within('gemm', 'bv', a.bv.buf, ((a.bv.off || 0) + (a.bv.up || 0) + (epi === 'swiglu' ? N / 2 : N)) * 4);
  return native().gemm({
    w: addr(a.w.buf), w_off: a.w.off || 0, w_enc: enc, w_rows: a.w.rows, w_cols: a.w.cols,
    x: addr(a.x.buf), x_off: a.x.off || 0, x_ld: a.x.ld || 0, x_k0: a.x.k0 || 0, x_mode: XMODE[mode],
    M, N, K, wr0: a.wr0 || 0, wr1: a.wr1 || 0, wk0: a.wk0 || 0, epi: GEPI[epi],
    y: addr(a.y.buf), y_off: a.y.off || 0, y_ld: a.y.ld || 0, y_n0: a.y.n0 || 0,
    ev: a.ev ? addr(a.ev.buf) : 0, ev_off: a.ev ? a.ev.off || 0 : 0,
    stats: a.stats ? addr(a.stats.buf) : 0, stats_off: a.stats ? a.stats.off || 0 : 0,
    pv: a.pv ? addr(a.pv.buf) : 0, pv_off: a.pv ? a.pv.off || 0 : 0, pv_stride: a.pv ? (a.pv.stride || 0) >>> 0 : 0,
    bv: a.bv ? addr(a.bv.buf) : 0, bv_off: a.bv ? a.bv.off || 0 : 0, bv_up: a.bv ? a.bv.up || 0 : 0,
    act: ACT[a.act || 'silu'], store: a.store ? 1 : 0, res: a.res ? 1 : 0,
    // the reference binds the RoPE table from the start of its buffer (engine/ops/gemm.js:304)
    heads_ltot: h.Ltot || 0, heads_row_off: h.rowOff || 0, heads_hq: h.Hq || 0, heads_hkv: h.Hkv || 0,
    heads_eps: h.eps || 1e-6, heads_rope: ROPE[h.ropeMode || 'inter'], rope: h.rope ? addr(h.rope.buf) : 0,
  });
}
