// gemm.mjs - gemm(gpu, a): Y[m, n] = sum_k X'[m, k] W[n, k] with q4g32a.t64 weights dequantised inside the kernel
// (engine/ops/gemm.js:255-322), on the MI355X library's MFMA kernel. Same argument object and return value (2 M N K).
// Prologues f16 | lnmod | rms (+ bf16 activations); epilogues f16 | f32 | resadd | swiglu | bias. The reference's
// conv / conv3 prologues and heads / onormgate epilogues belong to other models' paths and throw here.
'use strict';
import { native } from '../native.mjs';
import { ENC, addr } from '../llm/lops.mjs';

export const DEFAULT_TILE = { BM: 128, BN: 128 };
const XMODE = { f16: 0, lnmod: 1, rms: 2, bf16: 3 };
const GEPI = { f16: 0, f32: 1, resadd: 2, swiglu: 3, bias: 4 };
const ACT = { silu: 0, gelu: 1 };

/** a = { w: {buf, off, enc, rows (Nw), cols (Ktot)}, x: {buf, off (bytes), ld, k0, mode}, M, N, K, wr0, wr1, wk0, epi,
 *        y: {buf, off (bytes), ld, n0}, ev: {buf, off (floats)}, stats: {buf, off (rows)}, pv: {buf, off, stride},
 *        bv: {buf, off, up}, act, store, res }  ->  2 M N K */
export function gemm(gpu, a) {
  const enc = ENC[a.w.enc];
  if (!enc) throw new Error('gemm: unsupported weight encoding ' + a.w.enc);
  if (a.conv) throw new Error('gemm: the conv prologues are not part of this build');
  const mode = (a.x && a.x.mode) || 'f16', epi = a.epi || 'f16';
  if (!(mode in XMODE)) throw new Error('gemm: x mode ' + mode);
  if (!(epi in GEPI)) throw new Error('gemm: epilogue ' + epi + ' is not part of this build');
  return native().gemm({
    w: addr(a.w.buf), w_off: a.w.off || 0, w_enc: enc, w_rows: a.w.rows, w_cols: a.w.cols,
    x: addr(a.x.buf), x_off: a.x.off || 0, x_ld: a.x.ld || 0, x_k0: a.x.k0 || 0, x_mode: XMODE[mode],
    M: a.M, N: a.N, K: a.K, wr0: a.wr0 || 0, wr1: a.wr1 || 0, wk0: a.wk0 || 0, epi: GEPI[epi],
    y: addr(a.y.buf), y_off: a.y.off || 0, y_ld: a.y.ld || 0, y_n0: a.y.n0 || 0,
    ev: a.ev ? addr(a.ev.buf) : 0, ev_off: a.ev ? a.ev.off || 0 : 0,
    stats: a.stats ? addr(a.stats.buf) : 0, stats_off: a.stats ? a.stats.off || 0 : 0,
    pv: a.pv ? addr(a.pv.buf) : 0, pv_off: a.pv ? a.pv.off || 0 : 0, pv_stride: a.pv ? (a.pv.stride || 0) >>> 0 : 0,
    bv: a.bv ? addr(a.bv.buf) : 0, bv_off: a.bv ? a.bv.off || 0 : 0, bv_up: a.bv ? a.bv.up || 0 : 0,
    act: ACT[a.act || 'silu'], store: a.store ? 1 : 0, res: a.res ? 1 : 0,
  });
}
