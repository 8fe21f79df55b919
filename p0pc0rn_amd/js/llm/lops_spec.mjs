// lops_spec.mjs - gemvM(g, a): y[m] = x[m] W^T for M rows, each weight record read once (engine/llm/lops_spec.js:159-191),
// on the MI355X library. Same argument object, return value and errors as the reference.
'use strict';
import { native } from '../native.mjs';
import { ENC, PRO, EPI, addr, checkViews } from './lops.mjs';

/** a = { w: {buf, off, enc, rows, cols}, x: {buf, ldx, rowB}, M, N, K, kPer, pro: raw|rms|pleg, epi: store|geglu|softcap,
 *        y: {buf, ldy (floats between splits), ldm (floats between rows)}, stat: {buf, off, ld} (rms: rstd of row m at
 *        off + m * ld), norm: {buf, off}, src: {n, ld} (pleg: split partials), ev: {buf, off, ld} (pleg),
 *        mx: {buf} (softcap: [M][N/64][2]), cap }
 *  -> the number of splits written (store: Y[split * ldy + m * ldm + n]) */
export function gemvM(g, a) {
  const enc = ENC[a.w.enc];
  if (!enc || enc === ENC.f16) throw new Error('gemvM: encoding ' + a.w.enc);
  const pro = a.pro || 'raw', epi = a.epi || 'store';
  if (!(pro in PRO) || pro === 'sum') throw new Error('gemvM: prologue ' + pro);
  if (!(epi in EPI)) throw new Error('gemvM: epilogue ' + epi);
  const kp = a.kPer ? Math.min(a.kPer, 2048) : a.K;   // engine/llm/lops_spec.js:170
  checkViews('gemvM', a, a.M, kp > 0 ? Math.ceil(a.K / kp) : 1);
  return native().gemvM({
    w: addr(a.w.buf), w_off: a.w.off || 0, w_enc: enc, w_rows: a.w.rows, w_cols: a.w.cols,
    x: addr(a.x.buf), x_ldx: a.x.ldx || 0, x_rowB: a.x.rowB || 0,
    M: a.M, N: a.N, K: a.K, kPer: a.kPer || 0, pro: PRO[pro], epi: EPI[epi],
    y: addr(a.y.buf), y_ldy: a.y.ldy || 0, y_ldm: a.y.ldm || 0,
    stat: a.stat ? addr(a.stat.buf) : 0, stat_off: a.stat ? a.stat.off || 0 : 0, stat_ld: a.stat ? a.stat.ld || 0 : 0,
    norm: a.norm ? addr(a.norm.buf) : 0, norm_off: a.norm ? a.norm.off || 0 : 0,
    src_n: a.src ? a.src.n : 0, src_ld: a.src ? a.src.ld : 0,
    ev: a.ev ? addr(a.ev.buf) : 0, ev_off: a.ev ? a.ev.off || 0 : 0, ev_ld: a.ev ? a.ev.ld || 0 : 0,
    mx: a.mx ? addr(a.mx.buf) : 0, cap: a.cap || 30,
  });
}

/** argmax of each of M rows of n (max, bitcast index) pairs: out[2 m] = index, out[2 m + 1] = bits of the max
 *  (engine/llm/lops_spec.js:346-348) */
export function argmaxM(g, a) {
  native().argmaxM(addr(a.mx.buf), a.n, a.M, addr(a.out.buf));
}
