// lops.mjs - gemv(g, a): the one-row q4 GEMV of the LLM decode (engine/llm/lops.js:108-141), on the MI355X library.
// Same argument object, same return value (the number of K splits written) and the same thrown errors; the work runs
// in the library's gfx950 kernel (p0pc0rn_amd/csrc/gemv.hip) instead of a WGSL dispatch.
'use strict';
import { native } from '../native.mjs';

export const KCH = 2048;   // the reference's most k per split without a kPer (engine/llm/lops.js:27)
export const ENC = { 'q4g32a.t64': 1, 'q8g64s.t64': 2, f16: 3 };
export const PRO = { raw: 0, rms: 1, sum: 2, pleg: 3 };
export const EPI = { store: 0, geglu: 1, softcap: 2 };

/** the device address of a buffer handle (0 = absent) */
export const addr = (b) => (b ? b.ptr : 0);

function encOf(op, enc) {
  const e = ENC[enc];
  if (!e || e === ENC.f16) throw new Error(op + ': encoding ' + enc);
  return e;
}
function optOf(op, what, table, v) {
  const e = table[v];
  if (e === undefined) throw new Error(`${op}: ${what} ${v}`);
  return e;
}

/** a = {w: {buf, off (bytes), enc, rows (N), cols (K)}, x: {buf, rowB?}, N, K, pro: 'rms'|'raw'|'sum'|'pleg',
 *       epi: 'store'|'geglu'|'softcap', y: {buf}, ldy, kPer, stat: {buf, off (floats)} (rms) | src: {n, ld} (sum/pleg),
 *       norm: {buf, off (floats)}, ev: {buf, off}, mx: {buf}, cap }
 *  geglu: N = the gate rows (the up rows follow at N .. 2N); returns the number of splits written.
 *  a.kx (the reference's pick switch) is accepted and has no effect: this build has one kernel family per regime. */
export function gemv(g, a) {
  const w = encOf('gemv', a.w.enc);
  return native().gemv({
    w: addr(a.w.buf), w_off: a.w.off || 0, w_enc: w, w_rows: a.w.rows, w_cols: a.w.cols,
    x: addr(a.x.buf), x_rowB: a.x.rowB || 0,
    N: a.N, K: a.K, kPer: a.kPer || 0,
    pro: optOf('gemv', 'prologue', PRO, a.pro || 'raw'), epi: optOf('gemv', 'epilogue', EPI, a.epi || 'store'),
    y: addr(a.y.buf), ldy: a.ldy || 0,
    stat: a.stat ? addr(a.stat.buf) : 0, stat_off: a.stat ? a.stat.off || 0 : 0,
    norm: a.norm ? addr(a.norm.buf) : 0, norm_off: a.norm ? a.norm.off || 0 : 0,
    src_n: a.src ? a.src.n : 0, src_ld: a.src ? a.src.ld : 0,
    ev: a.ev ? addr(a.ev.buf) : 0, ev_off: a.ev ? a.ev.off || 0 : 0,
    mx: a.mx ? addr(a.mx.buf) : 0, cap: a.cap || 30,
  });
}

/** per row m < M: x_m = (x_m + rms(sum_j t_j,m) * w) * scale (mode 0) or x_m = sum_j t_j,m (mode 1); ST[statOff + m] =
 *  rstd(x_m) (engine/llm/lops.js:172-178). t: {buf, n (splits), ld (floats between splits)} rows of D;
 *  w: {buf, off}; x: {buf}; st: {buf, off}; eps, scale, mode */
export function normadd(g, a) {
  native().normadd({
    t: addr(a.t.buf), t_n: a.t.n || 1, t_ld: a.t.ld || a.D * (a.M || 1),
    w: a.w ? addr(a.w.buf) : 0, w_off: a.w ? a.w.off || 0 : 0,
    x: addr(a.x.buf), st: addr(a.st.buf), st_off: a.st.off || 0,
    D: a.D, M: a.M || 1, eps: a.eps || 1e-6, scale: a.scale == null ? 1 : a.scale, mode: a.mode || 0,
  });
}

/** argmax over the n per-tile (max, bitcast index) pairs of mx: out[0] = index, out[1] = bits of the max
 *  (engine/llm/lops.js:434-436) */
export function argmax(g, a) {
  native().argmaxM(addr(a.mx.buf), a.n, 1, addr(a.out.buf));
}
