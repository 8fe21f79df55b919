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

/** a view's extent against its buffer: a handle that knows its size (`_pf`, every Gpu.buffer) must hold `end` bytes.
 *  WebGPU bound-checks every binding; a HIP kernel reading or writing past an allocation can fault the device, so the
 *  ops check on the host before the call. */
export function within(op, name, buf, end) {
  if (buf && buf._pf != null && end > buf._pf) throw new Error(`${op}: ${name} needs ${end} B of a ${buf._pf} B buffer`);
}
/** bytes of a weight tensor of `rows` x `cols` in its record encoding */
export function weightBytes(enc, rows, cols) {
  return enc === 'q8g64s.t64' ? (rows / 64) * (cols / 64) * 4224 : (rows / 64) * (cols / 32) * 1280;
}
/** the number of K splits gemv writes (engine/llm/lops.js:116-121) */
function splitsOf(K, kPer) {
  const kch = !kPer && K > 2048 ? Math.ceil(K / 256) * 256 : KCH;
  const kp = kPer ? Math.min(kPer, kch) : Math.min(K, kch);
  return kp > 0 ? Math.ceil(K / kp) : 1;
}
/** host-side bounds of gemv / gemvM's views (M rows of x) */
export function checkViews(op, a, M, nsplit) {
  const K = a.K, N = a.N, geglu = a.epi === 'geglu', pro = a.pro || 'raw';
  within(op, 'w', a.w.buf, (a.w.off || 0) + weightBytes(a.w.enc, a.w.rows, a.w.cols));
  const ldx = a.x.ldx || K;
  if (pro === 'sum' || pro === 'pleg') {
    const n = (a.src && a.src.n) || 1, ld = (a.src && a.src.ld) || 0;
    within(op, 'x', a.x.buf, ((n - 1) * ld + (M - 1) * ldx + K) * 4);
  } else within(op, 'x', a.x.buf, ((a.x.rowB || 0) + (M - 1) * ldx + K) * 4);
  const ldm = (a.y.ldm || N), ldy = a.ldy || a.y.ldy || (M > 1 ? M * ldm : N);
  within(op, 'y', a.y.buf, ((geglu || a.epi === 'softcap' ? 0 : (nsplit - 1) * ldy) + (M - 1) * ldm + N) * 4);
  if (pro === 'rms') within(op, 'norm', a.norm && a.norm.buf, ((a.norm && a.norm.off || 0) + K) * 4);
  if (pro === 'pleg' && a.ev) within(op, 'ev', a.ev.buf, ((a.ev.off || 0) + (M - 1) * (a.ev.ld || 0) + K) * 4);
  if (a.epi === 'softcap' && a.mx) within(op, 'mx', a.mx.buf, M * (N / 64) * 8);
  if (geglu) within(op, 'w', a.w.buf, (a.w.off || 0) + weightBytes(a.w.enc, 2 * N, a.w.cols));
}

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
  checkViews('gemv', a, 1, splitsOf(a.K, a.kPer));
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
