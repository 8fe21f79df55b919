// lopsx.mjs - the kernel-pick surface of the reference's tuned GEMV (engine/llm/lopsx.js:225-328), on the MI355X
// library. The reference keeps two WGSL GEMV families and a per-shape table that sends a call to its "v5" family with
// thread-mapping options (ND rows per workgroup, L lanes per row, staged or direct x, the nibble decode). On this
// backend one gfx950 kernel family serves every shape, so the options choose nothing: gemvV5 / gemvMV5 check what the
// reference's v5 path requires, with its error texts, and then run the same kernels as gemv / gemvM. The pick state
// (PICK, KX, setKX, setPicks, picksNow, kxPick) is kept as data with the reference's semantics, because the tune
// harnesses (engine/tune/apply.js, engine/tune/kshipped.js) import and iterate it.
'use strict';
import { gemv, KCH } from './lops.mjs';
import { gemvM } from './lops_spec.mjs';

/** the v5 path takes 4-bit weights at 16-byte offsets with K % 32 == 0 (engine/llm/lopsx.js:225) */
export const okV5 = (a) => a.w.enc === 'q4g32a.t64' && !((a.w.off || 0) % 16) && !(a.K % 32);
/** direct x needs 4-float aligned x rows and norm weights (engine/llm/lopsx.js:227) */
export const directOkV5 = (a) => !((a.x.rowB || 0) % 4) && !((a.x.ldx || a.K) % 4) && !((a.norm ? a.norm.off || 0 : 0) % 4);
/** WGSL's packed_4x8_integer_dot_product, which the 'u8' decode needs (engine/llm/lopsx.js:230). There is no WebGPU
 *  adapter here, so this is false, as it is in the reference without one; the HIP kernel has no such variant. */
export const u8ok = () => false;
/** storage buffers a 'direct' v5 dispatch binds (engine/llm/lopsx.js:232); kept for the tune harness's checks */
export const DIRECT_NEEDS = { gemv: 9, gemvM: 10 };

/** the reference's shipped picks, 'pro.epi.NxK' -> v5 options (engine/llm/lopsx.js:312). Its keys are the shapes the
 *  kshipped harness checks; the option values select WGSL mappings and have no effect on this backend. */
export const PICK = {
  'rms.softcap.262144x1536': { ND: 4, L: 16, deq: 'mask' }, 'rms.geglu.6144x1536': { ND: 2, L: 8 },
  'raw.store.1536x6144': { ND: 4, L: 16, mode: 'direct' }, 'rms.geglu.12288x1536': { ND: 2, L: 8 },
  'raw.store.1536x12288': { ND: 4, L: 16, mode: 'direct' }, 'raw.store.8960x1536': { ND: 4, L: 16, mode: 'direct' },
  'rms.store.3072x2560': { ND: 2, L: 8 }, 'raw.store.2560x2048': { ND: 2, L: 8 }, 'rms.store.6144x2560': { ND: 2, L: 8 },
  'raw.store.2560x4096': { ND: 4, L: 16, mode: 'direct' }, 'rms.store.2048x2560': { ND: 2, L: 8 },
  'rms.store.4096x2560': { ND: 2, L: 8 }, 'rms.softcap.262144x2560': { ND: 4, L: 16, deq: 'mask' },
  'rms.geglu.10240x2560': { ND: 2, L: 8 }, 'raw.store.2560x10240': { ND: 4, L: 16, mode: 'direct' },
  'raw.store.256x2560': { ND: 4, L: 16, mode: 'direct', deq: 'u8' }, 'raw.store.10752x2560': { ND: 4, L: 8 },
};
export const KX = { on: true };
export function setKX(on) { KX.on = !!on; }
/** the kernel set's version: part of a device tune's cache key (engine/tune/apply.js), so a tune measured on another
 *  kernel set is never applied to this one */
export const KERNEL_VERSION = 'mi355x-hip-1';
const TUNED = { over: null };
/** this device's picks over PICK (null = PICK as shipped); a value that is not an object means the engine's own kernel */
export function setPicks(over) { TUNED.over = over && typeof over === 'object' ? Object.assign({}, over) : null; }
export function picksNow() { return TUNED.over ? Object.assign({}, TUNED.over) : null; }
/** the v5 options for a call, or null for the engine's own kernel (engine/llm/lopsx.js:323-328) */
export function kxPick(a) {
  if (!KX.on || !okV5(a)) return null;
  const key = `${a.pro || 'raw'}.${a.epi || 'store'}.${a.N}x${a.K}`;
  if (TUNED.over && Object.prototype.hasOwnProperty.call(TUNED.over, key)) {
    const o = TUNED.over[key];
    return o && typeof o === 'object' ? o : null;
  }
  return PICK[key] || null;
}

// the checks the reference's v5 option builder makes before any dispatch (engine/llm/lopsx.js:235-244)
function checkV5(g, a, opts) {
  if (!okV5(a)) throw new Error('kernx v5: not a 4-bit, 16-byte aligned, K % 32 weight');
  const ND = opts.ND || 4, L = opts.L || 8, lim = (g && g.limits && g.limits.maxComputeInvocationsPerWorkgroup) || 256;
  if ((64 / ND) * L > lim) throw new Error('kernx v5: ' + (64 / ND) * L + ' threads');
}
function checkSplits(a, kPer) {
  if (kPer % 32) throw new Error('kernx v5: kPer must be a multiple of 32');
  if ((a.epi || 'store') !== 'store' && Math.ceil(a.K / kPer) > 1) throw new Error('kernx v5: ' + a.epi + ' needs one split');
  if (a.N % 64) throw new Error('kernx v5: N % 64');
}

/** the v5 gemv (gemv's arguments, engine/llm/lopsx.js:250-276): the same splits as gemv, so the same return value */
export function gemvV5(g, a, opts = {}) {
  checkV5(g, a, opts);
  const kch = !a.kPer && a.K > KCH ? Math.ceil(a.K / 256) * 256 : KCH;
  if (kch > 3072) throw new Error('kernx v5: K ' + a.K + ' needs a kPer');
  checkSplits(a, Math.min(kch, a.kPer || a.K));
  return gemv(g, a);
}

/** the v5 gemvM (gemvM's arguments, engine/llm/lopsx.js:278-305); opts.XB (x floats per staged sub-chunk) has no
 *  counterpart here: the HIP kernel stages x' per split */
export function gemvMV5(g, a, opts = {}) {
  checkV5(g, a, opts);
  checkSplits(a, a.kPer ? Math.min(KCH, a.kPer) : a.K);
  return gemvM(g, a);
}

/** the reference returns a variant's generated WGSL here; this backend generates no shader code */
export function v5code(cfg) {
  throw new Error('kernx v5: no WGSL on the HIP backend (config ' + JSON.stringify(cfg || {}) + ')');
}
