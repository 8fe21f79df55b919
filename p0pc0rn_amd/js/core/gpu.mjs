// gpu.mjs - the host's device object on the MI355X library: the subset of the reference's Gpu
// (engine/core/gpu.js:17-170, 273-297) that the q4 ops and their callers use, with the same method names and meanings.
//
//   createGpu(opts)                   -> Gpu           (engine/core/gpu.js:18-23)
//   g.buffer(size, label)             -> buffer handle (rounded up to 16 B; alive / peak accounting, :81-88)
//   g.free(b), g.freeAll()                             (:89-95)
//   g.upload(data, label, dst, dstOff)                 (:98-105)
//   g.read(buf, off, size) -> Promise<ArrayBuffer>; g.readInto(buf, off, size, dst)   (:107-114)
//   g.done() -> Promise                                (:141-147)
//   g.describe(), g.limits, g.rate, g.runner.flush()/sync()
//   f2h, h2f, toF16, fromF16                           (:273-297)
//
// A buffer handle is { ptr (device address), _pf (bytes), label, size }. Ops are enqueued on the library's stream and
// return at once, as the reference's ops only record; read/done wait for them.
'use strict';
import { native } from '../native.mjs';

export const MB = 1e6;
export class GpuError extends Error {}

/** Create the device context (one per process). opts: {device = 0} */
export async function createGpu(opts = {}) {
  const g = new Gpu(opts);
  g.init();
  return g;
}

export class Gpu {
  constructor(opts = {}) {
    this.opts = Object.assign({ device: 0, maxDispatchSeconds: 0.2 }, opts);
    this.alive = 0; this.peak = 0; this.bufs = new Set();
    this.lostInfo = null;
    // measured-rate placeholders the reference uses for dispatch sizing; MI355X-scale defaults (HBM, fp16 MFMA)
    this.rate = { mm: 1.0e15, mm16: 1.0e15, mm32: 1.0e15, attn: 0.2e15, mem: 6e12 };
    // the reference's batching runner: ops are enqueued on the library's stream as they are called, so flush / sync
    // have nothing to do; copy is a stream-ordered device copy (engine/core/gpu.js:237-242)
    this.runner = {
      flush() {}, sync() {}, forget() {}, dispatches: 0, submits: 0,
      copy(src, srcOff, dst, dstOff, size) { native().copy(src.ptr, srcOff, dst.ptr, dstOff, size); },
    };
  }

  init() {
    const n = native();
    try { n.open(this.opts.device); } catch (e) { throw new GpuError(e.message); }
    this.info = n.info();
    this.device = { destroy: () => n.close() };
    this.f16 = true; this.subgroups = true; this.sgMin = 64; this.sgMax = 64; this.sgOK16 = true;
    this.limits = {
      maxBufferSize: this.info.hbmBytes,
      maxStorageBufferBindingSize: this.info.hbmBytes,   // no binding windows on this device
      maxComputeWorkgroupStorageSize: 65536,
      maxComputeInvocationsPerWorkgroup: 1024,
      maxStorageBuffersPerShaderStage: 64,
    };
  }

  get lost() { return !!this.lostInfo; }
  describe() {
    return Object.assign({ vendor: 'amd', architecture: this.info.name, description: 'MI355X (HIP)' }, {
      f16: true, subgroups: true, sgMin: 64, sgMax: 64, cuCount: this.info.cuCount, xcdCount: this.info.xcdCount,
      maxBufferMB: Math.round(this.limits.maxBufferSize / 1048576), maxBindMB: Math.round(this.limits.maxStorageBufferBindingSize / 1048576),
      wgMem: this.limits.maxComputeWorkgroupStorageSize, wgInv: this.limits.maxComputeInvocationsPerWorkgroup,
    });
  }

  // ------------------------------------------------------------------ buffers (every live byte is counted)
  buffer(size, label = '') {
    size = Math.max(16, Math.ceil(size / 16) * 16);
    if (size > this.limits.maxBufferSize) throw new GpuError(`buffer ${label} ${size} B exceeds maxBufferSize`);
    let ptr;
    try { ptr = native().buffer(size); } catch (e) { throw new GpuError(e.message); }
    const b = { ptr, _pf: size, size, label };
    this.bufs.add(b); this.alive += size;
    if (this.alive > this.peak) this.peak = this.alive;
    return b;
  }
  free(b) {
    if (!b || !this.bufs.has(b)) return;
    this.bufs.delete(b); this.alive -= b._pf;
    native().free(b.ptr);
    b.ptr = 0;
  }
  freeAll() { for (const b of Array.from(this.bufs)) this.free(b); }
  resetPeak() { this.peak = this.alive; }
  /** upload a TypedArray / ArrayBuffer into a NEW buffer (or into dst at dstOff) */
  upload(data, label = '', dst = null, dstOff = 0) {
    const u8 = data instanceof ArrayBuffer ? new Uint8Array(data) : new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
    const b = dst || this.buffer(u8.byteLength, label);
    if (u8.byteLength) native().upload(b.ptr, dstOff, u8);
    return b;
  }
  /** read back [off, off + size) of a buffer as an ArrayBuffer (waits for the ops before it) */
  async read(buf, off = 0, size = null) {
    size = size == null ? buf._pf - off : size;
    return native().read(buf.ptr, off, size);
  }
  async readInto(buf, off, size, dst) {
    const ab = native().read(buf.ptr, off, size);
    new Uint8Array(dst.buffer, dst.byteOffset, size).set(new Uint8Array(ab));
    return dst;
  }
  async done() {
    if (this.lost) throw new GpuError('GPU device lost: ' + JSON.stringify(this.lostInfo));
    try { native().done(); } catch (e) { this.lostInfo = { reason: 'hip', message: e.message, t: Date.now() }; throw new GpuError(e.message); }
  }
  /** fill a buffer with a 32-bit pattern (the NaN-fill of the reference's tuner, engine/tune/autotune.js:1-7) */
  fill(buf, off, u32, words) { native().fill(buf.ptr, off, u32 >>> 0, words); }
  cap(kind = 'mm') { return this.rate[kind] * this.opts.maxDispatchSeconds; }
}

/** a view {buffer, offset, size} (engine/core/gpu.js:267-270) */
export function view(buffer, offset = 0, size = null) {
  size = size == null ? buffer._pf - offset : size;
  return { buffer, offset, size: Math.ceil(size / 4) * 4 };
}

// ------------------------------------------------------------------ fp16 helpers (CPU side), the same results as
// engine/core/gpu.js:273-297 (IEEE binary16, round to nearest even), formulated on the binary16 ulp grid: a value a
// with binade exponent e (e >= -14; subnormals share e = -14) is r = round(a / 2^(e - 10)) ulps, and the bits are
// ((e + 14) << 10) + r for normals and subnormals alike (a carry out of the mantissa moves into the exponent).
export function f2h(v) {
  const f = Math.fround(v);
  if (f !== f) return 0x7e00;
  const sign = f < 0 || (f === 0 && 1 / f < 0) ? 0x8000 : 0, a = Math.abs(f);
  if (a >= 65520) return sign | 0x7c00;   // 65520 = the midpoint above the largest finite half: rounds to Inf
  let e = -14;
  while (e < 15 && a >= 2 ** (e + 1)) e++;
  const q = a / 2 ** (e - 10);              // exact: a power-of-two scaling of an f32
  let r = Math.floor(q);
  const d = q - r;
  if (d > 0.5 || (d === 0.5 && (r & 1))) r++;
  return sign | (((e + 14) << 10) + r);
}
export function h2f(h) {
  const s = h & 0x8000 ? -1 : 1, e = (h >>> 10) & 31, m = h & 1023;
  if (e === 31) return m ? NaN : s * Infinity;
  return s * (e ? 1024 + m : m) * 2 ** ((e || 1) - 25);
}
export function toF16(a) { const o = new Uint16Array(a.length); for (let i = 0; i < a.length; i++) o[i] = f2h(a[i]); return o; }
export function fromF16(u) { const o = new Float32Array(u.length); for (let i = 0; i < u.length; i++) o[i] = h2f(u[i]); return o; }
