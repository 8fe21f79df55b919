// drunner.mjs - the decode loop's recorder (engine/llm/drunner.js:13-122), on the MI355X library.
//
// The reference records one decode token's dispatches into a WebGPU command buffer while the GPU still runs the
// previous token, submits it when that token's id is known, and reads the token's result (argmax, max-logit bits) back
// from a per-parity staging buffer. The same contract here:
//   dr.begin(parity); <the token's ops, called as always>; const tk = dr.end(argBuf, bytes);
//   const o32 = await dr.submit(tk);   // Uint32Array [argmax, max-logit bits, ...] once the GPU has finished the token
//   ... await dr.destroy() after the last token.
// What a token becomes on this device:
//   mode 'graph' (default): the token's ops are captured as a HIP graph (p0_record_*), one kernel per op, any op kind;
//                           end() records the copy of the result words into the parity's staging buffer;
//   mode 'chain':           the token's ops become ONE persistent kernel (p0_chain_*) that streams the next op's
//                           weights while the previous op finishes: gemv / gemvM, copy, argmax / argmaxM, rowstats and
//                           normadd join a chain (the library refuses others, e.g. gemm, while a chain is being built);
//                           end() appends the copy of the result words into the parity's staging buffer, so the token
//                           and its result copy are one launch.
// A token is submitted once, as a command buffer is, and released when its result has been read; with {reuse: true}
// tokens stay until forget() / destroy() and may be submitted again (their buffers must still hold the token's inputs).
'use strict';
import { native } from '../native.mjs';

export class DecodeRunner {
  /** cap = most dispatches in one token; timer = host-side event timing of each submitted token (busyMs, tokens);
   *  stage = result bytes per token (spec passes: 128); mode = 'graph' | 'chain'; reuse = keep submitted tokens */
  constructor(g, { cap = 1024, timer = false, stage = 16, mode = 'graph', reuse = false } = {}) {
    if (mode !== 'graph' && mode !== 'chain') throw new Error('DecodeRunner: mode ' + mode);
    this.g = g; this.core = g.runner; this.cap = cap; this.mode = mode; this.reuse = reuse;
    this.stageBytes = Math.max(16, Math.ceil(stage / 4) * 4);
    this.stage = [0, 1].map((p) => g.buffer(this.stageBytes, 'decode-argmax-' + p));
    this.dispatches = 0; this.submits = 0; this.cur = null; this.open = false; this.kept = new Set();
    this.timer = timer ? { busyMs: 0, tokens: 0, bad: 0, parts: [0, 0, 0, 0] } : null;
  }

  /** start recording a token; parity = token index % 2 (its result staging buffer) */
  begin(parity) {
    if (this.cur) throw new Error('DecodeRunner: a token is already being recorded');
    this._discard();   // a recording left open by a token whose encoding threw (the caller nulled cur)
    if (this.mode === 'chain') native().chainBegin(); else native().recordBegin();
    this.open = true;
    this.cur = { parity: parity & 1, n: 0 };
  }
  _discard() {
    if (!this.open) return;
    this.open = false;
    try {
      const h = this.mode === 'chain' ? native().chainEnd() : native().recordEnd();
      if (this.mode === 'chain') native().chainFree(h); else native().recordFree(h);
    } catch (e) { /* an empty or failed recording: nothing to release */ }
  }
  /** the core Runner's signature: the ops of this build call the library directly, never through a runner */
  dispatch() { throw new Error('DecodeRunner: the MI355X ops record themselves; dispatch() is not used'); }
  /** copy between buffers inside the token (recorded into a graph token, or an op of a chain token) */
  copy(src, srcOff, dst, dstOff, size) {
    if (!this.cur) throw new Error('DecodeRunner: copy outside a token');
    native().copy(src.ptr, srcOff, dst.ptr, dstOff, size);
  }
  split() {}
  flush() {}
  sync() {}

  /** finish recording: the token's result (the first `bytes` of argBuf: argmax, max logit, ...) goes to the parity's
   *  staging buffer when the token runs */
  end(argBuf, bytes = 16) {
    const c = this.cur;
    this.cur = null;
    if (!c) throw new Error('DecodeRunner: end without begin');
    const nb = Math.min(this.stageBytes, Math.ceil(bytes / 4) * 4);
    if (argBuf) native().copy(argBuf.ptr, 0, this.stage[c.parity].ptr, 0, nb);   // recorded / a chain op
    this.open = false;
    const h = this.mode === 'chain' ? native().chainEnd() : native().recordEnd();
    const n = this.mode === 'chain' ? native().chainInfo(h) : native().recordInfo(h);
    if (n > this.cap) {
      if (this.mode === 'chain') native().chainFree(h); else native().recordFree(h);
      throw new Error(`DecodeRunner: more than ${this.cap} dispatches in one token`);
    }
    this.dispatches += n;
    const tk = { parity: c.parity, mode: this.mode, h, n, arg: argBuf, bytes: nb };
    if (this.reuse) this.kept.add(tk);
    return tk;
  }

  /** run the token -> a promise of Uint32Array [argmax, max-logit bits, ...] once the GPU has finished it */
  submit(tk) {
    if (!tk || !tk.h) return Promise.reject(new Error('DecodeRunner: the token was released (submitted once, or forgotten)'));
    const n = native();
    if (this.timer) n.timerStart();
    if (tk.mode === 'chain') n.chainRun(tk.h);
    else n.replay(tk.h);
    this.submits++;
    return Promise.resolve().then(() => {
      if (this.timer) {
        const ms = n.timerStop();
        if (ms >= 0) { this.timer.busyMs += ms; this.timer.parts[0] += ms; } else this.timer.bad++;
        this.timer.tokens++;
      }
      const ab = n.read(this.stage[tk.parity].ptr, 0, tk.bytes);   // waits for the token
      const gaveUp = tk.mode === 'chain' && n.chainStatus(tk.h);
      if (!this.reuse) this._release(tk);
      if (gaveUp) throw new Error('DecodeRunner: a chain wait gave up (the token is invalid)');
      return new Uint32Array(ab);
    });
  }
  _release(tk) {
    if (!tk.h) return;
    const h = tk.h;
    tk.h = null;
    this.kept.delete(tk);
    if (tk.mode === 'chain') native().chainFree(h); else native().recordFree(h);
  }
  /** release every kept token (their handles become unusable: a later submit rejects) */
  forget() { for (const tk of Array.from(this.kept)) this._release(tk); }

  /** after the last token: wait for the device, release the tokens and the staging buffers */
  async destroy() {
    this._discard();
    try { native().done(); } catch (e) { /* a lost device: release what can be released */ }
    this.forget();
    for (const b of this.stage) this.g.free(b);
    this.stage = [];
  }
}
