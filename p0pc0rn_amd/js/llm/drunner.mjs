// drunner.mjs - the decode loop's recorder (engine/llm/drunner.js:1-8, 37-101), on the MI355X library.
//
// The reference records one decode token's dispatches into a WebGPU command buffer once per token and submits it
// when the token's id is known. Here the ops of a token are recorded ONCE (their buffers are persistent, as in the
// reference's decode path) and every submit replays them with one launch:
//   mode 'chain': the token's gemv / gemvM calls become one persistent kernel (p0_chain_*), which streams the next
//                 op's weights while the previous op finishes (all ops of one chain share M);
//   mode 'graph': the calls are captured as a HIP graph (p0_record_*), one kernel per op, any op kind.
// Usage: r.begin(); <the token's ops, called as always>; const tk = r.end(); ... await r.submit(tk) per token.
'use strict';
import { native } from '../native.mjs';

export class DecodeRunner {
  constructor(g, { mode = 'graph' } = {}) {
    if (mode !== 'graph' && mode !== 'chain') throw new Error('DecodeRunner: mode ' + mode);
    this.g = g; this.mode = mode; this.cur = false; this.submits = 0; this.tokens = [];
  }
  /** start recording a token's ops (the reference's parity argument is accepted and not needed) */
  begin() {
    if (this.cur) throw new Error('DecodeRunner: a token is already being recorded');
    if (this.mode === 'chain') native().chainBegin(); else native().recordBegin();
    this.cur = true;
  }
  /** finish recording -> a token handle that submit() replays any number of times */
  end() {
    if (!this.cur) throw new Error('DecodeRunner: end without begin');
    this.cur = false;
    const h = this.mode === 'chain' ? native().chainEnd() : native().recordEnd();
    const tk = { mode: this.mode, h };
    this.tokens.push(tk);
    return tk;
  }
  /** enqueue the recorded token; the promise resolves once the GPU has finished it */
  submit(tk) {
    if (tk.mode === 'chain') native().chainRun(tk.h); else native().replay(tk.h);
    this.submits++;
    return Promise.resolve().then(() => {
      native().done();
      if (tk.mode === 'chain' && native().chainStatus(tk.h)) throw new Error('DecodeRunner: a chain wait gave up (the token is invalid)');
    });
  }
  /** release every recorded token */
  forget() {
    for (const tk of this.tokens) { if (tk.mode === 'chain') native().chainFree(tk.h); else native().recordFree(tk.h); }
    this.tokens = [];
  }
}
