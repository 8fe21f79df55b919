// store.mjs - PackStore: a weight pack (manifest.json + shard files) read straight into device buffers, the part of the
// reference's PackStore (engine/core/store.js) that the ops read their weights through. The reference downloads packs
// over HTTP into browser storage (OPFS) and verifies them chunk by chunk; this host reads a pack directory that is
// already on local disk, so there is no download, storage or verification step. What stays the same is the call
// surface the model code uses: init(), upload(shardName) -> {name, buf, bytes, t(tensorName)}, uploadPart(shardName,
// names), release(h), readRows(tensorName, ids), readFile(shardName), and the tensor views
// {buf, off, bytes, enc, shape, rows, cols} that gemv / gemvM / gemm take as `a.w` (engine/core/store.js:249-253).
// The bytes move through the library's p0_upload_file (file reads overlapping the host-to-device copies).
'use strict';
import fs from 'fs';
import path from 'path';
import { native } from '../native.mjs';
import { h2f } from './gpu.mjs';

const view = (buf, x, off) => ({ buf, off, bytes: x.bytes, enc: x.enc, shape: x.shape, rows: x.shape[0],
                                  cols: x.shape[x.shape.length - 1] });

export class PackStore {
  /** gpu: the Gpu object; opts: {dir: the pack directory (manifest.json lives there)} */
  constructor(gpu, opts = {}) {
    this.gpu = gpu;
    this.dir = opts.dir;
    this.m = null;
    this.shards = new Map();
    this.stats = { uploadBytes: 0, uploadMs: 0 };
  }

  /** reads the manifest: {pack_version, shards: [{name, file, bytes, ...}], tensors: {name: {shard, offset, bytes,
   *  enc, shape}}} (engine/core/store.js:57-65) */
  async init() {
    const p = path.join(this.dir, 'manifest.json');
    if (!fs.existsSync(p)) throw new Error('pack manifest unavailable');
    this.m = JSON.parse(fs.readFileSync(p, 'utf8'));
    this.shards = new Map(this.m.shards.map((s) => [s.name, s]));
    return this;
  }

  _file(s) { return path.join(this.dir, s.file); }

  /** one NEW device buffer holding the whole shard -> {name, buf, bytes, t(tensorName)} (engine/core/store.js:221-253) */
  async upload(shardName) {
    const s = this.shards.get(shardName);
    if (!s) throw new Error('unknown shard ' + shardName);
    const t0 = Date.now();
    const buf = this.gpu.buffer(s.bytes, 'shard ' + shardName);
    native().uploadFile(this._file(s), 0, s.bytes, buf.ptr, 0);
    this.stats.uploadBytes += s.bytes;
    this.stats.uploadMs += Date.now() - t0;
    return this._handle(shardName, buf, s.bytes);
  }

  _handle(shardName, buf, bytes) {
    const tensors = this.m.tensors, h = { name: shardName, buf, bytes };
    h.t = (tn) => {
      const x = tensors[tn];
      if (!x || x.shard !== shardName) throw new Error(`tensor ${tn} not in ${shardName}`);
      return view(h.buf, x, x.offset);
    };
    return h;
  }

  /** a few tensors of a shard in a NEW small buffer, each at a 256-byte aligned offset (engine/core/store.js:208-219) */
  async uploadPart(shardName, names) {
    const s = this.shards.get(shardName), T = this.m.tensors, A = 256;
    if (!s) throw new Error('unknown shard ' + shardName);
    let tot = 0;
    const lay = names.map((n) => {
      const x = T[n];
      if (!x || x.shard !== shardName) throw new Error(`tensor ${n} not in ${shardName}`);
      const o = tot;
      tot += Math.ceil(x.bytes / A) * A;
      return [n, x, o];
    });
    const buf = this.gpu.buffer(tot, 'part ' + shardName);
    for (const [, x, o] of lay) native().uploadFile(this._file(s), x.offset, x.bytes, buf.ptr, o);
    const map = new Map(lay.map(([n, x, o]) => [n, view(buf, x, o)]));
    return { name: shardName + '(part)', buf, bytes: tot, t: (tn) => {
      const r = map.get(tn);
      if (!r) throw new Error(`tensor ${tn} not in part`);
      return r;
    } };
  }

  /** frees a handle's buffer (the reference keeps the last one for a same-size reuse; here device memory is ample) */
  release(h) {
    if (!h || !h.buf) return;
    const b = h.buf;
    h.buf = null;
    if (this.gpu.bufs.has(b)) this.gpu.free(b);
  }

  /** gather + dequantise rows of a *.rows tensor (q4g32a.rows / q8g64s.rows) -> Float32Array [ids.length * K]
   *  (engine/core/store.js:275-301) */
  async readRows(tensorName, ids) {
    const x = this.m.tensors[tensorName], s = this.shards.get(x.shard), K = x.shape[1];
    const q4 = x.enc === 'q4g32a.rows';
    if (!q4 && x.enc !== 'q8g64s.rows') throw new Error('readRows: ' + x.enc);
    const rb = q4 ? K / 2 + (K / 32) * 4 : K + (K / 64) * 2;
    const fd = fs.openSync(this._file(s), 'r');
    const all = Buffer.alloc(ids.length * rb);
    try {
      ids.forEach((id, i) => fs.readSync(fd, all, i * rb, rb, x.offset + id * rb));
    } finally {
      fs.closeSync(fd);
    }
    const out = new Float32Array(ids.length * K), dv = new DataView(all.buffer, all.byteOffset, all.length);
    for (let i = 0; i < ids.length; i++) {
      const b = i * rb, o = i * K;
      if (q4) {
        for (let g = 0; g < K / 32; g++) {
          const sc = h2f(dv.getUint16(b + K / 2 + g * 4, true)), mn = h2f(dv.getUint16(b + K / 2 + g * 4 + 2, true));
          for (let j = 0; j < 16; j++) {
            const by = all[b + g * 16 + j];
            out[o + g * 32 + 2 * j] = (by & 15) * sc + mn;
            out[o + g * 32 + 2 * j + 1] = (by >> 4) * sc + mn;
          }
        }
      } else {
        for (let g = 0; g < K / 64; g++) {
          const sc = h2f(dv.getUint16(b + K + g * 2, true));
          for (let j = 0; j < 64; j++) out[o + g * 64 + j] = dv.getInt8(b + g * 64 + j) * sc;
        }
      }
    }
    return out;
  }

  /** a whole pack file as an ArrayBuffer (tokenizer files, small tables) */
  async readFile(shardName) {
    const s = this.shards.get(shardName);
    if (!s) throw new Error('unknown shard ' + shardName);
    const b = fs.readFileSync(this._file(s));
    return b.buffer.slice(b.byteOffset, b.byteOffset + s.bytes);
  }
}
