// store.mjs - WeightStore: a weight pack (manifest.json + shard files) read into device buffers, with the call surface
// the model code uses on the reference's WeightStore (engine/core/store.js:50-303): open(), status(), download(),
// upload(shardName) -> {name, buf, bytes, t(tensorName)}, uploadPart(shardName, names), release(h), drainPool(),
// readRows(tensorName, ids), readFile(shardName), and the tensor views {buf, off, bytes, enc, shape, rows, cols} that
// gemv / gemvM / gemm take as `a.w` (engine/core/store.js:249-253).
//
// Where the bytes come from differs: the reference downloads a pack over HTTP into browser storage (OPFS) and verifies
// it chunk by chunk; this host reads a pack directory already on local disk (opts.base or opts.dir), so download() only
// reports what is missing and there is nothing to verify. Shard bytes move to the device through the library's
// p0_upload_file (file reads overlapping the host-to-device copies).
'use strict';
import fs from 'fs';
import path from 'path';
import { fileURLToPath } from 'url';
import { native } from '../native.mjs';
import { h2f } from './gpu.mjs';

const PART_ALIGN = 256;   // a part upload places each tensor at a multiple of this many bytes

// The row-table encodings (one record per table row, for gathers of a few rows): the row's codes, then one group
// header per `group` k. q4g32a.rows: two 4-bit codes per byte (k even in the low nibble), header = fp16 scale, fp16
// min, value = q * scale + min. q8g64s.rows: one int8 code per k, header = fp16 scale, value = q * scale.
const ROWS = {
  'q4g32a.rows': {
    group: 32, codes: (K) => K >> 1, header: 4,
    decode(u8, dv, at, K, out, o) {
      const hdr = at + (K >> 1);
      for (let g = 0; g < K >> 5; g++) {
        const s = h2f(dv.getUint16(hdr + 4 * g, true)), m = h2f(dv.getUint16(hdr + 4 * g + 2, true));
        for (let k = g << 5; k < (g + 1) << 5; k++) out[o + k] = ((u8[at + (k >> 1)] >> ((k & 1) << 2)) & 15) * s + m;
      }
    },
  },
  'q8g64s.rows': {
    group: 64, codes: (K) => K, header: 2,
    decode(u8, dv, at, K, out, o) {
      for (let g = 0; g < K >> 6; g++) {
        const s = h2f(dv.getUint16(at + K + 2 * g, true));
        for (let k = g << 6; k < (g + 1) << 6; k++) out[o + k] = dv.getInt8(at + k) * s;
      }
    },
  },
};
const rowBytes = (f, K) => f.codes(K) + (K / f.group) * f.header;

/** the view of a manifest tensor entry inside a device buffer, at byte offset `at` */
function tensorView(buf, entry, at) {
  const shape = entry.shape;
  return { buf, off: at, bytes: entry.bytes, enc: entry.enc, shape, rows: shape[0], cols: shape[shape.length - 1] };
}

export class WeightStore {
  /** gpu: the Gpu object; opts: {base: the pack directory (a path or a file: URL; manifest.json lives there)}; the
   *  reference's `dir` (its storage folder) is taken as the directory when base is not given */
  constructor(gpu, opts = {}) {
    this.gpu = gpu;
    const b = opts.base || opts.dir || '.';
    this.root = b.startsWith('file:') ? fileURLToPath(b) : b;
    this.m = null; this.shards = new Map(); this.keep = null;
    this.stats = { uploadBytes: 0, uploadMs: 0, readMs: 0 };
  }

  /** read the manifest (engine/core/store.js:58-86): {format: 'pocketflux.pack', format_version: 1, pack_version,
   *  shards: [{name, file, bytes, ...}], tensors: {name: {shard, offset, bytes, enc, shape}}} -> the manifest */
  async open() {
    let text;
    try { text = fs.readFileSync(path.join(this.root, 'manifest.json'), 'utf8'); } catch (e) {
      throw new Error('pack manifest unavailable (offline and not downloaded)');
    }
    const m = JSON.parse(text);
    if (m.format !== 'pocketflux.pack' || m.format_version !== 1) throw new Error('unsupported pack format ' + m.format + '/' + m.format_version);
    this.m = m;
    this.shards = new Map(m.shards.map((s) => [s.name, s]));
    this.state = { pack_version: m.pack_version, done: {} };
    for (const s of m.shards) if (this._have(s) === s.bytes) this.state.done[s.name] = { sha256: s.sha256 };
    return m;
  }
  _path(s) { return path.join(this.root, s.file); }
  _have(s) { try { return Math.min(fs.statSync(this._path(s)).size, s.bytes); } catch (e) { return 0; } }
  _shard(name) {
    const s = this.shards.get(name);
    if (!s) throw new Error('unknown shard ' + name);
    return s;
  }
  _entry(name, shardName) {
    const x = this.m.tensors[name];
    if (!x || x.shard !== shardName) throw new Error(`tensor ${name} not in ${shardName}`);
    return x;
  }

  /** {have, total, missing, complete}: a shard is complete when its file holds all of its bytes */
  status() {
    const missing = [];
    let have = 0, total = 0;
    for (const s of this.m.shards) {
      const n = this._have(s);
      have += n; total += s.bytes;
      if (n < s.bytes) missing.push(s.name);
    }
    return { have, total, missing, complete: missing.length === 0 };
  }
  /** nothing is fetched: a local pack is complete or it is not (the missing shards are named) */
  async download() {
    const st = this.status();
    if (!st.complete) throw new Error('download: no network source; the pack directory lacks ' + st.missing.join(', '));
    return st;
  }
  /** the reference deletes its storage copy; a local pack directory is the user's and stays */
  async remove() { this.state = { pack_version: this.m && this.m.pack_version, done: {} }; }

  /** a whole pack file as an ArrayBuffer (tokenizer files, small tables) */
  async readFile(shardName) {
    const s = this._shard(shardName), b = fs.readFileSync(this._path(s));
    return b.buffer.slice(b.byteOffset, b.byteOffset + Math.min(b.length, s.bytes));
  }

  /** a shard in one device buffer -> {name, buf, bytes, t(tensorName)}; the buffer kept by the last release is reused
   *  when it has the same size (engine/core/store.js:223-248, 255-271) */
  async upload(shardName) {
    const s = this._shard(shardName), t0 = Date.now();
    const buf = this._reuse(s.bytes) || this.gpu.buffer(s.bytes, 'shard ' + shardName);
    native().uploadFile(this._path(s), 0, s.bytes, buf.ptr, 0);
    this.stats.uploadBytes += s.bytes;
    this.stats.uploadMs += Date.now() - t0;
    return this._handle(shardName, buf, s.bytes);
  }
  _handle(shardName, buf, bytes) {
    const h = { name: shardName, buf, bytes };
    h.t = (name) => { const x = this._entry(name, shardName); return tensorView(h.buf, x, x.offset); };
    return h;
  }

  /** some tensors of a shard in one NEW buffer, each at the next PART_ALIGN boundary (engine/core/store.js:208-219) */
  async uploadPart(shardName, names) {
    const s = this._shard(shardName), at = new Map();
    let size = 0;
    for (const n of names) {
      const x = this._entry(n, shardName);
      at.set(n, size);
      size += Math.ceil(x.bytes / PART_ALIGN) * PART_ALIGN;
    }
    const buf = this.gpu.buffer(size, 'part ' + shardName);
    for (const [n, o] of at) {
      const x = this.m.tensors[n];
      native().uploadFile(this._path(s), x.offset, x.bytes, buf.ptr, o);
    }
    return {
      name: shardName + '(part)', buf, bytes: size,
      t: (n) => {
        if (!at.has(n)) throw new Error(`tensor ${n} not in part`);
        return tensorView(buf, this.m.tensors[n], at.get(n));
      },
    };
  }

  /** done with a handle: its buffer is kept for the next upload of the same size, any earlier kept one freed */
  release(h) {
    if (!h || !h.buf) return;
    const b = h.buf;
    h.buf = null;
    if (!this.gpu.bufs || !this.gpu.bufs.has(b)) return;
    this.drainPool();
    this.keep = b;
  }
  _reuse(bytes) {
    const b = this.keep, size = Math.max(16, Math.ceil(bytes / 16) * 16);
    this.keep = null;
    if (!b) return null;
    if (b._pf === size && this.gpu.bufs.has(b)) return b;
    this.gpu.free(b);
    return null;
  }
  /** free the kept buffer */
  drainPool() {
    if (this.keep) this.gpu.free(this.keep);
    this.keep = null;
  }

  /** gather + dequantise rows of a *.rows tensor -> Float32Array [ids.length * K] (engine/core/store.js:275-301);
   *  runs of consecutive ids are read with one file read each */
  async readRows(tensorName, ids) {
    const x = this.m.tensors[tensorName], s = this._shard(x.shard), K = x.shape[1], f = ROWS[x.enc];
    if (!f) throw new Error('readRows: ' + x.enc);
    const rb = rowBytes(f, K), t0 = Date.now();
    const raw = Buffer.alloc(ids.length * rb), order = ids.map((id, i) => [id, i]).sort((a, b) => a[0] - b[0]);
    const fd = fs.openSync(this._path(s), 'r');
    try {
      for (let i = 0; i < order.length;) {
        let j = i + 1;
        while (j < order.length && order[j][0] === order[j - 1][0] + 1) j++;
        const tmp = Buffer.alloc((j - i) * rb);
        fs.readSync(fd, tmp, 0, tmp.length, x.offset + order[i][0] * rb);
        for (let r = i; r < j; r++) tmp.copy(raw, order[r][1] * rb, (r - i) * rb, (r - i + 1) * rb);
        i = j;
      }
    } finally {
      fs.closeSync(fd);
    }
    const out = new Float32Array(ids.length * K), dv = new DataView(raw.buffer, raw.byteOffset, raw.length);
    for (let i = 0; i < ids.length; i++) f.decode(raw, dv, i * rb, K, out, i * K);
    this.stats.readMs += Date.now() - t0;
    return out;
  }
}

/** the earlier name of this host's pack reader: init() = open() */
export class PackStore extends WeightStore {
  async init() { await this.open(); return this; }
}
