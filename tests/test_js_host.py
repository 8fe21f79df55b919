"""The Node.js host (p0pc0rn_amd/js), the reference-shaped boundary, driven through `node`.

CPU: argument errors arrive as thrown Errors with the reference's own texts (engine/llm/lops.js:114-124,
engine/llm/lops_spec.js:163-173, engine/ops/gemm.js:267-278), and opening a device where there is none throws
GpuError. GPU: gemv / gemvM / gemm called with the reference's argument objects agree with the oracle (relative L2
<= 1e-3, BASELINE, and this build's fp32 bar of 2e-5; 1e-5 for the fp32-out GEMM), and the DecodeRunner analogue
(engine/llm/drunner.js) replays a recorded two-op token in both of its modes.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INDEX = "file://" + os.path.join(ROOT, "p0pc0rn_amd", "js", "index.mjs")
NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "p0pc0rn_amd", "js", "p0pc0rn.node")

pytestmark = pytest.mark.skipif(not NODE or not os.path.exists(ADDON), reason="node or the N-API addon is missing")


def run_node(tmp_path, body, timeout=120):
    script = tmp_path / "t.mjs"
    # await_gpu(): the synchronous part of createGpu (Gpu + init), so the test bodies stay linear
    script.write_text("import * as P from '%s';\nimport fs from 'fs';\n"
                      "const await_gpu = () => { const g = new P.Gpu({ device: 0 }); g.init(); return g; };\n%s\n"
                      % (INDEX, body))
    r = subprocess.run([NODE, str(script)], cwd=str(tmp_path), capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout


def test_js_argument_errors_carry_the_reference_texts(tmp_path):
    out = run_node(tmp_path, r"""
const g = {}, B = { ptr: 0 };
const w = (rows, cols) => ({ buf: B, off: 0, enc: 'q4g32a.t64', rows, cols });
const res = [];
const t = (f) => { try { f(); res.push('no error'); } catch (e) { res.push(e.message); } };
t(() => P.gemv(g, { w: w(64, 8192), x: { buf: B }, N: 64, K: 8192, pro: 'raw', epi: 'store', y: { buf: B } }));
t(() => P.gemv(g, { w: w(96, 256), x: { buf: B }, N: 96, K: 256, pro: 'raw', epi: 'store', y: { buf: B } }));
t(() => P.gemv(g, { w: w(64, 4096), x: { buf: B }, N: 64, K: 4096, kPer: 2048, pro: 'rms', epi: 'geglu', y: { buf: B } }));
t(() => P.gemv(g, { w: w(64, 256), x: { buf: B }, N: 64, K: 256, kPer: 48, pro: 'raw', epi: 'store', y: { buf: B } }));
t(() => P.gemv(g, { w: Object.assign(w(64, 256), { off: 2 }), x: { buf: B }, N: 64, K: 256, y: { buf: B } }));
t(() => P.gemvM(g, { w: w(64, 256), x: { buf: B }, M: 2, N: 64, K: 256, pro: 'sum', epi: 'store', y: { buf: B } }));
t(() => P.gemm(g, { w: w(64, 100), x: { buf: B }, M: 4, N: 64, K: 100, y: { buf: B } }));
t(() => P.gemm(g, { w: { buf: B, enc: 'q3', rows: 64, cols: 64 }, x: { buf: B }, M: 4, N: 64, K: 64, y: { buf: B } }));
P.createGpu({ device: 0 }).then(() => res.push('no error'), (e) => res.push((e instanceof P.GpuError ? 'GpuError: ' : '') + e.message))
  .then(() => console.log(JSON.stringify(res)));
""")
    res = json.loads(out.strip().splitlines()[-1])
    assert res[0] == "gemv: K 8192 needs a kPer"
    assert res[1] == "gemv: N % 64"
    assert res[2] == "gemv: geglu needs one split"
    assert res[3] == "gemv: kPer must be a multiple of 32"
    assert res[4] == "gemv: weight offset"
    assert res[5] == "gemvM: prologue sum"
    assert res[6] == "gemm: K must be a multiple of 32"
    assert res[7].startswith("gemm: unsupported weight encoding")
    if not os.path.exists("/dev/kfd"):   # no GPU driver here: opening a device must fail with GpuError
        assert res[8].startswith("GpuError: ") and ("no HIP device" in res[8] or "gfx950" in res[8])


def _save(tmp_path, **arrays):
    for k, v in arrays.items():
        np.ascontiguousarray(v).tofile(str(tmp_path / (k + ".bin")))


@pytest.mark.gpu
def test_js_ops_match_the_oracle(tmp_path):
    N, K, M = 256, 2048, 5
    w, _ = O.pack_q4(O.randn(N * K, 3, 0.05), N, K)
    x = O.randn(M * K, 4)
    nw = np.linspace(0.8, 1.2, K).astype(np.float32)
    st = np.array([0, 0.7, 0, 0.9, 0, 1.1, 0, 0.8, 0, 1.2, 0, 0], np.float32)
    Mg, Ng, Kg = 64, 128, 256
    wg, _ = O.pack_q4(O.randn(Ng * Kg, 5, 0.05), Ng, Kg)
    xg = O.randn(Mg * Kg, 6).astype(np.float16)
    _save(tmp_path, w=w, x=x, nw=nw, st=st, wg=wg, xg=xg)
    run_node(tmp_path, r"""
const g = await_gpu();
const up = (name) => { const b = fs.readFileSync(name + '.bin'); return g.upload(new Uint8Array(b.buffer, b.byteOffset, b.length)); };
const [w, x, nw, st, wg, xg] = ['w', 'x', 'nw', 'st', 'wg', 'xg'].map(up);
const N = 256, K = 2048, M = 5, y1 = g.buffer(N * 4), yM = g.buffer(M * N * 4), yg = g.buffer(64 * 128 * 4);
const W = { buf: w, off: 0, enc: 'q4g32a.t64', rows: N, cols: K };
const ns = P.gemv(g, { w: W, x: { buf: x, rowB: 0 }, N, K, pro: 'rms', epi: 'store', y: { buf: y1 },
                       stat: { buf: st, off: 1 }, norm: { buf: nw, off: 0 } });
const nsM = P.gemvM(g, { w: W, x: { buf: x, ldx: K }, M, N, K, pro: 'rms', epi: 'store', y: { buf: yM, ldm: N },
                         stat: { buf: st, off: 1, ld: 2 }, norm: { buf: nw, off: 0 } });
const fl = P.gemm(g, { w: { buf: wg, off: 0, enc: 'q4g32a.t64', rows: 128, cols: 256 }, x: { buf: xg }, M: 64, N: 128,
                       K: 256, epi: 'f32', y: { buf: yg } });
(async () => {
  await g.done();
  fs.writeFileSync('y1.bin', Buffer.from(await g.read(y1)));
  fs.writeFileSync('yM.bin', Buffer.from(await g.read(yM)));
  fs.writeFileSync('yg.bin', Buffer.from(await g.read(yg)));
  console.log(JSON.stringify({ ns, nsM, fl }));
  g.freeAll(); g.device.destroy();
})();
""")
    y1 = np.fromfile(str(tmp_path / "y1.bin"), np.float32)
    yM = np.fromfile(str(tmp_path / "yM.bin"), np.float32)
    yg = np.fromfile(str(tmp_path / "yg.bin"), np.float32)
    want1 = np.zeros(N, np.float32)
    O.q4_gemv(capi.gemv_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, N=N, K=K, pro=capi.PRO["rms"],
                             y=want1.ctypes.data, stat=st.ctypes.data, stat_off=1, norm=nw.ctypes.data))
    wantM = np.zeros(M * N, np.float32)
    O.q4_gemvM(capi.gemvm_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, x_ldx=K, M=M, N=N, K=K,
                               pro=capi.PRO["rms"], y=wantM.ctypes.data, y_ldm=N, stat=st.ctypes.data, stat_off=1,
                               stat_ld=2, norm=nw.ctypes.data))
    wantg = np.zeros(Mg * Ng, np.float32)
    O.q4_gemm(capi.gemm_args(w=wg.ctypes.data, w_rows=Ng, w_cols=Kg, x=xg.ctypes.data, M=Mg, N=Ng, K=Kg,
                             epi=capi.GEPI["f32"], y=wantg.ctypes.data))
    for got, want, tol, what in ((y1, want1, 2e-5, "gemv"), (yM, wantM, 2e-5, "gemvM"), (yg, wantg, 1e-5, "gemm")):
        r = rel_l2(got, want)
        print(what, r)
        assert np.all(np.isfinite(got)) and r <= 1e-3 and r <= tol, what


@pytest.mark.gpu
@pytest.mark.parametrize("mode,enc2", [("graph", "q4"), ("chain", "q4"), ("graph", "q8"), ("chain", "q8")])
def test_js_decode_runner(tmp_path, mode, enc2):
    """a token of two dependent GEMVs (y1 = W1 x; y2 = W2 y1), recorded once and submitted three times; W2 in either
    encoding (a balanced 4/8-bit pack mixes them in one token)"""
    N1, K1, N2 = 512, 1024, 256
    w1, _ = O.pack_q4(O.randn(N1 * K1, 7, 0.05), N1, K1)
    w2, _ = (O.pack_q4 if enc2 == "q4" else O.pack_q8)(O.randn(N2 * N1, 8, 0.05), N2, N1)
    x = O.randn(K1, 9)
    _save(tmp_path, w1=w1, w2=w2, x=x)
    out = run_node(tmp_path, r"""
const g = await_gpu();
const up = (name) => { const b = fs.readFileSync(name + '.bin'); return g.upload(new Uint8Array(b.buffer, b.byteOffset, b.length)); };
const [w1, w2, x] = ['w1', 'w2', 'x'].map(up);
const y1 = g.buffer(512 * 4), y2 = g.buffer(256 * 4);
const r = new P.DecodeRunner(g, { mode: '%s', reuse: true });
r.begin(0);
P.gemv(g, { w: { buf: w1, off: 0, enc: 'q4g32a.t64', rows: 512, cols: 1024 }, x: { buf: x }, N: 512, K: 1024, y: { buf: y1 } });
P.gemv(g, { w: { buf: w2, off: 0, enc: '%s', rows: 256, cols: 512 }, x: { buf: y1 }, N: 256, K: 512, y: { buf: y2 } });
const tk = r.end(y2, 16);
(async () => {
  const outs = [];
  for (let i = 0; i < 3; i++) {
    g.fill(y1, 0, 0x7fc00000, 512); g.fill(y2, 0, 0x7fc00000, 256);
    const o32 = await r.submit(tk);   // the token's first four result words, through the parity's staging buffer
    const y = Buffer.from(await g.read(y2));
    if (Buffer.compare(Buffer.from(o32.buffer, o32.byteOffset, 16), y.subarray(0, 16)) !== 0) throw new Error('stage');
    outs.push(y.toString('base64'));
  }
  fs.writeFileSync('y1.bin', Buffer.from(await g.read(y1)));
  fs.writeFileSync('y2.bin', Buffer.from(await g.read(y2)));
  console.log(JSON.stringify({ same: outs.every((o) => o === outs[0]), submits: r.submits, dispatches: r.dispatches }));
  r.forget();
  let released = '';
  try { await r.submit(tk); } catch (e) { released = e.message; }
  if (!released.includes('released')) throw new Error('a forgotten token must not run: ' + released);
  await r.destroy(); g.freeAll(); g.device.destroy();
})();
""" % (mode, "q4g32a.t64" if enc2 == "q4" else "q8g64s.t64"))
    res = json.loads(out.strip().splitlines()[-1])
    assert res["same"] and res["submits"] == 3
    assert res["dispatches"] == 3   # 2 GEMVs + the result copy (graph: 3 launches; chain: 3 ops of one launch)
    y1 = np.fromfile(str(tmp_path / "y1.bin"), np.float32)
    y2 = np.fromfile(str(tmp_path / "y2.bin"), np.float32)
    want1 = np.zeros(N1, np.float32)
    O.q4_gemv(capi.gemv_args(w=w1.ctypes.data, w_rows=N1, w_cols=K1, x=x.ctypes.data, N=N1, K=K1, y=want1.ctypes.data))
    want2 = np.zeros(N2, np.float32)
    O.q4_gemv(capi.gemv_args(w=w2.ctypes.data, w_enc=1 if enc2 == "q4" else 2, w_rows=N2, w_cols=N1, x=y1.ctypes.data,
                             N=N2, K=N1, y=want2.ctypes.data))
    for got, want, what in ((y1, want1, "op 0"), (y2, want2, "op 1")):
        r = rel_l2(got, want)
        assert np.all(np.isfinite(got)) and r <= 2e-5, (mode, what, r)


@pytest.mark.gpu
def test_js_rowstats_normadd_argmax(tmp_path):
    """rowstats(gpu, a), normadd(g, a), argmax(g, a) and argmaxM(g, a) with the reference's argument objects
    (engine/ops/misc.js:33-40, engine/llm/lops.js:172-178 and 434-436, engine/llm/lops_spec.js:346-348), bit-exact
    against the oracle"""
    rows, cols, D, M, n = 3, 2048, 2048, 2, 300
    xs = (1.0 + O.randn(rows * cols, 91)).astype(np.float32)
    t = O.randn(4 * M * D, 92, 0.3).astype(np.float32)
    w = (0.5 + O.rng_uniform(93, D)).astype(np.float32)
    x0 = O.randn(M * D, 94).astype(np.float32)
    rng = np.random.default_rng(95)
    mx = np.zeros(2 * n * M, np.float32)
    mx[0::2] = rng.integers(-9, 9, n * M).astype(np.float32)
    mx[1::2] = np.tile(np.arange(n, dtype=np.uint32) * 64, M).view(np.float32)
    _save(tmp_path, xs=xs, t=t, w=w, x0=x0, mx=mx)
    run_node(tmp_path, r"""
const g = await_gpu();
const up = (name) => { const b = fs.readFileSync(name + '.bin'); return g.upload(new Uint8Array(b.buffer, b.byteOffset, b.length)); };
const [xs, t, w, x0, mx] = ['xs', 't', 'w', 'x0', 'mx'].map(up);
const st = g.buffer(2 * 3 * 4), sn = g.buffer(2 * 4), o1 = g.buffer(8), oM = g.buffer(16);
P.rowstats(g, { x: { buf: xs, off: 0, ld: 2048 }, rows: 3, cols: 2048, mode: 'ln', eps: 1e-5, st: { buf: st, off: 0 } });
P.normadd(g, { t: { buf: t, n: 4, ld: 2 * 2048 }, w: { buf: w, off: 0 }, x: { buf: x0 }, st: { buf: sn, off: 0 },
               D: 2048, M: 2, scale: 0.5 });
P.argmax(g, { mx: { buf: mx }, n: 300, out: { buf: o1 } });
P.argmaxM(g, { mx: { buf: mx }, n: 300, M: 2, out: { buf: oM } });
(async () => {
  await g.done();
  for (const [name, b] of [['st', st], ['x', x0], ['sn', sn], ['o1', o1], ['oM', oM]])
    fs.writeFileSync(name + '.out', Buffer.from(await g.read(b)));
  console.log('ok');
  g.freeAll(); g.device.destroy();
})();
""")
    # buffers are rounded up to 16 bytes (Gpu.buffer): read back only the values
    rd = lambda name, dt, k: np.fromfile(str(tmp_path / (name + ".out")), dt)[:k]
    want_st = np.zeros(6, np.float32)
    O.rowstats(capi.rowstats_args(x=xs.ctypes.data, x_ld=cols, rows=rows, cols=cols, mode=0, eps=1e-5,
                                  st=want_st.ctypes.data))
    assert np.array_equal(rd("st", np.uint32, 6), want_st.view(np.uint32))
    xw, sw = x0.copy(), np.zeros(M, np.float32)
    O.normadd(capi.normadd_args(t=t.ctypes.data, t_n=4, t_ld=M * D, w=w.ctypes.data, x=xw.ctypes.data,
                                st=sw.ctypes.data, D=D, M=M, eps=1e-6, scale=0.5, mode=0))
    assert np.array_equal(rd("x", np.uint32, M * D), xw.view(np.uint32))
    assert np.array_equal(rd("sn", np.uint32, M), sw.view(np.uint32))
    assert np.array_equal(rd("o1", np.uint32, 2), O.argmaxM(mx, n, 1))
    assert np.array_equal(rd("oM", np.uint32, 2 * M), O.argmaxM(mx, n, M))


# ------------------------------------------------------------------------------------------------ PackStore
def make_pack(root):
    """A small pack directory in the reference's layout (engine/core/store.js): manifest.json + two shard files.
    Shard "blk": a q4g32a.t64 weight [128][256] and a q8g64s.t64 weight [128][256] (the oracle's packers), each at a
    256-aligned offset; shard "emb": a q4g32a.rows table [10][64] (per row: 32 code bytes, then 2 x (f16 scale, f16
    min)) and a q8g64s.rows table [6][128] (per row: 128 int8 codes, then 2 f16 scales). Returns the expected
    dequantised rows and the weight records."""
    rng = np.random.default_rng(5)
    wq4, _ = O.pack_q4(O.randn(128 * 256, 21, 0.05), 128, 256)
    wq8, _ = O.pack_q8(O.randn(128 * 256, 22, 0.05), 128, 256)
    blk = bytearray(wq4.tobytes())
    blk += b"\0" * ((-len(blk)) % 256)
    off8 = len(blk)
    blk += wq8.tobytes()
    # q4 rows: codes in [0, 16), fp16 scale > 0 and min; the value is fl32(q s + m)
    q4c = rng.integers(0, 16, (10, 64)).astype(np.uint8)
    q4s = np.abs(rng.standard_normal((10, 2))).astype(np.float16) * np.float16(0.05)
    q4m = (-8 * q4s.astype(np.float32)).astype(np.float16)
    rows4 = bytearray()
    want4 = np.zeros((10, 64), np.float32)
    for r in range(10):
        rows4 += (q4c[r, 0::2] | (q4c[r, 1::2] << 4)).astype(np.uint8).tobytes()
        for g in range(2):
            rows4 += q4s[r, g].tobytes() + q4m[r, g].tobytes()
            want4[r, 32 * g:32 * g + 32] = (q4c[r, 32 * g:32 * g + 32].astype(np.float64) * float(q4s[r, g])
                                            + float(q4m[r, g])).astype(np.float32)
    q8c = rng.integers(-128, 128, (6, 128)).astype(np.int8)
    q8s = np.abs(rng.standard_normal((6, 2))).astype(np.float16) * np.float16(0.01)
    rows8 = bytearray()
    want8 = np.zeros((6, 128), np.float32)
    for r in range(6):
        rows8 += q8c[r].tobytes() + q8s[r].tobytes()
        for g in range(2):
            want8[r, 64 * g:64 * g + 64] = (q8c[r, 64 * g:64 * g + 64].astype(np.float64) * float(q8s[r, g])).astype(np.float32)
    emb = bytes(rows4) + bytes(rows8)
    (root / "blk.bin").write_bytes(bytes(blk))
    (root / "emb.bin").write_bytes(emb)
    manifest = {
        "format": "pocketflux.pack", "format_version": 1, "pack_version": "test-1",
        "shards": [{"name": "blk", "file": "blk.bin", "bytes": len(blk)}, {"name": "emb", "file": "emb.bin", "bytes": len(emb)}],
        "tensors": {
            "w.q4": {"shard": "blk", "offset": 0, "bytes": wq4.nbytes, "enc": "q4g32a.t64", "shape": [128, 256]},
            "w.q8": {"shard": "blk", "offset": off8, "bytes": wq8.nbytes, "enc": "q8g64s.t64", "shape": [128, 256]},
            "emb.q4": {"shard": "emb", "offset": 0, "bytes": len(rows4), "enc": "q4g32a.rows", "shape": [10, 64]},
            "emb.q8": {"shard": "emb", "offset": len(rows4), "bytes": len(rows8), "enc": "q8g64s.rows", "shape": [6, 128]},
        },
    }
    (root / "manifest.json").write_text(json.dumps(manifest))
    return {"want4": want4, "want8": want8, "wq4": wq4, "wq8": wq8}


def test_js_packstore_rows_files_and_errors(tmp_path):
    """PackStore on the CPU: manifest, readRows of both row encodings (engine/core/store.js:275-301), readFile, and
    the reference's error texts"""
    pk = tmp_path / "pack"
    pk.mkdir()
    exp = make_pack(pk)
    out = run_node(tmp_path, r"""
const st = new P.PackStore({}, { dir: 'pack' });
(async () => {
  await st.init();
  const r4 = await st.readRows('emb.q4', [3, 0, 9]), r8 = await st.readRows('emb.q8', [5, 1]);
  fs.writeFileSync('r4.bin', Buffer.from(r4.buffer)); fs.writeFileSync('r8.bin', Buffer.from(r8.buffer));
  const f = await st.readFile('emb');
  const res = [f.byteLength];
  const t = async (fn) => { try { await fn(); res.push('no error'); } catch (e) { res.push(e.message); } };
  await t(() => st.upload('nope'));
  await t(() => st.readRows('w.q4', [0]));
  await t(() => st.uploadPart('emb', ['w.q4']));
  console.log(JSON.stringify(res));
})();
""")
    res = json.loads(out.strip().splitlines()[-1])
    r4 = np.fromfile(str(tmp_path / "r4.bin"), np.float32).reshape(3, 64)
    r8 = np.fromfile(str(tmp_path / "r8.bin"), np.float32).reshape(2, 128)
    assert np.array_equal(r4, exp["want4"][[3, 0, 9]]) and np.array_equal(r8, exp["want8"][[5, 1]])
    assert res[0] == (pk / "emb.bin").stat().st_size
    assert res[1] == "unknown shard nope"
    assert res[2] == "readRows: q4g32a.t64"
    assert res[3] == "tensor w.q4 not in emb"


@pytest.mark.gpu
def test_js_packstore_upload_feeds_the_ops(tmp_path):
    """a shard uploaded whole and a part upload both give tensor views that gemv reads as the reference's a.w"""
    pk = tmp_path / "pack"
    pk.mkdir()
    exp = make_pack(pk)
    x = O.randn(256, 23)
    _save(tmp_path, x=x)
    run_node(tmp_path, r"""
const g = await_gpu();
const b = fs.readFileSync('x.bin'), x = g.upload(new Uint8Array(b.buffer, b.byteOffset, b.length));
const st = new P.PackStore(g, { dir: 'pack' });
(async () => {
  await st.init();
  const h = await st.upload('blk'), part = await st.uploadPart('blk', ['w.q8']);
  const outs = { q4: g.buffer(128 * 4), q8: g.buffer(128 * 4), q8p: g.buffer(128 * 4) };
  P.gemv(g, { w: h.t('w.q4'), x: { buf: x }, N: 128, K: 256, y: { buf: outs.q4 } });
  P.gemv(g, { w: h.t('w.q8'), x: { buf: x }, N: 128, K: 256, y: { buf: outs.q8 } });
  P.gemv(g, { w: part.t('w.q8'), x: { buf: x }, N: 128, K: 256, y: { buf: outs.q8p } });
  await g.done();
  for (const k of Object.keys(outs)) fs.writeFileSync(k + '.out', Buffer.from(await g.read(outs[k], 0, 512)));
  st.release(h); st.release(part);
  console.log('ok');
  g.freeAll(); g.device.destroy();
})();
""")
    for key, w, enc in (("q4", exp["wq4"], 1), ("q8", exp["wq8"], 2), ("q8p", exp["wq8"], 2)):
        got = np.fromfile(str(tmp_path / (key + ".out")), np.float32)
        want = np.zeros(128, np.float32)
        O.q4_gemv(capi.gemv_args(w=w.ctypes.data, w_enc=enc, w_rows=128, w_cols=256, x=x.ctypes.data, N=128, K=256,
                                 y=want.ctypes.data))
        assert rel_l2(got, want) <= 2e-5, key


def test_js_pick_surface_and_v5_errors(tmp_path):
    """engine/llm/lopsx.js:225-328: kxPick follows PICK, setPicks overrides it (a non-object value = the engine's own
    kernel), setKX(false) turns picks off, okV5 needs a 4-bit weight at a 16-byte offset with K % 32 == 0; the v5
    entry points refuse what the reference's v5 path refuses, with its texts, before any device call."""
    out = run_node(tmp_path, r"""
const g = {}, B = { ptr: 0 };
const w = (rows, cols, off = 0, enc = 'q4g32a.t64') => ({ buf: B, off, enc, rows, cols });
const a = (N, K, pro, epi, extra = {}) => Object.assign({ w: w(N, K), x: { buf: B }, N, K, pro, epi, y: { buf: B } }, extra);
const r = {};
r.nPick = Object.keys(P.PICK).length;
r.head = P.kxPick(a(262144, 1536, 'rms', 'softcap'));
r.e2b = P.kxPick(a(8192, 2048, 'rms', 'geglu'));
r.off8 = P.kxPick(Object.assign(a(262144, 1536, 'rms', 'softcap'), { w: w(262144, 1536, 8) }));
r.q8 = P.kxPick(Object.assign(a(262144, 1536, 'rms', 'softcap'), { w: w(262144, 1536, 0, 'q8g64s.t64') }));
P.setPicks({ 'rms.geglu.8192x2048': { ND: 2, L: 16 }, 'rms.softcap.262144x1536': 'engine' });
r.over = P.kxPick(a(8192, 2048, 'rms', 'geglu'));
r.engine = P.kxPick(a(262144, 1536, 'rms', 'softcap'));
r.kept = P.kxPick(a(1536, 6144, 'raw', 'store'));
r.now = P.picksNow();
P.setKX(false); r.off = P.kxPick(a(1536, 6144, 'raw', 'store')); P.setKX(true);
P.setPicks(null); r.reset = P.kxPick(a(262144, 1536, 'rms', 'softcap')); r.nowNull = P.picksNow();
r.direct = [P.directOkV5({ x: { rowB: 8 }, K: 64 }), P.directOkV5({ x: { rowB: 6 }, K: 64 }),
            P.directOkV5({ x: { ldx: 66 }, K: 64 }), P.directOkV5({ x: {}, K: 64, norm: { off: 2 } })];
r.u8 = P.u8ok(); r.needs = P.DIRECT_NEEDS; r.ver = P.KERNEL_VERSION;
const errs = [];
const t = (f) => { try { f(); errs.push('no error'); } catch (e) { errs.push(e.message); } };
t(() => P.gemvV5(g, Object.assign(a(64, 256, 'raw', 'store'), { w: w(64, 256, 4) })));
t(() => P.gemvV5(g, a(64, 256, 'raw', 'store'), { ND: 1, L: 16 }));
t(() => P.gemvV5(g, a(64, 4096, 'raw', 'store')));
t(() => P.gemvV5(g, a(64, 4096, 'rms', 'geglu', { kPer: 2048 })));
t(() => P.gemvV5(g, a(96, 256, 'raw', 'store')));
t(() => P.gemvV5(g, a(64, 256, 'raw', 'store', { kPer: 48 })));
t(() => P.gemvMV5(g, a(64, 8192, 'rms', 'softcap', { M: 2, kPer: 4096 })));
t(() => P.gemvMV5(g, a(96, 256, 'raw', 'store', { M: 2 })));
t(() => P.v5code({ M: 1 }));
r.errs = errs;
console.log(JSON.stringify(r));
""")
    r = json.loads(out.strip().splitlines()[-1])
    assert r["nPick"] == 17
    assert r["head"] == {"ND": 4, "L": 16, "deq": "mask"}
    assert r["e2b"] is None and r["off8"] is None and r["q8"] is None   # not a key / not okV5
    assert r["over"] == {"ND": 2, "L": 16} and r["engine"] is None
    assert r["kept"] == {"ND": 4, "L": 16, "mode": "direct"}
    assert r["now"] == {"rms.geglu.8192x2048": {"ND": 2, "L": 16}, "rms.softcap.262144x1536": "engine"}
    assert r["off"] is None and r["reset"] == {"ND": 4, "L": 16, "deq": "mask"} and r["nowNull"] is None
    assert r["direct"] == [True, False, False, False]
    assert r["u8"] is False and r["needs"] == {"gemv": 9, "gemvM": 10} and r["ver"] == "mi355x-hip-1"
    assert r["errs"] == [
        "kernx v5: not a 4-bit, 16-byte aligned, K % 32 weight",
        "kernx v5: 1024 threads",
        "kernx v5: K 4096 needs a kPer",
        "kernx v5: geglu needs one split",
        "kernx v5: N % 64",
        "kernx v5: kPer must be a multiple of 32",
        "kernx v5: softcap needs one split",
        "kernx v5: N % 64",
        'kernx v5: no WGSL on the HIP backend (config {"M":1})',
    ]


@pytest.mark.gpu
def test_js_v5_entry_points_match_gemv(tmp_path):
    """gemvV5 / gemvMV5 with the reference's pick options run the same kernels as gemv / gemvM: the same split count
    and the same bits, and those agree with the oracle (2e-5 relative L2, inside BASELINE's 1e-3)."""
    N, K, M = 1536, 6144, 3
    w, _ = O.pack_q4(O.randn(N * K, 21, 0.05), N, K)
    x = O.randn(M * K, 22)
    _save(tmp_path, w=w, x=x)
    out = run_node(tmp_path, r"""
const g = await_gpu();
const up = (name) => { const b = fs.readFileSync(name + '.bin'); return g.upload(new Uint8Array(b.buffer, b.byteOffset, b.length)); };
const [w, x] = ['w', 'x'].map(up);
const N = 1536, K = 6144, M = 3, kPer = 2048;
const W = { buf: w, off: 0, enc: 'q4g32a.t64', rows: N, cols: K };
const ys = [0, 1, 2, 3].map(() => g.buffer(M * N * 3 * 4));
const a1 = (y) => ({ w: W, x: { buf: x, rowB: 0 }, N, K, kPer, pro: 'raw', epi: 'store', y: { buf: y } });
const aM = (y) => ({ w: W, x: { buf: x, ldx: K }, M, N, K, kPer, pro: 'raw', epi: 'store', y: { buf: y, ldm: N } });
const pick = P.kxPick(a1(ys[0]));
const ns = [P.gemv(g, a1(ys[0])), P.gemvV5(g, a1(ys[1]), pick), P.gemvM(g, aM(ys[2])), P.gemvMV5(g, aM(ys[3]), pick)];
(async () => {
  await g.done();
  for (let i = 0; i < 4; ++i) fs.writeFileSync('y' + i + '.bin', Buffer.from(await g.read(ys[i])));
  console.log(JSON.stringify({ ns, pick }));
  g.freeAll(); g.device.destroy();
})();
""")
    r = json.loads(out.strip().splitlines()[-1])
    assert r["pick"] == {"ND": 4, "L": 16, "mode": "direct"} and r["ns"] == [3, 3, 3, 3]
    y = [np.fromfile(str(tmp_path / ("y%d.bin" % i)), np.float32) for i in range(4)]
    n1, nM = 3 * N, 3 * M * N
    assert np.array_equal(y[0][:n1], y[1][:n1]) and np.array_equal(y[2][:nM], y[3][:nM])
    want = np.zeros(3 * M * N, np.float32)
    O.q4_gemvM(capi.gemvm_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, x_ldx=K, M=M, N=N, K=K,
                               kPer=2048, y=want.ctypes.data, y_ldm=N))
    r2 = rel_l2(y[3][:nM], want)
    print("gemvMV5", r2)
    assert np.all(np.isfinite(y[3][:nM])) and r2 <= 2e-5


# ------------------------------------------------------------------------------------------------ DecodeRunner contract
@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["graph", "chain"])
def test_js_decode_loop_gemma4_shaped(tmp_path, mode):
    """engine/llm/gemma4.js:547-590's overlapped loop, unchanged in shape: token i is recorded with begin(parity) ...
    end(argBuf), submitted once its input is written, and `o32 = await pend; o32[0]` is the next id. A token is
    x = table[id] (written by the host before the submit, as the loop writes s.pler), h = W1 x' (rms), logits =
    softcap(W2 h') (rms) with per-tile maxima, then the argmax over the tiles into the result words, which end() copies
    to the parity's staging buffer: in graph mode four recorded launches, in chain mode one launch of four chain ops.
    Three tokens; each id must be the oracle's."""
    D, H, V = 256, 512, 1024
    w1, _ = O.pack_q4(O.randn(H * D, 41, 0.05), H, D)
    w2, _ = O.pack_q4(O.randn(V * H, 42, 0.05), V, H)
    table = O.randn(V * D, 43).reshape(V, D)
    nw1 = np.linspace(0.8, 1.2, D).astype(np.float32)
    nw2 = np.linspace(1.1, 0.9, H).astype(np.float32)
    _save(tmp_path, w1=w1, w2=w2, table=table, nw1=nw1, nw2=nw2)
    out = run_node(tmp_path, r"""
const g = await_gpu();
const up = (name) => { const b = fs.readFileSync(name + '.bin'); return g.upload(new Uint8Array(b.buffer, b.byteOffset, b.length)); };
const [w1, w2, nw1, nw2] = ['w1', 'w2', 'nw1', 'nw2'].map(up);
const tb = fs.readFileSync('table.bin'), table = new Float32Array(tb.buffer, tb.byteOffset, tb.length / 4);
const D = 256, H = 512, V = 1024, mode = '%s';
const s = { x: g.buffer(D * 4), h: g.buffer(H * 4), logits: g.buffer(V * 4), st: g.buffer(16),
            mx: g.buffer((V / 64 + 1) * 8), arg: g.buffer(16) };
g.upload(new Float32Array([0, 1, 0, 1]), '', s.st);          // rstd slots: the rms prologues read 1
g.upload(new Float32Array([1]), '', s.mx, (V / 64) * 8 + 4);  // the head's rstd lives past the tile maxima
const encodeStep = () => {
  P.gemv(g, { w: { buf: w1, off: 0, enc: 'q4g32a.t64', rows: H, cols: D }, x: { buf: s.x, rowB: 0 }, N: H, K: D,
              pro: 'rms', stat: { buf: s.st, off: 1 }, norm: { buf: nw1, off: 0 }, y: { buf: s.h } });
  P.gemv(g, { w: { buf: w2, off: 0, enc: 'q4g32a.t64', rows: V, cols: H }, x: { buf: s.h, rowB: 0 }, N: V, K: H,
              pro: 'rms', stat: { buf: s.mx, off: (V / 64) * 2 + 1 }, norm: { buf: nw2, off: 0 }, epi: 'softcap',
              cap: 30, mx: { buf: s.mx }, y: { buf: s.logits } });
  P.argmax(g, { mx: { buf: s.mx }, n: V / 64, out: { buf: s.arg } });
  return s.arg;
};
const core = g.runner, dr = new P.DecodeRunner(g, { mode });
const rec = (pos, parity) => { g.runner = dr; try { dr.begin(parity); const ob = encodeStep(pos); return dr.end(ob); } finally { g.runner = core; if (dr.cur) dr.cur = null; } };
const ids = [], words = [];
let pend = null, tk = null;
const feed = async (id, i) => {
  if (!tk) tk = rec(i, i & 1);
  g.upload(table.subarray(id * D, (id + 1) * D), '', s.x);
  pend = dr.submit(tk); tk = null;
};
(async () => {
  await feed(7, 0);
  tk = rec(1, 1);
  for (let i = 0; i < 3; i++) {
    const o32 = await pend; pend = null;
    const idx = o32[0], bits = o32[1];   // the argmax words [index, max bits]
    words.push([idx, bits]);
    const nxt = idx;
    ids.push(nxt);
    if (i + 1 < 3) await feed(nxt, i + 1);
    if (i + 2 < 3) tk = rec(i + 2, i & 1);
  }
  await dr.destroy();
  console.log(JSON.stringify({ ids, words, submits: dr.submits, dispatches: dr.dispatches }));
  g.freeAll(); g.device.destroy();
})();
""" % mode)
    res = json.loads(out.strip().splitlines()[-1])
    assert res["submits"] == 3
    st_mx = np.zeros((V // 64 + 1) * 2, np.float32)
    st_mx[(V // 64) * 2 + 1] = 1.0
    st = np.array([0, 1, 0, 1], np.float32)
    cur = 7
    for i in range(3):
        x = np.ascontiguousarray(table[cur])
        h = np.zeros(H, np.float32)
        O.q4_gemv(capi.gemv_args(w=w1.ctypes.data, w_rows=H, w_cols=D, x=x.ctypes.data, N=H, K=D, pro=capi.PRO["rms"],
                                 y=h.ctypes.data, stat=st.ctypes.data, stat_off=1, norm=nw1.ctypes.data))
        lg = np.zeros(V, np.float32)
        mx = st_mx.copy()
        O.q4_gemv(capi.gemv_args(w=w2.ctypes.data, w_rows=V, w_cols=H, x=h.ctypes.data, N=V, K=H,
                                 pro=capi.PRO["rms"], epi=capi.EPI["softcap"], y=lg.ctypes.data, mx=mx.ctypes.data,
                                 stat_off=(V // 64) * 2 + 1, norm=nw2.ctypes.data, cap=30.0))
        idx = int(np.argmax(lg))
        val = lg[idx]
        nxt = idx
        got_idx, got_bits = res["words"][i]
        assert got_idx == idx, (i, got_idx, idx)
        assert abs(np.uint32(got_bits).view(np.float32) - val) <= 1e-4 * max(1.0, abs(val))
        assert res["ids"][i] == nxt
        cur = nxt
    assert res["dispatches"] == 3 * 4   # 2 GEMVs + argmax + the result copy (launches, or ops of one chain launch)


def test_js_fp16_helpers_exhaustive(tmp_path):
    """the host's f2h / h2f (p0pc0rn_amd/js/core/gpu.mjs, the reference's CPU helpers engine/core/gpu.js:273-297):
    h2f over all 65536 patterns and f2h over random f32 bit patterns, every half value, every midpoint between
    neighbouring halves (ties to even) and the f32 neighbours of those midpoints, against numpy's IEEE binary16 RNE"""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(11)
    halves = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    vals = [rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
            halves.astype(np.float32), mids, np.nextafter(mids, np.float32(np.inf)),
            np.nextafter(mids, np.float32(-np.inf)),
            np.float32([65504, 65519, 65519.996, 65520, 65536, 1e9, np.inf, -np.inf, 0.0, -0.0, 2 ** -24, 2 ** -25,
                        1.5 * 2 ** -25, 2 ** -26, 6.1e-5, -6.1e-5])]
    f = np.concatenate([v.astype(np.float32) for v in vals])
    f = np.concatenate([f, -f])
    _save(tmp_path, h=h, f=f)
    run_node(tmp_path, r"""
const hb = fs.readFileSync('h.bin'), fb = fs.readFileSync('f.bin');
const H = new Uint16Array(hb.buffer, hb.byteOffset, hb.length / 2), F = new Float32Array(fb.buffer, fb.byteOffset, fb.length / 4);
const ho = new Float64Array(H.length), fo = new Uint16Array(F.length);
for (let i = 0; i < H.length; i++) ho[i] = P.h2f(H[i]);
for (let i = 0; i < F.length; i++) fo[i] = P.f2h(F[i]);
fs.writeFileSync('ho.bin', Buffer.from(ho.buffer)); fs.writeFileSync('fo.bin', Buffer.from(fo.buffer));
console.log('ok');
""")
    ho = np.fromfile(str(tmp_path / "ho.bin"), np.float64)
    want_h = h.view(np.float16).astype(np.float64)
    nan = np.isnan(want_h)
    assert np.array_equal(np.isnan(ho), nan) and np.array_equal(ho[~nan], want_h[~nan])
    assert np.array_equal(np.signbit(ho[~nan]), np.signbit(want_h[~nan]))   # -0 stays -0
    fo = np.fromfile(str(tmp_path / "fo.bin"), np.uint16)
    fn = np.isnan(f)
    assert np.array_equal(fo[~fn], f[~fn].astype(np.float16).view(np.uint16))
    assert np.all(fo[fn] == 0x7e00)


def test_js_weightstore_open_status_and_errors(tmp_path):
    """WeightStore (engine/core/store.js:50-115): open() reads and checks the manifest with the reference's texts,
    status() / download() report a missing shard, readRows takes unsorted and repeated ids, PackStore.init = open"""
    pk = tmp_path / "pack"
    pk.mkdir()
    exp = make_pack(pk)
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "manifest.json").write_text(json.dumps({"format": "other", "format_version": 2, "shards": [], "tensors": {}}))
    out = run_node(tmp_path, r"""
(async () => {
  const res = [];
  const t = async (fn) => { try { await fn(); res.push('no error'); } catch (e) { res.push(e.message); } };
  await t(() => new P.WeightStore({}, { base: 'nowhere' }).open());
  await t(() => new P.WeightStore({}, { base: 'bad' }).open());
  const st = new P.WeightStore({}, { base: 'pack' });
  const m = await st.open();
  res.push(m.pack_version, JSON.stringify(st.status()));
  const r4 = await st.readRows('emb.q4', [9, 3, 3, 4, 0]);
  fs.writeFileSync('r4.bin', Buffer.from(r4.buffer));
  fs.truncateSync('pack/emb.bin', 10);
  const s2 = st.status();
  res.push(s2.complete, s2.missing.join(','));
  await t(() => st.download());
  const ps = await new P.PackStore({}, { dir: 'pack' }).init();
  res.push(ps.m.pack_version);
  console.log(JSON.stringify(res));
})();
""")
    res = json.loads(out.strip().splitlines()[-1])
    assert res[0] == "pack manifest unavailable (offline and not downloaded)"
    assert res[1] == "unsupported pack format other/2"
    assert res[2] == "test-1"
    st = json.loads(res[3])
    assert st["complete"] and st["missing"] == [] and st["have"] == st["total"]
    r4 = np.fromfile(str(tmp_path / "r4.bin"), np.float32).reshape(5, 64)
    assert np.array_equal(r4, exp["want4"][[9, 3, 3, 4, 0]])
    assert res[4] is False and res[5] == "emb"
    assert res[6] == "download: no network source; the pack directory lacks emb"
    assert res[7] == "test-1"


def test_js_view_bounds_and_unsupported_options(tmp_path):
    """views are checked against their buffers on the host (a handle with _pf), and the options this build does not
    have are refused with an Error instead of running something else"""
    out = run_node(tmp_path, r"""
const buf = (n) => ({ ptr: 0, _pf: n });
const res = [];
const t = (f) => { try { f(); res.push('no error'); } catch (e) { res.push(e.message); } };
const W = (rows, cols, b) => ({ buf: b || buf(rows / 64 * cols / 32 * 1280), off: 0, enc: 'q4g32a.t64', rows, cols });
t(() => P.gemv({}, { w: W(128, 256), x: { buf: buf(255 * 4) }, N: 128, K: 256, y: { buf: buf(512) } }));
t(() => P.gemv({}, { w: W(128, 256), x: { buf: buf(1024) }, N: 128, K: 256, y: { buf: buf(511) } }));
t(() => P.gemv({}, { w: W(128, 256, buf(1000)), x: { buf: buf(1024) }, N: 128, K: 256, y: { buf: buf(512) } }));
t(() => P.gemvM({}, { w: W(128, 256), x: { buf: buf(1024 * 3 - 4), ldx: 256 }, M: 3, N: 128, K: 256, y: { buf: buf(1536) } }));
t(() => P.gemm({}, { w: W(128, 256), x: { buf: buf(4 * 256 * 2 - 2) }, M: 4, N: 128, K: 256, y: { buf: buf(1024) } }));
t(() => P.gemm({}, { w: W(128, 256), x: { buf: buf(2048) }, M: 4, N: 128, K: 256, epi: 'f32', y: { buf: buf(2047) } }));
t(() => P.gemm({}, { w: W(128, 256), x: { buf: buf(2048) }, M: 4, N: 128, K: 256, acc: 'f16', y: { buf: buf(1024) } }));
t(() => P.gemm({}, { w: W(128, 256), x: { buf: buf(2048) }, M: 4, N: 128, K: 256, epi: 'onormgate', y: { buf: buf(1024) } }));
t(() => P.gemm({}, { w: W(256, 256), x: { buf: buf(2048) }, M: 4, N: 256, K: 256, epi: 'heads', y: { buf: buf(4096) },
                     ev: { buf: buf(1024) }, heads: { Ltot: 4, Hq: 1, Hkv: 0, ropeMode: 'inter', rope: { buf: buf(2047) } } }));
t(() => P.gemm({}, { w: W(256, 256), x: { buf: buf(2048) }, M: 4, N: 256, K: 256, epi: 'heads', y: { buf: buf(4096) },
                     heads: { Ltot: 4, ropeMode: 'sideways' } }));
console.log(JSON.stringify(res));
""")
    res = json.loads(out.strip().splitlines()[-1])
    assert res[0] == "gemv: x needs 1024 B of a 1020 B buffer"
    assert res[1] == "gemv: y needs 512 B of a 511 B buffer"
    assert res[2] == "gemv: w needs 20480 B of a 1000 B buffer"
    assert res[3] == "gemvM: x needs 3072 B of a 3068 B buffer"
    assert res[4] == "gemm: x needs 2048 B of a 2046 B buffer"
    assert res[5] == "gemm: y needs 2048 B of a 2047 B buffer"
    assert res[6] == "gemm: acc f16 is not part of this build (it accumulates in fp32)"
    assert res[7] == "gemm: epilogue onormgate is not part of this build"
    assert res[8] == "gemm: heads.rope needs 2048 B of a 2047 B buffer"
    assert res[9] == "gemm: heads ropeMode sideways"
