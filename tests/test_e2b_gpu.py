"""GPU parity at the BASELINE decode configurations B and C (Gemma-4-E2B-shaped, hidden 2048), through the C ABI.

The op sequence is bench.py's decode step at its exact shapes, cut to two layers plus the whole head:
  qkv 3072x2048 (rms) -> o 2048x2048 (raw, kPer 2048) -> gate_up 2x8192x2048 (rms, geglu) -> down 2048x8192
  (raw, kPer 2048: 4 K-split partials) -> next layer's qkv (rms over down's first partial) ... -> lm_head
  262144x2048 (rms, softcap 30, per-tile max / argmax).
Every op reads its predecessor's output, as in bench.py (the norms between them in the model are not GEMVs; the rstd
slots are fixed inputs). Config B runs it at M = 1 as one pipelined chain (the headline path) and as a recording of
standalone launches; config C at M = 5 (the verify pass) both ways, and the M sweep {2, 4, 8, 16} as standalone gemvM
calls at the qkv and gate_up shapes. Each op is checked against the oracle run on the input that op read on the GPU
(its predecessor's output, read back), after every output was NaN-filled; the head's 4096 tile maxima are checked
against the oracle and its argmax indices by their defining property over the GPU's own logits.
Tolerance: relative L2 <= 1e-3 (BASELINE) and 2e-6 here, tighter than this build's general fp32 bar of 2e-5 since the
oracle runs on the exact weight bytes the GPU holds (read back); the largest seen is 5e-7.
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
D, QKV, MLP, V = 2048, 3072, 8192, 262144
NAN = 0x7FC00000


def _check(got, want, what):
    r = rel_l2(got, want)
    print(f"{what}: rel_l2 {r:.3e} (rms {float(np.sqrt(np.mean(np.square(want, dtype=np.float64)))):.3g})", flush=True)
    assert np.all(np.isfinite(got)), what + ": non-finite output"
    assert r <= 1e-3 and r <= 2e-6, (what, r)


def _device_fill(b, host, what):
    """the weights the GPU holds, read back, after checking them against the oracle's fill of the same seed: the code
    words bit for bit; the fp16 scales equal or one fp16 step apart, in a small fraction of the groups (the device's
    float64 log / cos and libm's may round a scale's last bit differently), and every min exactly -8 x its scale. The
    oracle then runs on the exact bytes the GPU reads."""
    dev = b.read(np.uint8, host.size)
    d, h = dev.reshape(-1, 1280), host.reshape(-1, 1280)
    assert np.array_equal(d[:, :1024], h[:, :1024]), what + ": code words differ from the oracle's fill"
    ds, hs = d[:, 1024:].view(np.uint16)[:, 0::2], h[:, 1024:].view(np.uint16)[:, 0::2]
    diff = np.abs(ds.astype(np.int32) - hs.astype(np.int32))   # positive fp16: adjacent values, adjacent bit patterns
    assert diff.max() <= 1 and np.mean(diff != 0) < 1e-3, (what, int(diff.max()), float(np.mean(diff != 0)))
    mins = d[:, 1024:].view(np.uint16)[:, 1::2]
    want = (np.float32(-8) * ds.view(np.float16).astype(np.float32)).astype(np.float16).view(np.uint16)
    assert np.array_equal(mins, want), what + ": min != -8 x scale"
    return dev


class E2B:
    """two decode layers + the head at bench.py's shapes, M rows; symmetric BASELINE weights filled on the device and
    on the host by the oracle's copy of the same counter hash (the oracle then runs on the device's bytes read back). bounded: bench.py's weight scales and
    sign-alternating norm weights, which keep every activation O(1) (|x'| < 255: an M > 1 chain then runs every op on
    the matrix cores); else sigma 0.02 everywhere, whose activations grow ~4x per op (later M > 1 ops take the VALU
    fallback)."""

    def __init__(self, M, layers=2, seed=5, bounded=False):
        self.M, self.L = M, layers
        shapes = {"qkv": (QKV, D), "o": (D, D), "gu": (2 * MLP, D), "dn": (D, MLP)}
        gain = {"qkv": 1.0, "o": 1.0, "gu": 1.0, "dn": 1.55}
        self.w_host, self.w_dev = {}, {}
        for l in range(layers):
            for i, (k, (n, kk)) in enumerate(shapes.items()):
                s = seed * 101 + l * 16 + i
                sig = float(gain[k] / np.sqrt(21.5 * kk)) if bounded else 0.02
                b = capi.Buffer(n // 64 * kk // 32 * 1280)
                capi.fill_q4_sym(b, n, kk, s, sig)
                self.w_dev[(l, k)] = b
                self.w_host[(l, k)] = _device_fill(b, O.fill_q4_sym(n, kk, s, sig), f"weights {l} {k}")
        self.w_dev["head"] = capi.Buffer(V // 64 * D // 32 * 1280)
        capi.fill_q4_sym(self.w_dev["head"], V, D, seed * 101 + 99, 0.02)
        self.w_host["head"] = _device_fill(self.w_dev["head"], O.fill_q4_sym(V, D, seed * 101 + 99, 0.02), "head")
        self.x = O.fill_randn(M * D, seed)[0]
        self.nw = np.linspace(0.8, 1.2, D).astype(np.float32)
        if bounded:
            self.nw *= 1 - 2 * (np.arange(D) % 2)
        # rstd slots: a (pad, rstd) pair per row for each rms op (qkv and gate_up of every layer), 1 / sqrt(1 + eps)
        # until calibrate() sets them from the activations
        st = np.zeros(2 * M * 2 * layers + 4, np.float32)
        st[1::2] = 1.0 / np.sqrt(1.0 + 1e-6)
        self.st = st
        self.rstd_head = np.full(M, 0.9, np.float32)
        NT = V // 64
        self.mx_len = M * NT * 2 + 2 * M + 4
        mx = np.zeros(self.mx_len, np.float32)
        mx[M * NT * 2 + 1::2][:M] = self.rstd_head
        self.mx = mx
        self.mx_stat_off = M * NT * 2 + 1
        self.dev = {"x": capi.to_device(self.x), "nw": capi.to_device(self.nw), "st": capi.to_device(st),
                    "mx": capi.to_device(mx),
                    # the token's tail: the rstd the token copies into the head's slot (mx's), the argmax words and
                    # the staging buffer they are copied to
                    "rsrc": capi.to_device(self._rsrc()),
                    "arg": capi.Buffer(8 * M + 8), "stage": capi.Buffer(8 * M + 8)}
        self.out_len = {}
        for l in range(layers):
            self.out_len.update({("qkv", l): M * QKV, ("o", l): M * D, ("gu", l): M * MLP, ("dn", l): 4 * M * D})
        self.out_len["head"] = M * V
        self.out = {k: capi.Buffer(4 * n) for k, n in self.out_len.items()}

    def _rsrc(self):
        r = np.zeros(2 * self.M, np.float32)
        r[1::2] = self.rstd_head
        return r

    def rms_off(self, j):
        """stat_off of rms op j (qkv of layer l: j = 2 l, gate_up: 2 l + 1)"""
        return 2 * self.M * j + 1

    def calibrate(self, ch):
        """sets every rms op's rstd slots, the head's included, to 1 / sqrt(mean(x^2) + 1e-6) over each row that op
        reads on the GPU, as the model's RMSNorm computes them, so that activations stay O(1) through every layer
        (with fixed slots the geglu's square makes the magnitude an unstable balance: it collapses towards 0 within a
        few layers). One slot per run of ch (a chain, or a recording: anything with run / replay): its arithmetic is
        fixed, so a run reproduces every op before the slot just set bit for bit, and the next slot is computed from
        that run's output."""
        M = self.M

        def rstd(x):
            x = x.reshape(M, D).astype(np.float64)
            return (1.0 / np.sqrt(np.mean(x * x, axis=1) + 1e-6)).astype(np.float32)

        self.st[self.rms_off(0)::2][:M] = rstd(self.x)
        self.dev["st"].upload(self.st)
        for j in range(1, 2 * self.L + 1):
            if hasattr(ch, "replay"):
                ch.replay()
            else:
                ch.run()
                assert not ch.status()
            src = ("o", (j - 1) // 2) if j % 2 else ("dn", j // 2 - 1)   # gate_up reads o, qkv / head a down partial
            r = rstd(self.out[src].read(np.float32, M * D))
            assert np.all((r > 0.01) & (r < 100)), (j, r)   # every op's input stays O(1)
            if j < 2 * self.L:
                self.st[self.rms_off(j)::2][:M] = r
                self.dev["st"].upload(self.st)
            else:
                self.rstd_head = r
                self.mx[self.mx_stat_off::2][:M] = r
                self.dev["mx"].upload(self.mx)
                self.dev["rsrc"].upload(self._rsrc())

    def fields(self, bufs, w):
        """(name, weight key, input key, field dict) per op; bufs / w map keys to Buffers or host pointers"""
        M, ops = self.M, []
        P, E = capi.PRO, capi.EPI
        for l in range(self.L):
            xin = "x" if l == 0 else ("dn", l - 1)   # the previous down's first K-split partial
            ops.append((("qkv", l), (l, "qkv"), xin, dict(w_rows=QKV, w_cols=D, N=QKV, K=D, pro=P["rms"],
                                                             stat=bufs["st"], stat_off=self.rms_off(2 * l),
                                                             norm=bufs["nw"])))
            ops.append((("o", l), (l, "o"), ("qkv", l), dict(w_rows=D, w_cols=D, N=D, K=D, kPer=2048, pro=P["raw"],
                                                              x_ldx=QKV)))
            ops.append((("gu", l), (l, "gu"), ("o", l), dict(w_rows=2 * MLP, w_cols=D, N=MLP, K=D, pro=P["rms"],
                                                              epi=E["geglu"], stat=bufs["st"],
                                                              stat_off=self.rms_off(2 * l + 1),
                                                              norm=bufs["nw"])))
            ops.append((("dn", l), (l, "dn"), ("gu", l), dict(w_rows=D, w_cols=MLP, N=D, K=MLP, kPer=2048,
                                                               pro=P["raw"])))
        ops.append(("head", "head", ("dn", self.L - 1), dict(w_rows=V, w_cols=D, N=V, K=D, pro=P["rms"],
                                                              epi=E["softcap"], stat=bufs["mx"],
                                                              stat_off=self.mx_stat_off, norm=bufs["nw"],
                                                              mx=bufs["mx"], cap=30.0)))
        out = []
        for name, wk, xk, f in ops:
            f = dict(f, w=w[wk], x=bufs[xk], y=bufs[name])
            if M > 1:
                f.setdefault("x_ldx", f["K"])
                f.update(M=M, stat_ld=2, y_ldm=f["N"])
                if f.get("epi", 0) == E["store"]:
                    f["y_ldy"] = M * f["N"]
            else:
                f.pop("x_ldx", None)
                if f.get("epi", 0) == E["store"]:
                    f["ldy"] = f["N"]
            out.append((name, wk, xk, f))
        return out

    def enqueue(self, tail=False):
        """the ops; tail: the whole token as bench.py times it, with the head's rstd copied into its stat slot before
        it, the argmax over its tile maxima after it and the copy of the result words (engine/llm/gemma4.js:503-511,
        engine/llm/drunner.js:82-90)"""
        M = self.M
        for name, wk, xk, f in self.fields({**self.dev, **self.out}, self.w_dev):
            if name == "head" and tail:
                for m in range(M):
                    capi.copy(self.dev["rsrc"], (2 * m + 1) * 4, self.dev["mx"], (self.mx_stat_off + 2 * m) * 4, 4)
            if M == 1:
                capi.q4_gemv(capi.gemv_args(**f))
            else:
                capi.q4_gemvM(capi.gemvm_args(**f))
        if tail:
            capi.argmaxM(self.dev["mx"], V // 64, M, self.dev["arg"])
            capi.copy(self.dev["arg"], 0, self.dev["stage"], 0, 8 * M)

    def reset(self, tail=False):
        for b in self.out.values():
            b.fill_u32(NAN)
        self.dev["mx"].upload(self.mx)
        if tail:   # the rstd slots and the result words must be written by this run
            mx = self.mx.copy()
            mx[self.mx_stat_off::2][:self.M] = np.nan
            self.dev["mx"].upload(mx)
            self.dev["arg"].fill_u32(NAN)
            self.dev["stage"].fill_u32(NAN)

    def check_tail(self, what):
        """the argmax words and their copy against the oracle's argmax over the tile maxima the chain wrote"""
        M, NT = self.M, V // 64
        gmx = self.dev["mx"].read(np.float32, self.mx_len)
        np.testing.assert_array_equal(gmx[self.mx_stat_off::2][:M], self.rstd_head)
        want = np.asarray(O.argmaxM(gmx, NT, M), np.uint32).ravel()
        assert np.array_equal(self.dev["arg"].read(np.uint32, 2 * M), want), what + ": argmax"
        assert np.array_equal(self.dev["stage"].read(np.uint32, 2 * M), want), what + ": result copy"
        lg = self.out["head"].read(np.float32, M * V).reshape(M, V)
        assert np.array_equal(want[0::2], np.argmax(lg, axis=1).astype(np.uint32)), what + ": argmax of the logits"
        print(what, "argmax", want[0::2].tolist(), flush=True)

    def check(self, what, layers=None, head_rows=None):
        """every op (or those of `layers` and the head) against the oracle on the input it read on the GPU; head_rows:
        the head's first head_rows rows only (a multiple of 64: its logits and tile maxima; rows are independent)"""
        got = {k: self.out[k].read(np.float32, n) for k, n in self.out_len.items()}
        gmx = self.dev["mx"].read(np.float32, self.mx_len)
        M = self.M
        hostbuf = {"x": self.x, "st": self.st, "nw": self.nw}
        NT, HR = V // 64, head_rows or V
        for name, wk, xk, f in self.fields({k: 0 for k in list(self.out_len) + ["x", "st", "nw", "mx"]}, self.w_host):
            if layers is not None and name != "head" and name[1] not in layers:
                continue
            xin = np.ascontiguousarray(hostbuf["x"] if xk == "x" else got[xk], np.float32)
            y = np.full(self.out_len[name], np.nan, np.float32)
            f = dict(f, w=self.w_host[wk].ctypes.data, x=xin.ctypes.data, y=y.ctypes.data, norm=self.nw.ctypes.data)
            if name == "head":
                # the rstd slots past the tile pairs (a softcap GEMV at M = 1 reads them from mx, as the reference's
                # gemv does); the oracle writes the first HR rows' tile pairs at the front, as M rows of HR / 64
                mx = self.mx.copy()
                f.update(w_rows=HR, N=HR, stat=mx.ctypes.data, mx=mx.ctypes.data)
            else:
                f["stat"] = self.st.ctypes.data if "stat" in f else None
            (O.q4_gemv if M == 1 else O.q4_gemvM)((capi.gemv_args if M == 1 else capi.gemvm_args)(**f))
            if name == "head":
                _check(got[name].reshape(M, V)[:, :HR], y.reshape(M, V)[:, :HR], f"{what} head rows < {HR}")
            else:
                _check(got[name], y, f"{what} {name}")
        # the head's per-tile (max, argmax): maxima against the oracle, indices by their defining property over the
        # GPU's own logits (the first row of the tile holding the tile's largest value)
        lg = got["head"].reshape(M, NT, 64)
        gm = gmx[:2 * NT * M:2].reshape(M, NT)
        gi = gmx[1:2 * NT * M:2].view(np.uint32).reshape(M, NT)
        wm = mx[:2 * M * (HR // 64):2].reshape(M, HR // 64)
        _check(gm[:, :HR // 64], wm, what + " tile maxima")   # the maxima are logits: the logits' bar
        print(what, "tile maxima: largest |diff|", float(np.max(np.abs(gm[:, :HR // 64] - wm))), flush=True)
        want_i = (np.argmax(lg, axis=2) + np.arange(NT)[None, :] * 64).astype(np.uint32)
        assert np.array_equal(gi, want_i), what + ": tile argmax"
        assert np.array_equal(gm, np.take_along_axis(lg, (gi % 64).astype(np.int64)[:, :, None], 2)[:, :, 0])

    def free(self):
        for b in list(self.w_dev.values()) + list(self.dev.values()) + list(self.out.values()):
            b.free()


@pytest.fixture(scope="module")
def e2b1(dev):
    s = E2B(1)
    yield s
    s.free()


def test_config_b_decode_step_as_one_chain(e2b1):
    """config B: the E2B-shaped layers + head planned into ONE pipelined chain launch (bench.py's headline path)"""
    s = e2b1
    ch = capi.chain(s.enqueue)
    info = ch.info()
    print("chain", info, flush=True)
    assert info["n_ops"] == 4 * s.L + 1 and info["m"] == 1
    for run in range(2):   # a second run of the same chain (the run tag advances; no reset)
        s.reset()
        ch.run()
        assert not ch.status()
        s.check(f"config B chain run {run}")
    ch.free()


def test_config_b_decode_step_as_a_recording(e2b1):
    """config B as a recording of one launch per op (the DecodeRunner's graph mode)"""
    s = e2b1
    rec = capi.record(s.enqueue)
    assert rec.launches() == 4 * s.L + 1
    s.reset()
    rec.replay()
    s.check("config B graph")
    rec.free()


def test_config_b_full_token_as_one_chain(dev):
    """config B at full depth, as bench.py times it: 30 layers (bench.py's weight scales) + the rstd copy, the head,
    the argmax and the result copy = 124 ops in one pipelined launch (120 mailbox hand-offs, ring wrap-arounds across
    the whole step), twice; every op against the oracle on the input it read, the argmax and its copy exactly. The rstd
    slots are calibrated from the chain's own activations first, so every layer and the head compute on O(1) data."""
    s = E2B(1, layers=30, seed=9, bounded=True)
    try:
        ch = capi.chain(lambda: s.enqueue(tail=True))
        info = ch.info()
        print("chain", info, flush=True)
        assert info["n_ops"] == 4 * 30 + 4 and info["passes"] == 1 and info["mailboxes"] == 119
        s.calibrate(ch)
        print("head rstd", s.rstd_head.tolist(), flush=True)
        for run in range(2):
            s.reset(tail=True)
            ch.run()
            assert not ch.status()
            s.check(f"config B full token run {run}")
            s.check_tail(f"config B full token run {run}")
        ch.free()
    finally:
        s.free()


def test_config_b_full_token_many_runs(dev):
    """the full-depth token chain run 1000 times back to back, as a decode loop runs it (the run tag advancing, no
    reset in between): no wait gives up, and the last run's logits, tile pairs, argmax and result copy equal the first
    run's bit for bit (the chain's arithmetic is fixed and its counters return to zero by themselves); rstd slots
    calibrated as above"""
    s = E2B(1, layers=30, seed=9, bounded=True)
    try:
        ch = capi.chain(lambda: s.enqueue(tail=True))
        s.calibrate(ch)
        s.reset(tail=True)
        ch.run()
        assert not ch.status()
        V = s.out_len["head"]
        first = (s.out["head"].read(np.uint32, V).copy(), s.dev["mx"].read(np.uint32, s.mx_len).copy(),
                 s.dev["arg"].read(np.uint32, 2).copy(), s.dev["stage"].read(np.uint32, 2).copy())
        for block in range(10):
            for _ in range(100):
                ch.run()
            assert not ch.status(), f"a wait gave up within runs {100 * block + 1}-{100 * block + 100}"
            print(f"runs up to {100 * block + 101}: no wait gave up", flush=True)
        last = (s.out["head"].read(np.uint32, V), s.dev["mx"].read(np.uint32, s.mx_len),
                s.dev["arg"].read(np.uint32, 2), s.dev["stage"].read(np.uint32, 2))
        for what, a, b in zip(("logits", "tile pairs", "argmax", "result copy"), first, last):
            assert np.array_equal(a, b), what
        s.check_tail("config B token run 1001")
        ch.free()
    finally:
        s.free()


@pytest.mark.parametrize("M,data", [(8, "bounded"), (8, "large"), (16, "bounded"), (16, "large"), (6, "bounded"),
                                    (12, "large")])
def test_config_c_verify_chain_m8_m16(dev, M, data):
    """config C's verify chains of 6 - 16 rows at the E2B shapes (two layers + the head, then argmaxM over the head's
    tile maxima) in one pass of the wide kernel, each op against the oracle on the input it read; with large
    activations the producer's 2^8 staging overflows from the second layer on and the waves stage x' with their own
    scale"""
    s = E2B(M, seed=10 + M, bounded=data == "bounded")
    try:
        def token():
            s.enqueue()
            capi.argmaxM(s.dev["mx"], V // 64, M, s.dev["arg"])
        ch = capi.chain(token)
        info = ch.info()
        print("chain", info, flush=True)
        assert info["passes"] == 1 and info["waves_per_workgroup"] == 12 and info["staged"] == 4 * s.L
        s.reset()
        s.dev["arg"].fill_u32(NAN)
        ch.run()
        assert not ch.status()
        ch.free()
        s.check(f"config C M={M} chain {data}")
        gmx = s.dev["mx"].read(np.float32, s.mx_len)
        want = np.asarray(O.argmaxM(gmx, V // 64, M), np.uint32).ravel()
        assert np.array_equal(s.dev["arg"].read(np.uint32, 2 * M), want)
    finally:
        s.free()


@pytest.mark.parametrize("M", [5, 16])
def test_config_c_full_depth_many_runs(dev, M):
    """the full-depth verify chain (30 layers + the head + the tail; the pipelined kernel at M = 5, the wide kernel at
    M = 16) run 500 times back to back with no reset: no wait gives up, and the last run's logits, tile pairs, argmax
    words and result copy equal the first run's bit for bit; rstd slots calibrated as in the full-depth test"""
    s = E2B(M, layers=30, seed=60 + M, bounded=True)
    try:
        ch = capi.chain(lambda: s.enqueue(tail=True))
        s.calibrate(ch)
        s.reset(tail=True)
        ch.run()
        assert not ch.status()
        V_ = s.out_len["head"]
        first = (s.out["head"].read(np.uint32, V_).copy(), s.dev["mx"].read(np.uint32, s.mx_len).copy(),
                 s.dev["arg"].read(np.uint32, 2 * M).copy(), s.dev["stage"].read(np.uint32, 2 * M).copy())
        for block in range(5):
            for _ in range(100):
                ch.run()
            assert not ch.status(), f"a wait gave up within runs {100 * block + 2}-{100 * block + 101}"
            print(f"M={M}: runs up to {100 * block + 101}: no wait gave up", flush=True)
        last = (s.out["head"].read(np.uint32, V_), s.dev["mx"].read(np.uint32, s.mx_len),
                s.dev["arg"].read(np.uint32, 2 * M), s.dev["stage"].read(np.uint32, 2 * M))
        for what, a, b in zip(("logits", "tile pairs", "argmax", "result copy"), first, last):
            assert np.array_equal(a, b), what
        s.check_tail(f"config C M={M} run 501")
        ch.free()
    finally:
        s.free()


@pytest.mark.parametrize("M", [8, 16])
def test_config_c_row_group_passes(dev, M):
    """config C's verify chain at 8 and 16 rows (two layers + the head, argmaxM) with the wide kernel off
    (p0_chain_tune knob 12 = 0): pipelined passes over row groups of at most 5 rows, each pass's staged x', 4-split down
    projection and softcap tile maxima at their row group's offsets, every op against the oracle"""
    s = E2B(M, seed=40 + M, bounded=True)
    old = capi.chain_tune(12, 0)
    try:
        def token():
            s.enqueue()
            capi.argmaxM(s.dev["mx"], V // 64, M, s.dev["arg"])
        ch = capi.chain(token)
    finally:
        capi.chain_tune(12, old)
    try:
        info = ch.info()
        print("chain", info, flush=True)
        assert info["passes"] == -(-M // 5) and info["passes"] > 1
        s.reset()
        s.dev["arg"].fill_u32(NAN)
        ch.run()
        assert not ch.status()
        s.check(f"config C M={M} row-group passes")
        gmx = s.dev["mx"].read(np.float32, s.mx_len)
        want = np.asarray(O.argmaxM(gmx, V // 64, M), np.uint32).ravel()
        assert np.array_equal(s.dev["arg"].read(np.uint32, 2 * M), want)
    finally:
        ch.free()
        s.free()


@pytest.mark.parametrize("M,way", [(5, "chain"), (5, "graph"), (16, "chain")])
def test_config_c_full_depth(dev, M, way):
    """config C at full depth, as bench.py times the verify pass: 30 layers + the head (M rows), with the token's tail
    (the rstd copies, argmaxM, the result copy), as one chain launch (the pipelined kernel at M = 5, the wide kernel at
    M = 16) or as a recording of standalone launches. The rstd slots are calibrated from the path's own activations
    first, so every layer computes on O(1) data and every M > 1 op runs on the matrix cores. Checked against the
    oracle on the inputs they read: every op of the 30 layers, the head (at M = 16 its first 65536 rows and their tile
    maxima: the oracle's cost grows with M) and the whole tail"""
    s = E2B(M, layers=30, seed=20 + M, bounded=True)
    try:
        run = (capi.chain if way == "chain" else capi.record)(lambda: s.enqueue(tail=True))
        if way == "chain":
            info = run.info()
            print("chain", info, flush=True)
            assert info["n_ops"] == 4 * 30 + M + 3 and info["passes"] == 1
        s.calibrate(run)
        print("head rstd", s.rstd_head.tolist(), flush=True)
        s.reset(tail=True)
        if way == "chain":
            run.run()
            assert not run.status()
        else:
            run.replay()
        s.check(f"config C full depth M={M} {way}", head_rows=65536 if M > 8 else None)
        s.check_tail(f"config C full depth M={M} {way}")
        run.free()
    finally:
        s.free()


@pytest.mark.parametrize("data", ["bounded", "large"])
@pytest.mark.parametrize("way", ["chain", "graph"])
def test_config_c_verify_pass_m5(dev, way, data):
    """config C: the verify pass (M = 1 + 4 draft tokens) at the E2B shapes, as one pipelined chain and as a
    recording of standalone gemvM launches (both run on the matrix cores for M >= 2, the chain's spread shares and its
    lm_head alike; with large activations later ops take the VALU fallback)"""
    s = E2B(5, seed=6, bounded=data == "bounded")
    try:
        if way == "chain":
            ch = capi.chain(s.enqueue)
            print("chain", ch.info(), flush=True)
            s.reset()
            ch.run()
            assert not ch.status()
            ch.free()
        else:
            rec = capi.record(s.enqueue)
            s.reset()
            rec.replay()
            rec.free()
        s.check(f"config C M=5 {way}")
    finally:
        s.free()


@pytest.mark.parametrize("M,knob9", [(2, 2), (3, 6), (4, 6)])
def test_config_c_chain_both_arithmetics(dev, M, knob9):
    """the pipelined chain's two slot arithmetics at the rows where the default picks the other one (p0_chain_tune
    knob 9: the fewest rows on the matrix cores, default 3): M = 2 on the matrix cores, M = 3 and 4 on the fp32 VALU"""
    s = E2B(M, seed=7, bounded=True)
    old = capi.chain_tune(9, knob9)
    try:
        ch = capi.chain(s.enqueue)
    finally:
        capi.chain_tune(9, old)
    try:
        print("chain", ch.info(), flush=True)
        s.reset()
        ch.run()
        assert not ch.status()
        s.check(f"M={M} chain, knob 9 = {knob9}")
    finally:
        ch.free()
        s.free()


@pytest.mark.parametrize("M", [2, 4, 8, 16])
@pytest.mark.parametrize("op", ["qkv", "gate_up"])
def test_config_c_sweep_standalone(dev, M, op):
    """config C's M sweep at the qkv (rms) and gate_up (rms + geglu) shapes: standalone gemvM, each record read once
    for all M rows"""
    N, rows, epi = (QKV, QKV, capi.EPI["store"]) if op == "qkv" else (MLP, 2 * MLP, capi.EPI["geglu"])
    w = O.fill_q4_sym(rows, D, 300 + M, 0.02)
    x = O.fill_randn(M * D, 301 + M)[0]
    nw = np.linspace(0.9, 1.1, D).astype(np.float32)
    st = np.zeros(2 * M, np.float32)
    st[1::2] = 0.8
    f = dict(w_rows=rows, w_cols=D, x_ldx=D, M=M, N=N, K=D, pro=capi.PRO["rms"], epi=epi, stat_off=0, stat_ld=2,
             y_ldm=N)
    want = np.full(M * N, np.nan, np.float32)
    O.q4_gemvM(capi.gemvm_args(**f, w=w.ctypes.data, x=x.ctypes.data, y=want.ctypes.data, stat=st.ctypes.data,
                               norm=nw.ctypes.data))
    d = {k: capi.to_device(v) for k, v in dict(w=w, x=x, stat=st, norm=nw).items()}
    yb = capi.Buffer(M * N * 4).fill_u32(NAN)
    capi.q4_gemvM(capi.gemvm_args(**f, **d, y=yb))
    _check(yb.read(np.float32), want, f"gemvM M={M} {op}")
    for b in list(d.values()) + [yb]:
        b.free()


@pytest.mark.parametrize("M", [3, 5])
def test_config_c_chain_staged_hand_off(dev, M):
    """a pipelined M > 1 chain on the matrix cores takes each op's x' as its predecessor staged it (p0_chain_tune knob
    10): every op after the first reads one split of its predecessor's output, so all of them are staged, and the
    outputs are bit-identical to the chain whose ops stage their own x' (the staged values are stage_rows's, computed
    in the same order), and within the bars of the oracle; with large activations (the VALU fallback marked through the
    staged group sums) as well"""
    for bounded in (True, False):
        s = E2B(M, seed=8, bounded=bounded)
        try:
            outs, infos = [], []
            for knob in (1, 0):
                old = capi.chain_tune(10, knob)
                try:
                    ch = capi.chain(s.enqueue)
                finally:
                    capi.chain_tune(10, old)
                try:
                    infos.append(ch.info())
                    s.reset()
                    ch.run()
                    assert not ch.status()
                    outs.append({k: s.out[k].read(np.float32, n) for k, n in s.out_len.items()})
                    outs[-1]["mx"] = s.dev["mx"].read(np.float32, s.mx_len)
                finally:
                    ch.free()
            print("staged chain", infos[0], "unstaged", infos[1], flush=True)
            assert infos[0]["staged"] == 4 * s.L and infos[1]["staged"] == 0
            for k in outs[0]:
                assert np.array_equal(outs[0][k].view(np.uint32), outs[1][k].view(np.uint32)), (M, bounded, k)
            s.check(f"config C M={M} staged chain, {'bounded' if bounded else 'large'}")
        finally:
            s.free()
