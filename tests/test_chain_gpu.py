"""GPU parity of GEMV chains (p0_chain_*): a decode step's GEMVs planned once and run as ONE persistent launch.

Each op of a chain is checked against the CPU oracle run on the input that op actually read on the GPU (the previous
op's output, read back), so a wrong result and a broken dependency wait fail separately: every intermediate buffer is
NaN-filled before the run, and an op that read its input before the producer finished writing it cannot pass.
Tolerance as for single GEMVs: relative L2 <= 1e-3 and this build's fp32 bar of 2e-5.
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL, TOL_FP32 = 1e-3, 2e-5
NAN = 0x7FC00000


def _check(got, want, what):
    r = rel_l2(got, want)
    print(f"{what}: rel_l2 {r:.3e}", flush=True)
    assert np.all(np.isfinite(got)), what + ": non-finite output"
    assert r <= TOL and r <= TOL_FP32, what


def _w(rows, K, seed):
    return O.pack_q4(O.randn(rows * K, seed, 0.05), rows, K)[0]


class MiniStep:
    """A decode-like op sequence at M rows: qkv (rms) -> o (raw, reads qkv) -> gate/up (rms + geglu, reads o) ->
    down (raw, 2 K-splits, reads the geglu output) -> sum of the 2 partials (pro sum) -> head (rms + softcap).
    Scalar rms statistics are fixed inputs (computed on the host), so every op's input is the previous op's output."""

    def __init__(self, M=1, D=256, QKV=384, MLP=512, V=4096, seed=3, gemvM=False):
        self.M, self.D, self.QKV, self.MLP, self.V, self.gemvM = M, D, QKV, MLP, V, gemvM
        self.host = {
            "x": O.randn(M * D, seed), "w_qkv": _w(QKV, D, seed + 1), "w_o": _w(D, D, seed + 2),
            "w_gu": _w(2 * MLP, D, seed + 3), "w_dn": _w(D, MLP, seed + 4), "w_sum": _w(D, D, seed + 5),
            "w_hd": _w(V, D, seed + 6), "norm": (0.8 + 0.4 * O.rng_uniform(seed + 7, D)).astype(np.float32),
        }
        st = np.zeros(2 * M + 8, np.float32)
        st[1::2][:M] = 0.7                      # rstd of each row for the rms prologues
        self.host["stat"] = st
        NT = V // 64
        self.mx_len = M * NT * 2 + 2 * M + 8
        mx = np.zeros(self.mx_len, np.float32)
        mx[M * NT * 2 + 1::2][:M] = 0.9         # head rms rstd slot (gemv softcap reads it from mx)
        self.host["mx"] = mx
        self.dev = {k: capi.to_device(v) for k, v in self.host.items()}
        self.out_len = {"qkv": M * QKV, "o": M * D, "gu": M * MLP, "dn": 2 * M * D, "sum": M * D, "hd": M * V}
        self.out = {k: capi.Buffer(4 * n) for k, n in self.out_len.items()}
        self.mx_stat_off = M * NT * 2 + 1

    def ops(self, b):
        """field dicts of the 6 ops over buffer map b (device Buffers or host pointers)"""
        M, D, QKV, MLP, V = self.M, self.D, self.QKV, self.MLP, self.V
        E, P = capi.EPI, capi.PRO
        ops = [
            dict(w=b["w_qkv"], w_rows=QKV, w_cols=D, x=b["x"], N=QKV, K=D, pro=P["rms"], epi=E["store"], y=b["qkv"],
                 stat=b["stat"], stat_off=1, norm=b["norm"]),
            dict(w=b["w_o"], w_rows=D, w_cols=D, x=b["qkv"], N=D, K=D, pro=P["raw"], epi=E["store"], y=b["o"]),
            dict(w=b["w_gu"], w_rows=2 * MLP, w_cols=D, x=b["o"], N=MLP, K=D, pro=P["rms"], epi=E["geglu"],
                 y=b["gu"], stat=b["stat"], stat_off=1, norm=b["norm"]),
            dict(w=b["w_dn"], w_rows=D, w_cols=MLP, x=b["gu"], N=D, K=MLP, kPer=256, pro=P["raw"], epi=E["store"],
                 y=b["dn"]),
            dict(w=b["w_sum"], w_rows=D, w_cols=D, x=b["dn"], N=D, K=D, pro=P["sum"] if not self.gemvM else P["raw"],
                 epi=E["store"], y=b["sum"], src_n=2, src_ld=D if not self.gemvM else M * D),
            dict(w=b["w_hd"], w_rows=V, w_cols=D, x=b["sum"], N=V, K=D, pro=P["rms"], epi=E["softcap"], y=b["hd"],
                 norm=b["norm"], mx=b["mx"], cap=30.0),
        ]
        for o in ops:
            if self.gemvM:
                o.update(M=M, x_ldx=o["K"], stat_ld=2, y_ldm=o["N"])
                if o["epi"] == E["store"]:
                    o.update(y_ldy=M * o["N"])
            if o["epi"] == E["softcap"]:   # the head's rms rstd sits in mx (engine/llm/lops.js:125)
                o.update(stat=b["mx"], stat_off=self.mx_stat_off)
        if self.gemvM:
            ops[1]["x_ldx"] = QKV                # o reads the q rows of the qkv output (row stride QKV)
            ops[4].update(src_n=0, src_ld=0)     # gemvM has no 'sum' prologue (engine/llm/lops_spec.js:64): raw
        return ops

    def _args(self, f):
        return capi.gemvm_args(**f) if self.gemvM else capi.gemv_args(**f)

    def _enqueue(self):
        for f in self.ops(self.dev | self.out):
            (capi.q4_gemvM if self.gemvM else capi.q4_gemv)(self._args(f))

    def make_chain(self):
        return capi.chain(self._enqueue)

    def reset_outputs(self):
        for b in self.out.values():
            b.fill_u32(NAN)
        self.dev["mx"].upload(self.host["mx"])

    def read(self):
        r = {k: self.out[k].read(np.float32, n) for k, n in self.out_len.items()}
        r["mx"] = self.dev["mx"].read(np.float32, self.mx_len)
        return r

    def check_against_oracle(self, got, what):
        """each op vs the oracle on the input it read (the GPU's previous output)"""
        mx = self.host["mx"].copy()
        names = ["qkv", "o", "gu", "dn", "sum", "hd"]
        weights = ["w_qkv", "w_o", "w_gu", "w_dn", "w_sum", "w_hd"]
        inputs = {"qkv": self.host["x"], "o": got["qkv"], "gu": got["o"], "dn": got["gu"], "sum": got["dn"],
                  "hd": got["sum"]}
        for i, (name, f) in enumerate(zip(names, self.ops({k: 0 for k in list(self.host) + names}))):
            y = np.full(self.out_len[name], np.nan, np.float32)
            xin = np.ascontiguousarray(inputs[name], np.float32)
            ptrs = {"w": self.host[weights[i]].ctypes.data,
                    "x": xin.ctypes.data, "y": y.ctypes.data, "norm": self.host["norm"].ctypes.data}
            f = dict(f, **ptrs)
            if "stat" in f:
                f["stat"] = (mx if f["epi"] == capi.EPI["softcap"] else self.host["stat"]).ctypes.data
            if "mx" in f:
                f["mx"] = mx.ctypes.data
            (O.q4_gemvM if self.gemvM else O.q4_gemv)(self._args(f))
            _check(got[name], y, f"{what} op {i} ({name})")
        NT = self.V // 64
        gm, om = got["mx"][:2 * NT * self.M:2], mx[:2 * NT * self.M:2]
        assert np.allclose(gm, om, rtol=1e-5, atol=1e-5), what + ": tile maxima"
        gi = got["mx"][1:2 * NT * self.M:2].view(np.uint32)
        oi = mx[1:2 * NT * self.M:2].view(np.uint32)
        assert np.mean(gi == oi) > 0.99, what + ": tile argmax"

    def free(self):
        for b in list(self.dev.values()) + list(self.out.values()):
            b.free()


@pytest.mark.parametrize("M,gemvM,pipe_m", [(1, False, 1), (1, True, 1), (2, True, 1), (3, True, 1), (5, True, 1),
                                             (5, True, 0), (8, True, 1)])
def test_chain_matches_oracle(dev, M, gemvM, pipe_m):
    """M <= 5 rows run on the pipelined kernel in one launch and M = 8 on the wide pipelined kernel, also one launch
    (knob 8 on); knob 8 off puts M = 5 on the general kernel"""
    s = MiniStep(M=M, gemvM=gemvM, seed=10 + M)
    old = capi.chain_tune(8, pipe_m)
    try:
        ch = s.make_chain()
    finally:
        capi.chain_tune(8, old)
    info = ch.info()
    print("chain", info, flush=True)
    assert info["n_ops"] == 6 and info["m"] == M
    if pipe_m:
        assert info["waves_per_workgroup"] == 12 and info["passes"] == 1
    else:
        assert info["waves_per_workgroup"] == 8 and info["passes"] == 1
    if M == 1 and info["waves_per_workgroup"] == 12:
        # o takes qkv's output, gate_up (rms) o's, down the geglu output, the head (rms) the 'sum' op's; qkv and the
        # 'sum' op (two partials per element) wait for flags. As gemvM calls, op 4 reads down's first split raw (gemvM
        # has no 'sum' prologue), which is a mailbox hand-off too.
        assert info["mailboxes"] == (5 if gemvM else 4)
    s.reset_outputs()
    ch.run()
    assert not ch.status()
    s.check_against_oracle(s.read(), f"chain M={M} gemvM={gemvM}")
    ch.free()
    s.free()


@pytest.mark.parametrize("M", [8, 16])
def test_wide_chain_fp32_staging_predicted(dev, M):
    """the wide kernel: qkv's outputs lie far beyond the producer's 2^8 fp16 staging, o's back inside it, so o's waves
    find their staged halves marked and take the fp32 x', and with knob 14 on gate_up's waves then load the fp32 x'
    straight away: they must build the same operands as the staged halves (fixed 2^8 scale where it fits), so every
    output equals the run with knob 14 off bit for bit, and each op matches the oracle"""
    s = MiniStep(M=M, gemvM=True, seed=40 + M)
    for name, rows, K, sd, sigma in (("w_qkv", s.QKV, s.D, 41, 400.0), ("w_o", s.D, s.D, 42, 4e-4)):
        s.host[name] = O.pack_q4(O.randn(rows * K, sd, sigma), rows, K)[0]
        s.dev[name].free()
        s.dev[name] = capi.to_device(s.host[name])
    outs = {}
    for knob in (1, 0):
        old = capi.chain_tune(14, knob)
        try:
            ch = s.make_chain()
        finally:
            capi.chain_tune(14, old)
        info = ch.info()
        print("chain", info, flush=True)
        assert info["waves_per_workgroup"] == 12 and info["passes"] == 1 and info["staged"] >= 2
        s.reset_outputs()
        ch.run()
        assert not ch.status()
        outs[knob] = s.read()
        ch.free()
    qkv_q = outs[1]["qkv"].reshape(M, s.QKV)[:, :s.D]   # the rows o reads
    assert np.max(np.abs(qkv_q)) > 255 * 16 and np.max(np.abs(outs[1]["o"])) < 200
    for k in outs[1]:
        assert np.array_equal(outs[1][k].view(np.uint32), outs[0][k].view(np.uint32)), k
    s.check_against_oracle(outs[1], f"wide chain M={M}, fp32 staging predicted")
    s.free()


@pytest.mark.parametrize("M,wide", [(6, 0), (11, 0), (16, 0), (6, 1), (8, 1), (11, 1), (16, 1)])
def test_chain_row_group_passes(dev, M, wide):
    """a gemvM chain of 6-16 rows runs in one launch of the wide pipelined kernel (p0_chain_tune knob 12 on, the
    default), or, with it off, as pipelined passes over row groups of at most 5 rows (6 = 3 + 3, 11 = 4 + 4 + 3,
    16 = 4 x 4), one launch each: every op against the oracle, a rerun, and replays of a recording of the run
    (bit-identical to the eager run)"""
    s = MiniStep(M=M, gemvM=True, seed=70 + M)
    old = capi.chain_tune(12, wide)
    try:
        ch = s.make_chain()
    finally:
        capi.chain_tune(12, old)
    info = ch.info()
    print("chain", info, flush=True)
    assert info["passes"] == (1 if wide else (M + 4) // 5) and info["waves_per_workgroup"] == 12 and info["m"] == M
    for r in range(2):
        s.reset_outputs()
        ch.run()
        assert not ch.status()
        s.check_against_oracle(s.read(), f"chain M={M} run {r}")
    want = s.read()
    rec = capi.record(ch.run)
    for r in range(2):
        s.reset_outputs()
        rec.replay()
        capi.done()
        got = s.read()
        for k in want:
            assert np.array_equal(want[k].view(np.uint32), got[k].view(np.uint32)), f"replay {r}: {k}"
    assert not ch.status()
    rec.free()
    ch.free()
    s.free()


@pytest.mark.parametrize("wide", [1, 0])
def test_chain_rows_sharing_memory_take_the_general_kernel(dev, wide):
    """rows of different row groups that share memory (op 1 reads x rows 128 floats apart, each 256 long: row m reads
    op 0's output around its row m / 2, so rows 4-7 read rows 2-3) run in one pass of the wide kernel, which needs no
    row independence; with it off (knob 12) they cannot run as row-group passes, and the chain takes the general
    kernel, one launch; both match the oracle"""
    M, N0, K = 8, 256, 256
    w0, w1 = _w(N0, K, 81), _w(128, K, 82)
    x = O.randn(M * K, 83)
    dv = {"w0": capi.to_device(w0), "w1": capi.to_device(w1), "x": capi.to_device(x),
          "y0": capi.Buffer(4 * M * N0), "y1": capi.Buffer(4 * M * 128)}
    raw, store = capi.PRO["raw"], capi.EPI["store"]

    def ops(b):
        return [dict(w=b["w0"], w_rows=N0, w_cols=K, x=b["x"], N=N0, K=K, pro=raw, epi=store, y=b["y0"], M=M,
                     x_ldx=K, y_ldm=N0, y_ldy=M * N0),
                dict(w=b["w1"], w_rows=128, w_cols=K, x=b["y0"], N=128, K=K, pro=raw, epi=store, y=b["y1"], M=M,
                     x_ldx=128, y_ldm=128, y_ldy=M * 128)]

    def enqueue():
        for f in ops(dv):
            capi.q4_gemvM(capi.gemvm_args(**f))

    for k in ("y0", "y1"):
        dv[k].fill_u32(NAN)
    old = capi.chain_tune(12, wide)
    try:
        ch = capi.chain(enqueue)
    finally:
        capi.chain_tune(12, old)
    info = ch.info()
    print("chain", info, flush=True)
    assert info["passes"] == 1 and info["waves_per_workgroup"] == (12 if wide else 8)
    ch.run()
    assert not ch.status()
    g0 = dv["y0"].read(np.float32, M * N0)
    g1 = dv["y1"].read(np.float32, M * 128)
    # op 1 reads rows up to (M - 1) * 128 + K floats of y0: inside its M * N0 floats
    want0 = np.full(M * N0, np.nan, np.float32)
    want1 = np.full(M * 128, np.nan, np.float32)
    host = {"w0": w0.ctypes.data, "w1": w1.ctypes.data, "x": x.ctypes.data, "y0": want0.ctypes.data,
            "y1": want1.ctypes.data}
    f0, f1 = ops(host)
    O.q4_gemvM(capi.gemvm_args(**f0))
    _check(g0, want0, "op 0")
    g0c = np.ascontiguousarray(g0)
    O.q4_gemvM(capi.gemvm_args(**dict(f1, x=g0c.ctypes.data)))
    _check(g1, want1, "op 1")
    ch.free()
    for b in dv.values():
        b.free()


@pytest.mark.parametrize("M,knob", [(1, 6), (3, 11), (5, 11)])
def test_chain_loader_depth_not_default(dev, M, knob):
    """the pipelined chain with the loader depth its rows do not take by default (p0_chain_tune knob 6: M = 1,
    default 2 slots in flight per loader; knob 11: M > 1, default 1)"""
    s = MiniStep(M=M, gemvM=M > 1, seed=60 + M)
    old = capi.chain_tune(knob, 1 if knob == 6 else 2)
    try:
        ch = s.make_chain()
    finally:
        capi.chain_tune(knob, old)
    assert ch.info()["waves_per_workgroup"] == 12
    for r in range(2):
        s.reset_outputs()
        ch.run()
        assert not ch.status()
        s.check_against_oracle(s.read(), f"chain M={M} knob {knob} run {r}")
    ch.free()
    s.free()


@pytest.mark.parametrize("M", [2, 3, 5])
def test_chain_rows_not_16_byte_aligned(dev, M):
    """M > 1 rows are staged with 16-byte loads when an op's row start and stride allow them, else element by
    element: the o op here reads the qkv output from element 1 of each row on, and must still match the oracle"""
    s = MiniStep(M=M, gemvM=True, seed=40 + M)
    base_ops = s.ops

    def ops(b):
        o = base_ops(b)
        o[1]["x_rowB"] = 1   # K = D elements from 1 on, inside each QKV-long row
        return o

    s.ops = ops
    ch = s.make_chain()
    assert ch.info()["m"] == M
    s.reset_outputs()
    ch.run()
    assert not ch.status()
    s.check_against_oracle(s.read(), f"chain M={M} o at row offset 1")
    ch.free()
    s.free()


def test_chain_reruns_are_identical_and_reset(dev):
    """the chain leaves its counts at zero: every run computes the same bits (fixed plan, ordered reductions)"""
    s = MiniStep(seed=21)
    ch = s.make_chain()
    first = None
    for r in range(4):
        s.reset_outputs()
        ch.run()
        assert not ch.status()
        got = s.read()
        if first is None:
            first = got
            s.check_against_oracle(got, "chain run 0")
        else:
            for k in first:
                assert np.array_equal(first[k].view(np.uint32), got[k].view(np.uint32)), f"run {r}: {k}"
    ch.free()
    s.free()


def test_chain_equals_standalone_calls(dev):
    """the same ops launched one by one agree with the chain to the fp32 bar"""
    s = MiniStep(seed=31)
    ch = s.make_chain()
    s.reset_outputs()
    ch.run()
    assert not ch.status()
    chained = s.read()
    s.reset_outputs()
    s._enqueue()
    capi.done()
    single = s.read()
    for k in ("qkv", "o", "gu", "dn", "sum", "hd"):
        _check(chained[k], single[k], f"chain vs standalone {k}")
    ch.free()
    s.free()


def test_chain_layers_reuse_buffers(dev):
    """Six layers that read and rewrite the same two buffers (a -> b -> a ...), then two ops that write one output.
    Each op must read what the op before it wrote in this run, never a copy that an earlier layer left in a cache, and
    the last writer of a buffer must win. The final a is checked against the oracle run op by op on the host (twelve
    dependent fp32 GEMVs: relative L2 within 1e-4, the fp32 bar compounded); the last writer's output exactly, to the
    fp32 bar, on the chain's own input."""
    D, L = 256, 6
    ws = [_w(D, D, 100 + i) for i in range(2 * L + 2)]
    a0 = O.randn(D, 99)
    wd = [capi.to_device(w) for w in ws]
    a, b, z = capi.to_device(a0), capi.Buffer(4 * D), capi.Buffer(4 * D)

    def op(w, x, y):
        capi.q4_gemv(capi.gemv_args(w=w, w_rows=D, w_cols=D, x=x, N=D, K=D, y=y))

    def enqueue():
        for l in range(L):
            op(wd[2 * l], a, b)
            op(wd[2 * l + 1], b, a)
        op(wd[2 * L], a, z)
        op(wd[2 * L + 1], a, z)

    ch = capi.chain(enqueue)
    want = a0.copy()
    for i in range(2 * L):
        y = np.zeros(D, np.float32)
        O.q4_gemv(capi.gemv_args(w=ws[i].ctypes.data, w_rows=D, w_cols=D, x=want.ctypes.data, N=D, K=D,
                                 y=y.ctypes.data))
        want = y
    for r in range(3):
        a.upload(a0)
        b.fill_u32(NAN)
        z.fill_u32(NAN)
        ch.run()
        assert not ch.status()
        ga, gz = a.read(np.float32), z.read(np.float32)
        r_a = rel_l2(ga, want)
        print(f"run {r}: final a rel_l2 {r_a:.3e}", flush=True)
        assert np.all(np.isfinite(ga)) and r_a <= 1e-4
        wz = np.zeros(D, np.float32)
        O.q4_gemv(capi.gemv_args(w=ws[2 * L + 1].ctypes.data, w_rows=D, w_cols=D, x=ga.ctypes.data, N=D, K=D,
                                 y=wz.ctypes.data))
        _check(gz, wz, f"run {r}: last writer of z")
    ch.free()
    for buf in wd + [a, b, z]:
        buf.free()


@pytest.mark.parametrize("knobs", [{0: 8}, {4: 0}, {1: 2, 4: 0}, {0: 8, 4: 0}, {7: 0}])
def test_chain_other_plans(dev, knobs):
    """8-wave workgroups; every op streamed (no LDS staging); streamed ops with K split across workgroups inside
    the chain (cross-workgroup reduction + counts); the pipelined chain without mailbox hand-offs"""
    old = {k: capi.chain_tune(k, v) for k, v in knobs.items()}
    try:
        s = MiniStep(seed=41 + sum(knobs))
        ch = s.make_chain()
    finally:
        for k, v in old.items():
            capi.chain_tune(k, v)
    print("chain", ch.info(), flush=True)
    for _ in range(2):
        s.reset_outputs()
        ch.run()
        assert not ch.status()
        s.check_against_oracle(s.read(), f"chain knobs {knobs}")
    ch.free()
    s.free()


def test_chain_inside_recording(dev):
    """a chain run captured into a recording replays correctly, with eager work between the replays"""
    s = MiniStep(seed=51)
    ch = s.make_chain()
    s.reset_outputs()
    ch.run()
    want = s.read()
    rec = capi.record(ch.run)
    for r in range(3):
        s.reset_outputs()
        rec.replay()
        capi.done()
        got = s.read()
        for k in want:
            assert np.array_equal(want[k].view(np.uint32), got[k].view(np.uint32)), f"replay {r}: {k}"
    assert not ch.status()
    rec.free()
    ch.free()
    s.free()


def test_chain_large_ops(dev):
    """decode-sized ops: a head with two tiles per wave (65536 rows) after a 2048-wide qkv, checked on sampled rows"""
    D, V = 2048, 65536
    w1 = O.fill_q4_sym(3072, D, 5, 0.02)
    w2 = O.fill_q4_sym(V, 3072, 6, 0.02)
    x = O.randn(D, 7)
    b = {k: capi.to_device(v) for k, v in dict(w1=w1, w2=w2, x=x).items()}
    y1, y2 = capi.Buffer(3072 * 4).fill_u32(NAN), capi.Buffer(V * 4).fill_u32(NAN)

    def enqueue():
        capi.q4_gemv(capi.gemv_args(w=b["w1"], w_rows=3072, w_cols=D, x=b["x"], N=3072, K=D, y=y1))
        capi.q4_gemv(capi.gemv_args(w=b["w2"], w_rows=V, w_cols=3072, x=y1, N=V, K=3072, y=y2))

    ch = capi.chain(enqueue)
    print("chain", ch.info(), flush=True)
    ch.run()
    assert not ch.status()
    g1, g2 = y1.read(np.float32), y2.read(np.float32)
    want1 = np.full(3072, np.nan, np.float32)
    O.q4_gemv(capi.gemv_args(w=w1.ctypes.data, w_rows=3072, w_cols=D, x=x.ctypes.data, N=3072, K=D,
                             y=want1.ctypes.data))
    _check(g1, want1, "large chain op 0")
    rows = np.r_[0:64, 30000:30064, V - 64:V]
    tiles = np.unique(rows // 64)
    sub = np.concatenate([w2.reshape(V // 64, -1)[t] for t in tiles])     # the sampled tiles' records
    want2 = np.full(len(tiles) * 64, np.nan, np.float32)
    O.q4_gemv(capi.gemv_args(w=sub.ctypes.data, w_rows=len(tiles) * 64, w_cols=3072, x=g1.ctypes.data,
                             N=len(tiles) * 64, K=3072, y=want2.ctypes.data))
    _check(g2[np.concatenate([np.arange(t * 64, t * 64 + 64) for t in tiles])], want2, "large chain op 1 (sampled)")
    assert np.all(np.isfinite(g2))
    ch.free()
    for v in list(b.values()) + [y1, y2]:
        v.free()


def test_chain_bounded_wait_reports_and_recovers(dev):
    """waits forced from the host to give up (knob 3) are reported by p0_chain_status, the launch still ends, and the
    next run with normal waits is correct again (the status call resets the chain and split-K counters)"""
    D, V = 2048, 65536
    w1 = O.fill_q4_sym(V, D, 8, 0.02)
    w2 = O.fill_q4_sym(V, D, 9, 0.02)
    x = O.randn(D, 10)
    b = {k: capi.to_device(v) for k, v in dict(w1=w1, w2=w2, x=x).items()}
    y1, y2 = capi.Buffer(V * 4), capi.Buffer(V * 4)

    def enqueue():
        capi.q4_gemv(capi.gemv_args(w=b["w1"], w_rows=V, w_cols=D, x=b["x"], N=V, K=D, y=y1))
        capi.q4_gemv(capi.gemv_args(w=b["w2"], w_rows=V, w_cols=D, x=y1, x_rowB=4096, N=V, K=D, y=y2))

    ch = capi.chain(enqueue)
    assert capi.chain_tune(3, 1) == 0
    try:
        ch.run()
        assert ch.status(), "waits forced to give up must be reported"
        assert not ch.status(), "the timed-out mark is cleared once read"
    finally:
        capi.chain_tune(3, 0)
    y1.fill_u32(NAN)
    y2.fill_u32(NAN)
    ch.run()
    assert not ch.status()
    g1, g2 = y1.read(np.float32), y2.read(np.float32)
    assert np.all(np.isfinite(g2))
    want = np.full(128, np.nan, np.float32)
    head = np.ascontiguousarray(w2[:2 * (D // 32) * 1280])            # tiles 0 and 1
    O.q4_gemv(capi.gemv_args(w=head.ctypes.data, w_rows=128, w_cols=D, x=g1.ctypes.data, x_rowB=4096, N=128, K=D,
                             y=want.ctypes.data))
    _check(g2[:128], want, "after recovery")
    ch.free()
    for v in list(b.values()) + [y1, y2]:
        v.free()


def test_chain_errors(dev):
    capi.check(capi.lib().p0_chain_begin())
    with pytest.raises(capi.P0Error, match="already being built"):
        capi.check(capi.lib().p0_chain_begin())
    with pytest.raises(capi.P0Error, match="holds no ops"):
        capi.check(capi.lib().p0_chain_end(capi.C.byref(capi.vp())))
    w, x, y = capi.to_device(_w(64, 64, 1)), capi.to_device(O.randn(64, 2)), capi.Buffer(256)

    def mixed():
        capi.q4_gemv(capi.gemv_args(w=w, w_rows=64, w_cols=64, x=x, N=64, K=64, y=y))
        capi.q4_gemvM(capi.gemvm_args(w=w, w_rows=64, w_cols=64, x=x, x_ldx=0, M=2, N=64, K=64, y=y))

    with pytest.raises(capi.P0Error, match="one M"):
        capi.chain(mixed)
    # the failed build left no chain open: a fresh one builds
    ch = capi.chain(lambda: capi.q4_gemv(capi.gemv_args(w=w, w_rows=64, w_cols=64, x=x, N=64, K=64, y=y)))
    ch.run()
    assert not ch.status()
    ch.free()
    for v in (w, x, y):
        v.free()


def test_chain_mailboxes_match_flags(dev):
    """Mailbox hand-offs (an op polls the previous op's tagged outputs instead of its completion flags) compute the
    same bits as the flag hand-offs, run after run: the x values an op stages are the same floats either way. Checked
    over the mini step (store -> raw, store -> rms, geglu -> raw into a 2-split op, and rms into the softcap head) and
    over a chain of layers that read and rewrite the same two buffers (every op after the first a mailbox consumer)."""
    s = MiniStep(seed=61)
    old = capi.chain_tune(7, 1)
    try:
        ch_m = s.make_chain()
        capi.chain_tune(7, 0)
        ch_f = s.make_chain()
    finally:
        capi.chain_tune(7, old)
    im, iff = ch_m.info(), ch_f.info()
    print("mailbox chain", im, "flag chain", iff, flush=True)
    if im["waves_per_workgroup"] != 12:
        pytest.skip("this device plans the general chain kernel (mailboxes are a pipelined-chain feature)")
    assert im["mailboxes"] == 4 and iff["mailboxes"] == 0
    res = []
    for ch in (ch_f, ch_m, ch_m, ch_f, ch_m):
        s.reset_outputs()
        ch.run()
        assert not ch.status()
        res.append(s.read())
    s.check_against_oracle(res[1], "mailbox chain")
    for r in res[1:]:
        for k in res[0]:
            assert np.array_equal(res[0][k].view(np.uint32), r[k].view(np.uint32)), k
    ch_m.free()
    ch_f.free()
    s.free()

    D, L = 512, 5
    ws = [_w(D, D, 300 + i) for i in range(2 * L)]
    wd = [capi.to_device(w) for w in ws]
    a0 = O.randn(D, 301)
    a, b = capi.to_device(a0), capi.Buffer(4 * D)

    def enqueue():
        for l in range(L):
            capi.q4_gemv(capi.gemv_args(w=wd[2 * l], w_rows=D, w_cols=D, x=a, N=D, K=D, y=b))
            capi.q4_gemv(capi.gemv_args(w=wd[2 * l + 1], w_rows=D, w_cols=D, x=b, N=D, K=D, y=a))

    old = capi.chain_tune(7, 1)
    try:
        ch_m = capi.chain(enqueue)
        capi.chain_tune(7, 0)
        ch_f = capi.chain(enqueue)
    finally:
        capi.chain_tune(7, old)
    assert ch_m.info()["mailboxes"] == 2 * L - 1 and ch_f.info()["mailboxes"] == 0
    outs = []
    for ch in (ch_f, ch_m, ch_m):
        a.upload(a0)
        ch.run()
        assert not ch.status()
        outs.append(a.read(np.float32, D))
    want = a0.copy()
    for i in range(2 * L):
        y = np.zeros(D, np.float32)
        O.q4_gemv(capi.gemv_args(w=ws[i].ctypes.data, w_rows=D, w_cols=D, x=want.ctypes.data, N=D, K=D,
                                 y=y.ctypes.data))
        want = y
    r = rel_l2(outs[1], want)
    print(f"10 dependent GEMVs through mailboxes: rel_l2 {r:.3e}", flush=True)
    assert r <= 1e-4
    for o in outs[1:]:
        assert np.array_equal(outs[0].view(np.uint32), o.view(np.uint32))
    ch_m.free()
    ch_f.free()
    for buf in wd + [a, b]:
        buf.free()


def _both_chains(enqueue):
    """the same ops planned with and without mailbox hand-offs"""
    old = capi.chain_tune(7, 1)
    try:
        ch_m = capi.chain(enqueue)
        capi.chain_tune(7, 0)
        ch_f = capi.chain(enqueue)
    finally:
        capi.chain_tune(7, old)
    return ch_m, ch_f


def _gemv(w, N, K, x, y, **kw):
    capi.q4_gemv(capi.gemv_args(w=w, w_rows=kw.pop("w_rows", N), w_cols=K, x=x, N=N, K=K, y=y, **kw))


def test_chain_mailbox_cases(dev):
    """Which hand-offs take a mailbox, and that each computes what the flag hand-off computes:
      a. op 1 reads x at an offset inside op 0's output (rows 128..383 of 384): mailbox, and so does op 2 (op 1's
         whole output; a consumer may itself be a producer);
      b. op 3 writes into op 2's output (write after write): flags;
      c. op 5, 16 K-splits, reads op 4's output, which op 4 writes with large per-workgroup shares (one wave per
         64-row unit): mailbox;
      d. op 7 reads x running past op 6's output (rows 64..319 of a 256-row output): flags.
    Every output is compared bit for bit between the two chains, and (a) and (c) with the oracle."""
    D = 256
    ws = {"w384": _w(384, D, 401), "w256": _w(D, D, 402), "wbig": _w(32768, 2048, 403), "wback": _w(2048, 32768, 404)}
    dv = {k: capi.to_device(v) for k, v in ws.items()}
    x0 = O.randn(2048, 405)
    tail = O.randn(512, 406)
    x = capi.to_device(x0)
    sizes = {"p384": 384, "o1": D, "bB": 512, "big": 32768, "back": 16 * 2048, "o2": 512, "o3": D}
    b = {k: capi.Buffer(4 * n) for k, n in sizes.items()}

    def enqueue():
        _gemv(dv["w384"], 384, D, x, b["p384"])                                   # 0
        _gemv(dv["w256"], D, D, b["p384"], b["o1"], x_rowB=128)                   # 1 (a)
        _gemv(dv["w384"], 384, D, b["o1"], b["bB"])                               # 2
        _gemv(dv["w256"], D, D, b["bB"], b["bB"].ptr + 4 * 256)                   # 3 (b)
        _gemv(dv["wbig"], 32768, 2048, x, b["big"])                               # 4
        _gemv(dv["wback"], 2048, 32768, b["big"], b["back"], kPer=2048)           # 5 (c)
        _gemv(dv["w256"], D, D, b["o1"], b["o2"])                                 # 6
        _gemv(dv["w256"], D, D, b["o2"].ptr + 4 * 64, b["o3"])                    # 7 (d)

    ch_m, ch_f = _both_chains(enqueue)
    im = ch_m.info()
    print("mailbox chain", im, flush=True)
    if im["waves_per_workgroup"] != 12:
        pytest.skip("this device plans the general chain kernel (mailboxes are a pipelined-chain feature)")
    assert im["mailboxes"] == 3 and ch_f.info()["mailboxes"] == 0
    outs = []
    for ch in (ch_f, ch_m, ch_m):
        for k in b:
            b[k].fill_u32(NAN)
        b["o2"].upload(tail)   # rows 256.. of o2 are read by op 7 and written by no op
        ch.run()
        assert not ch.status()
        outs.append({k: b[k].read(np.float32) for k in b})
    for r in outs[1:]:
        for k in b:
            assert np.array_equal(outs[0][k].view(np.uint32), r[k].view(np.uint32)), k
    got = outs[1]
    for k in b:
        assert np.all(np.isfinite(got[k])), k

    def ref(w, N, K, xin, kPer=0, nsplit=1):
        y = np.zeros(N * nsplit, np.float32)
        xin = np.ascontiguousarray(xin, np.float32)
        O.q4_gemv(capi.gemv_args(w=ws[w].ctypes.data, w_rows=N, w_cols=K, x=xin.ctypes.data, N=N, K=K,
                                 y=y.ctypes.data, kPer=kPer))
        return y
    _check(got["p384"], ref("w384", 384, D, x0[:D]), "op 0")
    _check(got["o1"], ref("w256", D, D, got["p384"][128:384]), "op 1 (mailbox at an offset)")
    _check(got["big"], ref("wbig", 32768, 2048, x0), "op 4 (large shares)")
    _check(got["back"], ref("wback", 2048, 32768, got["big"], kPer=2048, nsplit=16), "op 5 (mailbox, 16 splits)")
    _check(got["o3"], ref("w256", D, D, got["o2"][64:320]), "op 7 (flags: x past the producer's rows)")
    ch_m.free()
    ch_f.free()
    for buf in list(dv.values()) + [x] + list(b.values()):
        buf.free()


@pytest.mark.parametrize("enc", ["q4", "q8"])
def test_chain_small_and_ragged_shapes(dev, enc):
    """The pipelined chain at the edges of its slots: one group (K = 32 / 64), a K that leaves most of a slot empty,
    a ragged last K-split (K = 320, kPer = 128: splits of 128, 128 and 64 k; q8: K = 384, kPer = 256: 256 and 128), the
    fewest rows (N = 64) and a softcap on one tile, each op checked against the oracle on the input it read"""
    G = 32 if enc == "q4" else 64
    pack = (lambda w, r, k: O.pack_q4(w, r, k)[0]) if enc == "q4" else (lambda w, r, k: O.pack_q8(w, r, k)[0])
    we = 1 if enc == "q4" else 2
    Kr, kPr = (320, 128) if enc == "q4" else (384, 256)
    ops = [   # (N, K, kPer, epi, input)
        (64, G, 0, "store", "x"),
        (256, 64, 0, "store", 0),
        (192, 3 * G, 0, "store", 1),
        (64, 192, 0, "softcap", 2),
        (Kr, 64, 0, "store", 1),
        (128, Kr, kPr, "store", 4),
    ]
    x0 = O.randn(256, 601)
    ws = [pack(O.randn(N * K, 610 + i, 0.05), N, K) for i, (N, K, kPer, epi, src) in enumerate(ops)]
    dw = [capi.to_device(w) for w in ws]
    x = capi.to_device(x0)
    nsp = [(-(-K // kPer) if kPer else 1) for (N, K, kPer, epi, src) in ops]
    ys = [capi.Buffer(4 * N * s) for (N, K, kPer, epi, src), s in zip(ops, nsp)]
    mx0 = np.zeros(16, np.float32)
    mx0[3] = 0.8
    mx = capi.to_device(mx0)

    def f(i, b_in, b_out, mxp):
        N, K, kPer, epi, src = ops[i]
        d = dict(w=dw[i] if mxp is None else ws[i].ctypes.data, w_enc=we, w_rows=N, w_cols=K, x=b_in, N=N, K=K, kPer=kPer,
                 epi=capi.EPI[epi], y=b_out)
        if epi == "softcap":
            d.update(mx=mx if mxp is None else mxp, pro=capi.PRO["rms"], stat=mx if mxp is None else mxp, stat_off=3,
                     norm=x if mxp is None else x0.ctypes.data)
        return d

    def enqueue():
        for i, (N, K, kPer, epi, src) in enumerate(ops):
            capi.q4_gemv(capi.gemv_args(**f(i, x if src == "x" else ys[src], ys[i], None)))

    ch = capi.chain(enqueue)
    print("chain", ch.info(), flush=True)
    for b in ys:
        b.fill_u32(NAN)
    mx.upload(mx0)
    ch.run()
    assert not ch.status()
    got = [b.read(np.float32) for b in ys]
    gmx = mx.read(np.float32)
    mxh = mx0.copy()
    for i, (N, K, kPer, epi, src) in enumerate(ops):
        xin = np.ascontiguousarray(x0 if src == "x" else got[src], np.float32)
        y = np.full(N * nsp[i], np.nan, np.float32)
        O.q4_gemv(capi.gemv_args(**f(i, xin.ctypes.data, y.ctypes.data, mxh.ctypes.data)))
        _check(got[i], y, f"{enc} op {i} N {N} K {K} kPer {kPer} {epi}")
    assert np.allclose(gmx[0], mxh[0], rtol=1e-5, atol=1e-6) and gmx[1].view(np.uint32) == mxh[1].view(np.uint32)
    ch.free()
    for b in dw + ys + [x, mx]:
        b.free()
