"""GPU parity of the chain ops that are not GEMVs (p0pc0rn_amd/csrc/chain_aux.hpp): p0_copy, p0_argmax / p0_argmaxM,
p0_rowstats and p0_normadd called while a chain is being built join the chain, so a whole decode token (the reference's
command buffer: engine/llm/gemma4.js:503-511's rstd copy, softcap head and argmax, then DecodeRunner.end's result copy,
engine/llm/drunner.js:82-90) is one launch.

Each aux op in a chain must give the standalone op's result bit for bit (the same sums in the same order), which the
oracle pins (tests/test_misc_oracle.py). Dependencies are checked by data: every buffer an op writes is NaN-filled
before the run, and ops read what the op before them wrote (a copy's output feeds rowstats, a rowstats slot feeds a
GEMV's rms prologue, a head's tile maxima feed the argmax, the argmax feeds the result copy).
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2
from tests.test_chain_gpu import MiniStep

pytestmark = pytest.mark.gpu
NAN = 0x7FC00000


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_aux_only_chain_matches_oracle(dev):
    """copy -> rowstats (both modes) -> normadd (both modes) -> argmaxM, one chain of no GEMV, run twice; each result
    against the oracle bit for bit on the input the chain's previous op wrote"""
    R, C, ld, c0 = 5, 700, 711, 3
    src = (2.0 + O.randn(R * ld, 90)).astype(np.float32)
    D, M, nsrc, ldp = 2048, 3, 2, 3 * 2048 + 64
    t = O.randn(nsrc * ldp, 91, 0.3).astype(np.float32)
    w = (0.5 + O.rng_uniform(92, D)).astype(np.float32)
    x0 = O.randn(M * D, 93).astype(np.float32)
    n, MA = 4096, 2
    rng = np.random.default_rng(94)
    mx = np.zeros(2 * n * MA, np.float32)
    mx[0::2] = rng.integers(-40, 40, n * MA).astype(np.float32)   # ties everywhere
    mx[1::2] = rng.integers(0, 1 << 24, n * MA).astype(np.uint32).view(np.float32)

    d = {k: capi.to_device(v) for k, v in dict(src=src, t=t, w=w, x=x0, mx=mx).items()}
    cp = capi.Buffer(src.nbytes)
    st0 = capi.Buffer((R + 1) * 8)
    st1 = capi.Buffer((R + 1) * 8)
    xs = [capi.Buffer(x0.nbytes) for _ in range(2)]
    sts = [capi.Buffer((M + 2) * 4) for _ in range(2)]
    out = capi.Buffer(2 * MA * 4)
    nk = dict(t_n=nsrc, t_ld=ldp, w_off=0, st_off=2, D=D, M=M, eps=1e-6, scale=0.9)

    def token():
        capi.copy(d["src"], 0, cp, 0, src.nbytes)
        for mode, st in ((0, st0), (1, st1)):
            capi.rowstats(capi.rowstats_args(x=cp, x_ld=ld, x_c0=c0, rows=R, cols=C, mode=mode, eps=1e-5, st=st,
                                             st_off=1))
        for mode in (0, 1):
            capi.copy(d["x"], 0, xs[mode], 0, x0.nbytes)
            capi.normadd(capi.normadd_args(t=d["t"], w=d["w"], x=xs[mode], st=sts[mode], mode=mode, **nk))
        capi.argmaxM(d["mx"], n, MA, out)

    ch = capi.chain(token)
    info = ch.info()
    assert info["n_ops"] == 8 and info["passes"] == 1, info
    for run in range(2):
        for b in [cp, st0, st1, out] + xs + sts:
            b.fill_u32(NAN)
        ch.run()
        assert ch.status() == 0
        got_cp = cp.read(np.float32)
        assert np.array_equal(_bits(got_cp), _bits(src)), "copy"
        for mode, st in ((0, st0), (1, st1)):
            want = np.full((R + 1) * 2, np.nan, np.float32)
            O.rowstats(capi.rowstats_args(x=got_cp.ctypes.data, x_ld=ld, x_c0=c0, rows=R, cols=C, mode=mode,
                                          eps=1e-5, st=want.ctypes.data, st_off=1))
            assert np.array_equal(_bits(st.read(np.float32)[2:]), _bits(want[2:])), f"rowstats mode {mode}"
        for mode in (0, 1):
            xw, sw = x0.copy(), np.full(M + 2, np.nan, np.float32)
            O.normadd(capi.normadd_args(t=t.ctypes.data, w=w.ctypes.data, x=xw.ctypes.data, st=sw.ctypes.data,
                                        mode=mode, **nk))
            assert np.array_equal(_bits(xs[mode].read(np.float32)), _bits(xw)), f"normadd x mode {mode}"
            assert np.array_equal(_bits(sts[mode].read(np.float32)[2:]), _bits(sw[2:])), f"normadd st mode {mode}"
        want = O.argmaxM(mx, n, MA)
        assert np.array_equal(out.read(np.uint32), np.asarray(want, np.uint32).ravel()), "argmaxM"
        print(f"aux-only chain run {run}: copy, rowstats x2, normadd x2, argmaxM bit-exact", flush=True)
    ch.free()
    for b in list(d.values()) + [cp, st0, st1, out] + xs + sts:
        b.free()


class TokenStep(MiniStep):
    """MiniStep as a whole decode token: after the layer ops, the rstd copy into the head's stat slot, the softcap
    head (rms, its rstd read from that slot), the argmax over its tile maxima and the copy of the result words into a
    staging buffer (engine/llm/gemma4.js:503-511, engine/llm/drunner.js:82-90)"""

    def __init__(self, M=1, **kw):
        super().__init__(M=M, gemvM=M > 1, **kw)
        NT = self.V // 64
        self.host["mx"][self.mx_stat_off::2][:M] = 0.85   # what the rstd copy writes (the oracle reads it here)
        self.dev["mx"].upload(self.host["mx"])
        self.rsrc = capi.to_device(np.array([0.0, 0.85, 0.0, 0.0] * M, np.float32))   # rstd(x) of each row at 4 m + 1
        self.arg = capi.Buffer(max(16, 8 * M))
        self.stage = capi.Buffer(max(16, 8 * M))
        self.NT = NT

    def enqueue_token(self):
        ops = self.ops(self.dev | self.out)
        for f in ops[:-1]:
            (capi.q4_gemvM if self.gemvM else capi.q4_gemv)(self._args(f))
        for m in range(self.M):   # the rstd copy (one slot per row)
            capi.copy(self.rsrc, (4 * m + 1) * 4, self.dev["mx"], (self.mx_stat_off + 2 * m) * 4, 4)
        (capi.q4_gemvM if self.gemvM else capi.q4_gemv)(self._args(ops[-1]))
        if self.M == 1:
            capi.argmax(self.dev["mx"], self.NT, self.arg)
        else:
            capi.argmaxM(self.dev["mx"], self.NT, self.M, self.arg)
        capi.copy(self.arg, 0, self.stage, 0, 8 * self.M)

    def free_token(self):
        for b in (self.rsrc, self.arg, self.stage):
            b.free()


@pytest.mark.parametrize("M", [1, 3, 5, 8, 16])
def test_token_chain_ends_in_argmax_and_result_copy(dev, M):
    """a whole token as one chain (M = 1 decode, M = 3 and 5 verify passes on the pipelined kernel, 8 and 16 on the wide
    one): the
    head reads the rstd the chain copied, the argmax reads the head's tile maxima, the staging buffer gets the argmax
    words; each op against the oracle on the input it read, the argmax against the oracle's over the head's maxima"""
    print("case token chain M", M, flush=True)
    s = TokenStep(M=M)
    ch = capi.chain(s.enqueue_token)
    info = ch.info()
    assert info["n_ops"] == 6 + M + 2, info
    assert info["passes"] == 1, info
    for run in range(2):
        s.reset_outputs()
        for b in (s.arg, s.stage):
            b.fill_u32(NAN)
        mx = s.host["mx"].copy()
        mx[s.mx_stat_off::2][:M] = np.nan   # the copy must have landed before the head reads its rstd
        s.dev["mx"].upload(mx)
        ch.run()
        assert ch.status() == 0
        got = s.read()
        np.testing.assert_array_equal(got["mx"][s.mx_stat_off::2][:M], np.float32(0.85))
        s.check_against_oracle(got, f"token chain M={M} run {run}")
        want = np.asarray(O.argmaxM(got["mx"], s.NT, M), np.uint32).ravel()
        assert np.array_equal(s.arg.read(np.uint32)[:2 * M], want), "argmax of the head's tile maxima"
        assert np.array_equal(s.stage.read(np.uint32)[:2 * M], want), "the result copy"
        for m in range(M):   # the argmax row's logit is the largest of the row (the head output the chain wrote)
            hd = got["hd"][m * s.V:(m + 1) * s.V]
            assert want[2 * m] == int(np.argmax(hd)) and hd[want[2 * m]] == np.float32(want[2 * m + 1:2 * m + 2].view(np.float32)[0])
    ch.free()
    s.free_token()


@pytest.mark.parametrize("M", [1, 3, 8])
def test_token_chain_forced_give_up_reports_and_recovers(dev, M):
    """every wait of a token chain forced to give up at once (knob 3; M = 1 and 3 on the pipelined kernel, 8 on the wide
    one, with the copy, the argmax and the result copy in the chain): the launch ends, p0_chain_status reports the run
    once, and the next run with normal waits is correct. The compute waves that leave early release their
    workgroup's barrier, so none of the others waits for them."""
    print("case forced give-up M", M, flush=True)
    s = TokenStep(M=M)
    ch = capi.chain(s.enqueue_token)
    assert capi.chain_tune(3, 1) == 0
    try:
        s.reset_outputs()
        ch.run()
        assert ch.status(), "waits forced to give up must be reported"
        assert not ch.status(), "the timed-out mark is cleared once read"
    finally:
        capi.chain_tune(3, 0)
    s.reset_outputs()
    for b in (s.arg, s.stage):
        b.fill_u32(NAN)
    ch.run()
    assert ch.status() == 0
    got = s.read()
    s.check_against_oracle(got, f"token chain M={M} after a forced give-up")
    want = np.asarray(O.argmaxM(got["mx"], s.NT, M), np.uint32).ravel()
    assert np.array_equal(s.stage.read(np.uint32)[:2 * M], want), "the result copy"
    ch.free()
    s.free_token()


@pytest.mark.parametrize("wide", [1, 0])
def test_row_group_passes_end_in_argmaxM(dev, wide):
    """M = 8 verify rows in one pass of the wide kernel, and (knob 12 off) as row-group passes (rows that share no
    memory: argmaxM over the head's tile maxima is a row op and moves with each group's rows); against the oracle's
    argmax of the maxima the chain wrote"""
    M = 8
    s = MiniStep(M=M, gemvM=True)
    NT = s.V // 64
    arg = capi.Buffer(8 * M)

    def token():
        s._enqueue()
        capi.argmaxM(s.dev["mx"], NT, M, arg)

    old = capi.chain_tune(12, wide)
    try:
        ch = capi.chain(token)
    finally:
        capi.chain_tune(12, old)
    assert ch.info()["passes"] == (1 if wide else 2), ch.info()
    s.reset_outputs()
    arg.fill_u32(NAN)
    ch.run()
    assert ch.status() == 0
    got = s.read()
    s.check_against_oracle(got, "row-group chain M=8")
    want = np.asarray(O.argmaxM(got["mx"], NT, M), np.uint32).ravel()
    assert np.array_equal(arg.read(np.uint32), want)
    ch.free()
    arg.free()


def test_layer_chain_rowstats_feeds_rms_gemv(dev):
    """the model's own order inside a layer: rowstats of the residual -> an rms GEMV whose rstd slot that rowstats
    wrote -> normadd of the GEMV's split partials into the residual -> rowstats again -> the next rms GEMV; the GEMVs
    against the oracle on the residual and slots the chain wrote, the aux ops bit-exact"""
    D, N, K = 2048, 2048, 2048
    x0 = (0.5 + O.randn(D, 95)).astype(np.float32)
    w1 = O.pack_q4(O.randn(N * K, 96, 0.03), N, K)[0]
    w2 = O.pack_q4(O.randn(N * K, 97, 0.03), N, K)[0]
    nw = (0.8 + 0.4 * O.rng_uniform(98, D)).astype(np.float32)
    d = {k: capi.to_device(v) for k, v in dict(x=x0, w1=w1, w2=w2, nw=nw).items()}
    st = capi.Buffer(64)
    rst = capi.Buffer(64)
    y1 = capi.Buffer(2 * N * 4)
    y2 = capi.Buffer(N * 4)

    def token():
        capi.rowstats(capi.rowstats_args(x=d["x"], rows=1, cols=D, mode=1, eps=1e-6, st=st, st_off=0))
        capi.q4_gemv(capi.gemv_args(w=d["w1"], w_rows=N, w_cols=K, x=d["x"], N=N, K=K, kPer=1024, pro=capi.PRO["rms"],
                                    y=y1, stat=st, stat_off=1, norm=d["nw"]))
        capi.normadd(capi.normadd_args(t=y1, t_n=2, t_ld=N, w=d["nw"], x=d["x"], st=rst, st_off=0, D=D, M=1,
                                       eps=1e-6, scale=1.0, mode=0))
        capi.q4_gemv(capi.gemv_args(w=d["w2"], w_rows=N, w_cols=K, x=d["x"], N=N, K=K, pro=capi.PRO["rms"], y=y2,
                                    stat=rst, stat_off=0, norm=d["nw"]))

    ch = capi.chain(token)
    for run in range(2):
        d["x"].upload(x0)
        for b in (st, rst, y1, y2):
            b.fill_u32(NAN)
        ch.run()
        assert ch.status() == 0
        g_st, g_y1, g_x, g_rst, g_y2 = (b.read(np.float32) for b in (st, y1, d["x"], rst, y2))
        want_st = np.full(2, np.nan, np.float32)
        O.rowstats(capi.rowstats_args(x=x0.ctypes.data, rows=1, cols=D, mode=1, eps=1e-6, st=want_st.ctypes.data,
                                      st_off=0))
        assert np.array_equal(_bits(g_st[:2]), _bits(want_st))
        y1o = np.zeros(2 * N, np.float32)
        O.q4_gemv(capi.gemv_args(w=w1.ctypes.data, w_rows=N, w_cols=K, x=x0.ctypes.data, N=N, K=K, kPer=1024,
                                 pro=capi.PRO["rms"], y=y1o.ctypes.data, stat=g_st.ctypes.data, stat_off=1,
                                 norm=nw.ctypes.data))
        r1 = rel_l2(g_y1, y1o)
        assert r1 <= 2e-5, r1
        xw, sw = x0.copy(), np.full(1, np.nan, np.float32)
        O.normadd(capi.normadd_args(t=g_y1.ctypes.data, t_n=2, t_ld=N, w=nw.ctypes.data, x=xw.ctypes.data,
                                    st=sw.ctypes.data, st_off=0, D=D, M=1, eps=1e-6, scale=1.0, mode=0))
        assert np.array_equal(_bits(g_x), _bits(xw)) and np.array_equal(_bits(g_rst[:1]), _bits(sw))
        y2o = np.zeros(N, np.float32)
        O.q4_gemv(capi.gemv_args(w=w2.ctypes.data, w_rows=N, w_cols=K, x=g_x.ctypes.data, N=N, K=K,
                                 pro=capi.PRO["rms"], y=y2o.ctypes.data, stat=g_rst.ctypes.data, stat_off=0,
                                 norm=nw.ctypes.data))
        r2 = rel_l2(g_y2, y2o)
        assert r2 <= 2e-5, r2
        print(f"layer chain run {run}: gemv rel_l2 {r1:.2e} {r2:.2e}, rowstats / normadd bit-exact", flush=True)
    ch.free()
    for b in list(d.values()) + [st, rst, y1, y2]:
        b.free()


def test_chain_with_copy_is_refused_where_only_the_general_kernel_runs(dev):
    """aux ops run only on the pipelined kernel: with the pipelined kernel switched off (knob 4) a chain holding one
    is refused at p0_chain_end, with the reason"""
    s = MiniStep(M=1)
    old = capi.chain_tune(4, 0)
    try:
        capi.check(capi.lib().p0_chain_begin())
        f = s.ops(s.dev | s.out)[0]
        capi.q4_gemv(s._args(f))
        capi.copy(s.out["qkv"], 0, s.out["o"], 0, 64)
        h = capi.vp()
        assert capi.lib().p0_chain_end(capi.C.byref(h)) == capi.P0_EINVAL
        assert "join only pipelined chains" in capi.last_error()
    finally:
        capi.chain_tune(4, old)
