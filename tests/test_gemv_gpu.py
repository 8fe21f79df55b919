"""GPU parity of the q4 GEMV / GEMV-M (p0_q4_gemv / p0_q4_gemvM) against the CPU oracle, through the C ABI.

Outputs are NaN-filled before each call (a kernel that skipped a row cannot pass, engine/tune/autotune.js:1-7).
Tolerance: relative L2 <= 1e-3 against the oracle's float64 sum, plus this build's own fp32 bar
of 2e-5 (the kernel computes in fp32 with fp32 activations, so anything looser means a lost term).
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3          # 1e-3 relative L2
TOL_FP32 = 2e-5     # this build's fp32 path
NAN = 0x7FC00000


def _check(got, want, what):
    r = rel_l2(got, want)
    print(f"{what}: rel_l2 {r:.3e}", flush=True)
    assert np.all(np.isfinite(got)), what + ": non-finite output (a row was not written)"
    assert r <= TOL, what
    assert r <= TOL_FP32, what


class Case:
    """One gemv / gemvM call on identical seeded inputs, run on the GPU and on the oracle."""

    def __init__(self, M, N, K, pro="raw", epi="store", kPer=0, seed=1, w_off=0, rowB=0, ldx=0, ldy=0, ldm=0,
                 gemvM=False, nsrc=2, weights=None):
        self.M, self.N, self.K, self.pro, self.epi = M, N, K, pro, epi
        rows = 2 * N if epi == "geglu" else N
        if weights is None:
            weights = O.pack_q4(O.randn(rows * K, seed, 0.05), rows, K)[0]
        self.w = np.zeros(w_off + weights.nbytes, np.uint8)
        self.w[w_off:] = weights
        ldx = ldx or K
        self.x = O.randn(max(rowB + M * ldx, nsrc * M * ldx) + 64, seed + 1)
        self.nw = (0.9 + 0.2 * ((np.arange(K) * 7919) % 100) / 100).astype(np.float32)
        self.ev = O.randn(M * K + 64, seed + 2, 0.5)
        NT = N // 64
        self.stat = np.zeros(NT * 2 * M + 2 * M + 8, np.float32)
        st_off = NT * 2 * M
        for m in range(M):
            xr = self.x[rowB + m * ldx: rowB + m * ldx + K].astype(np.float64)
            self.stat[st_off + 2 * m + 1] = np.float32(1 / np.sqrt((xr ** 2).mean() + 1e-6))
        if gemvM:
            kp = min(2048, kPer) if kPer else K
        else:
            kch = ((K + 255) // 256) * 256 if (not kPer and K > 2048) else 2048
            kp = min(kch, kPer or K)
        self.nsplit = -(-K // kp)
        ldm = ldm or N
        ldy = ldy or (M * ldm if gemvM else N)
        self.ylen = (self.nsplit * ldy if epi == "store" else M * ldm) + 64
        self.fields = dict(w_off=w_off, w_rows=rows, w_cols=K, N=N, K=K, kPer=kPer, pro=capi.PRO[pro],
                           epi=capi.EPI[epi], norm_off=0, src_n=nsrc, src_ld=M * ldx if gemvM else ldx, ev_off=0,
                           cap=30.0)
        if gemvM:
            self.fields.update(M=M, x_ldx=ldx, x_rowB=rowB, y_ldy=ldy, y_ldm=ldm, stat_off=st_off + 1, stat_ld=2,
                               ev_ld=K)
        else:
            self.fields.update(x_rowB=rowB, ldy=ldy, stat_off=st_off + 1)
        self.gemvM = gemvM

    def _args(self, w, x, y, stat, norm, ev, mx):
        f = dict(self.fields, w=w, x=x, y=y, norm=norm, ev=ev, mx=mx)
        f["stat"] = mx if (self.epi == "softcap" and not self.gemvM) else stat
        return (capi.gemvm_args if self.gemvM else capi.gemv_args)(**f)

    def run_oracle(self):
        y = np.full(self.ylen, np.nan, np.float32)
        mx = self.stat.copy()
        a = self._args(self.w.ctypes.data, self.x.ctypes.data, y.ctypes.data, self.stat.ctypes.data,
                       self.nw.ctypes.data, self.ev.ctypes.data, mx.ctypes.data)
        ns = (O.q4_gemvM if self.gemvM else O.q4_gemv)(a)
        assert ns == self.nsplit
        return y, mx

    def run_gpu(self):
        bufs = [capi.to_device(v) for v in (self.w, self.x, self.stat, self.nw, self.ev, self.stat)]
        yb = capi.Buffer(self.ylen * 4).fill_u32(NAN)
        wb, xb, sb, nb, eb, mb = bufs
        a = self._args(wb, xb, yb, sb, nb, eb, mb)
        ns = (capi.q4_gemvM if self.gemvM else capi.q4_gemv)(a)
        assert ns == self.nsplit
        y, mx = yb.read(np.float32), mb.read(np.float32)
        for b in bufs + [yb]:
            b.free()
        return y, mx

    def rows_written(self):
        """indices of Y this call writes"""
        ldy = self.fields.get("ldy", self.fields.get("y_ldy"))
        ldm = self.fields.get("y_ldm", 0)
        idx = []
        for s in range(self.nsplit if self.epi == "store" else 1):
            for m in range(self.M):
                base = (s * ldy if self.epi == "store" else 0) + m * ldm
                idx.append(np.arange(base, base + self.N))
        return np.concatenate(idx)

    def check(self, what):
        yo, mxo = self.run_oracle()
        yg, mxg = self.run_gpu()
        idx = self.rows_written()
        _check(yg[idx], yo[idx], what)
        untouched = np.setdiff1d(np.arange(self.ylen), idx)
        assert np.all(np.isnan(yg[untouched])), what + ": wrote outside its rows"
        if self.epi == "softcap":
            NT = self.N // 64
            for m in range(self.M):
                o = (m * NT) * 2
                gv, ov = mxg[o:o + 2 * NT:2], mxo[o:o + 2 * NT:2]
                gi = mxg[o + 1:o + 2 * NT:2].view(np.uint32)
                oi = mxo[o + 1:o + 2 * NT:2].view(np.uint32)
                assert np.allclose(gv, ov, rtol=1e-5, atol=1e-5), what + ": tile max"
                yrow = yo[m * self.fields.get("y_ldm", 0): m * self.fields.get("y_ldm", 0) + self.N]
                bad = (gi != oi) & (np.abs(yrow[gi.astype(np.int64)] - yrow[oi.astype(np.int64)]) > 1e-5)
                assert not bad.any(), what + ": tile argmax"   # the kshipped.js:41 rule
        return yg


# ------------------------------------------------------------------------------------------------ gemv (M = 1)
@pytest.mark.parametrize("pro", ["raw", "rms", "sum", "pleg"])
@pytest.mark.parametrize("epi", ["store", "geglu", "softcap"])
def test_gemv_prologue_epilogue(dev, pro, epi):
    Case(1, 256, 512, pro, epi, seed=3).check(f"gemv {pro}.{epi} 256x512")


@pytest.mark.parametrize("N,K,kPer", [
    (2048, 8192, 2048),      # E2B down projection: 4 partials (gemma4.js:485)
    (2048, 2048, 2048),      # o projection with kPer 2048: one split
    (64, 2048 + 96, 1024),   # ragged last split
    (192, 2560, 0),          # K in (2048, 3072] without a kPer: one split of the whole K (lops.js:116-117)
    (64, 32, 0),             # one record
    (320, 96, 0),            # tile count not a multiple of the workgroup's 4
])
def test_gemv_splits_and_shapes(dev, N, K, kPer):
    Case(1, N, K, "raw", "store", kPer=kPer, seed=5).check(f"gemv raw.store {N}x{K} kPer {kPer}")


def test_gemv_offsets_and_strides(dev):
    # 4-byte (not 16-byte) aligned weight offset, an x row offset, and an output stride wider than N
    Case(1, 256, 1024, "rms", "store", kPer=512, w_off=4, rowB=7, ldy=256 + 64, seed=9).check("gemv offsets")


def test_gemv_config_a_full_size(dev):
    """BASELINE config A: M=1, K=2048, N=8192, symmetric 4-bit weights, fp16 activations N(0,1), seed 0"""
    N, K = 8192, 2048
    w = O.fill_q4_sym(N, K, 0, 0.02)
    c = Case(1, N, K, "raw", "store", weights=w)
    c.x[:] = O.fill_randn(c.x.size, 0)[0]
    c.check("config A 8192x2048")


def test_gemv_deterministic(dev):
    c = Case(1, 2048, 8192, "raw", "store", kPer=2048, seed=13)
    a, b = c.run_gpu()[0], c.run_gpu()[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_gemv_decompositions_agree(dev):
    """the split-K decomposition is a tuning choice: every choice gives the oracle's result"""
    c = Case(1, 1024, 4096, "raw", "store", kPer=2048, seed=17)
    want = c.run_oracle()[0]
    idx = c.rows_written()
    old = [capi.gemv_tune(k) for k in range(4)]
    try:
        for knobs in [(1, 100000, 1, 1), (64, 8, 1, 8), (100000, 1, 1, 2), (512, 100000, 4, 4), (8192, 2, 2, 8),
                      (4096, 100000, 1, 3)]:
            for k, v in enumerate(knobs):
                capi.gemv_tune(k, v)
            _check(c.run_gpu()[0][idx], want[idx], f"decomposition knobs {knobs}")
    finally:
        for k, v in enumerate(old):
            capi.gemv_tune(k, v)


def test_gemv_split_k_workspace_across_reopen(dev):
    """K in many slices per workgroup (the uncached split-K workspace and its arrival counters), run after run, then
    after closing and reopening the device (the workspace is kept, not freed): the same bits, the oracle's values"""
    c = Case(1, 512, 4096, "rms", "store", kPer=2048, seed=23)
    want = c.run_oracle()[0]
    idx = c.rows_written()
    old = [capi.gemv_tune(k) for k in range(4)]
    try:
        for k, v in enumerate((100000, 100000, 1, 2)):   # 2 waves per slot, 1 group per wave: 32 slices per split
            capi.gemv_tune(k, v)
        runs = [c.run_gpu()[0] for _ in range(3)]
        capi.close_device()
        capi.open_device(0)
        runs.append(c.run_gpu()[0])
    finally:
        for k, v in enumerate(old):
            capi.gemv_tune(k, v)
    for r in runs:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    _check(runs[-1][idx], want[idx], "split-K after reopen")


@pytest.mark.parametrize("M,epi,K,kPer", [(3, "store", 4096, 2048), (5, "geglu", 2048, 0), (16, "store", 4096, 2048),
                                          (4, "store", 3168, 1024), (1, "store", 3168, 1024)])
def test_gemvM_many_k_slices(dev, M, epi, K, kPer):
    """gemvM (matrix cores) with K in many slices: the last workgroup to arrive loads the slices' partials of every x
    row in batches (fewer slices per batch as M grows) and adds them in slice order; the oracle's values. K = 3168 in
    splits of 1024 leaves a last split of 3 groups, whose later slices hold no group (they store zeros and still count
    their arrival); at M = 1 the same through gemv"""
    c = Case(M, 256, K, "rms", epi, kPer=kPer, seed=29 + M, gemvM=M > 1)
    old = [capi.gemv_tune(k) for k in range(4)]
    try:
        for k, v in enumerate((100000, 100000, 1, 2)):
            capi.gemv_tune(k, v)
        c.check(f"gemvM M={M} {epi}, many K slices")
    finally:
        for k, v in enumerate(old):
            capi.gemv_tune(k, v)


def test_gemv_head_shape_softcap(dev):
    """a head-like softcap GEMV: 65,536 rows x 2,048, per-tile max / argmax (engine/llm/gemma4.js:503-511)"""
    Case(1, 65536, 2048, "rms", "softcap", seed=21).check("head-like softcap 65536x2048")


def test_gemv_softcap_ties_take_the_lower_row(dev):
    # identical rows inside a tile: equal logits, the argmax must be the lowest row (engine/llm/lops.js:99)
    N, K = 128, 64
    W = O.randn(N * K, 3, 0.05).reshape(N, K)
    W[5] = W[40] = W[63] = W[0] * 0 + 0.5
    W[64 + 7] = W[64 + 9] = 0.5
    w = O.pack_q4(W, N, K)[0]
    c = Case(1, N, K, "raw", "softcap", weights=w)
    c.x[:K] = np.abs(c.x[:K])
    yg = c.check("softcap ties")
    mx = c.run_gpu()[1]
    assert mx[1:2].view(np.uint32)[0] == 5 and mx[3:4].view(np.uint32)[0] == 64 + 7


# ------------------------------------------------------------------------------------------------ gemvM
@pytest.fixture(params=["valu", "mfma"])
def mf(request):
    """p0_gemv_tune knob 4: every M on the fp32 VALU kernel (17), or M >= 2 on the matrix-core kernel (2, the
    default)"""
    old = capi.gemv_tune(4, 2 if request.param == "mfma" else 17)
    yield request.param
    capi.gemv_tune(4, old)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16])
def test_gemvM_rms_store(dev, mf, M):
    Case(M, 256, 1024, "rms", "store", seed=30 + M, gemvM=True).check(f"gemvM M={M} rms.store ({mf})")


@pytest.mark.parametrize("pro,epi", [("raw", "geglu"), ("rms", "softcap"), ("pleg", "store"), ("raw", "store")])
def test_gemvM_verify_shapes(dev, mf, pro, epi):
    Case(5, 192, 512, pro, epi, seed=41, gemvM=True).check(f"gemvM M=5 {pro}.{epi} ({mf})")


@pytest.mark.parametrize("M", [9, 16])
@pytest.mark.parametrize("pro,epi", [("raw", "geglu"), ("rms", "softcap")])
def test_gemvM_large_M_epilogues(dev, M, pro, epi):
    Case(M, 192, 512, pro, epi, seed=45 + M, gemvM=True).check(f"gemvM M={M} {pro}.{epi}")


def test_gemvM_splits_and_strides(dev, mf):
    Case(5, 128, 8192, "raw", "store", kPer=2048, ldx=8192 + 32, ldm=128 + 64, seed=43, gemvM=True).check(
        f"gemvM splits ({mf})")


def test_gemvM_mf_knob(dev):
    old = capi.gemv_tune(4, 0)
    assert old == 2, "default: the matrix-core GEMV-M for every M > 1"
    assert capi.gemv_tune(4, 3) == 2 and capi.gemv_tune(4, old) == 3


def test_gemvM_row_equals_gemv(dev):
    """a gemvM row is gemv on that row (engine/llm/lops_spec.js:6-8)"""
    M, N, K = 5, 256, 2048
    w = O.pack_q4(O.randn(N * K, 51, 0.05), N, K)[0]
    cm = Case(M, N, K, "raw", "store", weights=w, gemvM=True, seed=52)
    ym = cm.run_gpu()[0]
    for m in (0, 3):
        c1 = Case(1, N, K, "raw", "store", weights=w, seed=52)
        c1.x[:K] = cm.x[m * K:(m + 1) * K]
        y1 = c1.run_gpu()[0][:N]
        assert rel_l2(ym[m * N:(m + 1) * N], y1) < 1e-6


def test_gemvM_two_tiles_per_wave(dev, mf):
    """1024 output tiles and more: each wave streams two tiles (the head's mode), here with the softcap epilogue"""
    Case(3, 65536, 256, "rms", "softcap", seed=61, gemvM=True).check(f"gemvM M=3 two tiles per wave ({mf})")


@pytest.mark.parametrize("M", [2, 5, 16])
def test_gemvM_large_activations_keep_fp32(dev, mf, M):
    """M >= 2 runs on MFMA with 2^8 x' split into fp16 hi + lo; a workgroup whose x' reaches 255 (fp16 would
    overflow) takes the fp32 path instead. Large values sit in one K-slice only, so both paths run in one call, and the
    split partials still meet the fp32 bar."""
    c = Case(M, 128, 8192, "raw", "store", kPer=2048, seed=62 + M, gemvM=True)
    for m in range(M):
        c.x[m * 8192 + 4096: m * 8192 + 4096 + 7] = np.float32([400.0, -900.0, 330.0, 1.0e5, -3.5e3, 600.0, 2.0e4])
    c.check(f"gemvM M={M} large activations ({mf})")
