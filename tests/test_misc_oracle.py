"""CPU pins of the oracle's rowstats, normadd and argmax (oracle/q4oracle.c), the GEMV's producer and consumers:
  * closed forms in float64 (the statistics they define), on data whose mean is far from zero, so that a LayerNorm
    that forgets to centre, or an rms that subtracts a mean, fails;
  * an independent numpy restatement of the reference's fp32 order (256 strided lane sums, then the halving tree,
    engine/ops/misc.js:20-27, engine/llm/lops.js:155-166): the oracle must equal it bit for bit;
  * argmax by brute force, including ties (the lower index wins, engine/llm/lops.js:424), and n = 0 (the reference's
    initial values, -3.4e38 and 0xFFFFFFFF).
The C-ABI error texts for these entry points are checked without a device."""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi


def lane_tree(vals):
    """fp32: lane t sums vals[t::256] in order, then red[t] += red[t + s] for s = 128 .. 1"""
    v = np.asarray(vals, np.float32)
    red = np.zeros(256, np.float32)
    for t in range(256):
        s = np.float32(0)
        for e in v[t::256]:
            s = np.float32(s + e)
        red[t] = s
    s = 128
    while s:
        red[:s] = (red[:s] + red[s:2 * s]).astype(np.float32)
        s //= 2
    return np.float32(red[0])


def rsqrt32(v):
    return np.float32(np.float32(1.0) / np.sqrt(np.float32(v)))


@pytest.mark.parametrize("mode", [0, 1])
def test_rowstats_closed_form_and_order(mode):
    rows, cols, ld, c0 = 5, 700, 720, 11
    x = (3.0 + O.randn(rows * ld, 41 + mode)).astype(np.float32)
    st = np.full((rows + 2) * 2, np.nan, np.float32)
    O.rowstats(capi.rowstats_args(x=x.ctypes.data, x_off=0, x_ld=ld, x_c0=c0, rows=rows, cols=cols, mode=mode,
                                  eps=1e-5, st=st.ctypes.data, st_off=2))
    for r in range(rows):
        xr = x[r * ld + c0: r * ld + c0 + cols].astype(np.float64)
        mean = xr.mean() if mode == 0 else 0.0
        var = ((xr - mean) ** 2).mean()
        got_mean, got_rstd = st[(2 + r) * 2], st[(2 + r) * 2 + 1]
        assert abs(got_mean - mean) <= 1e-5 * max(1.0, abs(mean))
        assert abs(got_rstd - 1.0 / np.sqrt(var + 1e-5)) <= 1e-5 / np.sqrt(var + 1e-5)
        # the reference's own fp32 order, restated independently
        m32 = np.float32(lane_tree(x[r * ld + c0: r * ld + c0 + cols]) / np.float32(cols)) if mode == 0 else np.float32(0)
        d = (x[r * ld + c0: r * ld + c0 + cols] - m32).astype(np.float32)
        q = np.float32(lane_tree((d * d).astype(np.float32)) / np.float32(cols))
        assert got_mean == m32 and got_rstd == rsqrt32(np.float32(q + np.float32(1e-5)))
    assert np.isnan(st[:4]).all()   # rows before st_off untouched
    if mode == 0:   # a LayerNorm of data with mean 3 is far from the rms statistics
        assert abs(st[5] - 1.0 / np.sqrt((x[c0:c0 + cols].astype(np.float64) ** 2).mean())) > 0.5


@pytest.mark.parametrize("mode", [0, 1])
def test_normadd_closed_form_and_order(mode):
    D, M, nsrc = 300, 2, 3
    t = O.randn(nsrc * (M * D + 7), 51).astype(np.float32)
    w = (0.5 + O.rng_uniform(52, D + 4)).astype(np.float32)
    x0 = (1.0 + O.randn(M * D, 53)).astype(np.float32)
    x = x0.copy()
    st = np.full(M + 3, np.nan, np.float32)
    O.normadd(capi.normadd_args(t=t.ctypes.data, t_n=nsrc, t_ld=M * D + 7, w=w.ctypes.data, w_off=4, x=x.ctypes.data,
                                st=st.ctypes.data, st_off=1, D=D, M=M, eps=1e-6, scale=0.75, mode=mode))
    for m in range(M):
        tv = sum(t[j * (M * D + 7) + m * D: j * (M * D + 7) + (m + 1) * D].astype(np.float64) for j in range(nsrc))
        rs = 1.0 / np.sqrt((tv ** 2).mean() + 1e-6)
        want = (x0[m * D:(m + 1) * D] + tv * rs * w[4:4 + D]) * 0.75 if mode == 0 else tv
        got = x[m * D:(m + 1) * D]
        assert np.max(np.abs(got - want)) <= 2e-5 * np.max(np.abs(want))
        assert abs(st[1 + m] - 1.0 / np.sqrt((want ** 2).mean() + 1e-6)) <= 1e-5 * st[1 + m]
        # fp32 order: the j sums in order per element, lane sums of squares, tree
        tv32 = np.zeros(D, np.float32)
        for j in range(nsrc):
            tv32 = (tv32 + t[j * (M * D + 7) + m * D: j * (M * D + 7) + (m + 1) * D]).astype(np.float32)
        rs32 = rsqrt32(np.float32(lane_tree((tv32 * tv32).astype(np.float32)) / np.float32(D)) + np.float32(1e-6))
        if mode == 0:
            x32 = (((x0[m * D:(m + 1) * D] + ((tv32 * rs32).astype(np.float32) * w[4:4 + D]).astype(np.float32))
                    .astype(np.float32)) * np.float32(0.75)).astype(np.float32)
        else:
            x32 = tv32
        assert np.array_equal(got.view(np.uint32), x32.view(np.uint32))
        s32 = rsqrt32(np.float32(lane_tree((x32 * x32).astype(np.float32)) / np.float32(D)) + np.float32(1e-6))
        assert st[1 + m] == s32
    assert np.isnan(st[0]) and np.isnan(st[1 + M:]).all()


def test_normadd_defaults():
    """t.n 0 -> 1, t.ld 0 -> D M, M 0 -> 1, eps 0 -> 1e-6 (engine/llm/lops.js:175-177)"""
    D = 64
    t = O.randn(D, 61).astype(np.float32)
    x, st = np.zeros(D, np.float32), np.zeros(2, np.float32)
    O.normadd(capi.normadd_args(t=t.ctypes.data, x=x.ctypes.data, st=st.ctypes.data, D=D, mode=1))
    assert np.array_equal(x, t)
    assert abs(st[0] - 1.0 / np.sqrt((t.astype(np.float64) ** 2).mean() + 1e-6)) <= 1e-6 * st[0]


def _pairs(vals, idx):
    mx = np.zeros(2 * len(vals), np.float32)
    mx[0::2] = vals
    mx[1::2] = np.asarray(idx, np.uint32).view(np.float32)
    return mx


@pytest.mark.parametrize("n", [1, 255, 256, 257, 4096, 5000])
def test_argmax_brute_force_with_ties(n):
    rng = np.random.default_rng(n)
    vals = rng.integers(-20, 20, n).astype(np.float32)   # many equal values: ties are common
    idx = rng.permutation(n * 64)[:n].astype(np.uint32)   # tile argmax rows: any order, unique
    got = O.argmaxM(_pairs(vals, idx), n, 1)
    best = vals.max()
    want_idx = idx[vals == best].min()
    assert got[0] == want_idx and got[1] == np.float32(best).view(np.uint32)


def test_argmaxM_rows_and_empty():
    n, M = 300, 3
    rng = np.random.default_rng(7)
    vals = rng.standard_normal(M * n).astype(np.float32)
    idx = np.tile(np.arange(n, dtype=np.uint32) * 64, M)
    got = O.argmaxM(_pairs(vals, idx), n, M).reshape(M, 2)
    for m in range(M):
        k = int(np.argmax(vals[m * n:(m + 1) * n]))
        assert got[m, 0] == idx[m * n + k] and got[m, 1] == vals[m * n + k].view(np.uint32)
    empty = O.argmaxM(np.zeros(2, np.float32), 0, 1)
    assert empty[0] == 0xFFFFFFFF and empty[1] == np.float32(-3.4e38).view(np.uint32)


def test_misc_errors_without_device():
    with pytest.raises(capi.P0Error, match="rowstats: mode 3"):
        capi.rowstats(capi.rowstats_args(x=8, st=8, rows=1, cols=4, mode=3))
    with pytest.raises(capi.P0Error, match="rowstats: missing x or st buffer"):
        capi.rowstats(capi.rowstats_args(rows=1, cols=4))
    with pytest.raises(capi.P0Error, match="normadd: missing t, w, x or st buffer"):
        capi.normadd(capi.normadd_args(t=8, x=8, st=8, D=4, mode=0))
    with pytest.raises(capi.P0Error, match="normadd: mode 2"):
        capi.normadd(capi.normadd_args(t=8, x=8, st=8, D=4, mode=2))
    with pytest.raises(capi.P0Error, match="argmax: n -1"):
        capi.argmax(8, -1, 8)
