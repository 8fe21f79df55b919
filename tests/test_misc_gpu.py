"""GPU parity of rowstats, normadd and argmax/argmaxM (p0pc0rn_amd/csrc/misc.hip) through the C ABI: every result is
compared with the oracle (oracle/q4oracle.c, itself pinned in tests/test_misc_oracle.py) on the same inputs. The
kernels sum in the reference's order with no FMA contraction, so rowstats and normadd are bit-exact, and the argmax
(max, index) pairs are exact, ties included."""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi

pytestmark = pytest.mark.gpu
NAN = 0x7FC00000


@pytest.mark.parametrize("rows,cols,mode", [(1, 2048, 1), (7, 700, 0), (300000, 8, 0), (3, 3, 1), (2, 8192, 0)])
def test_rowstats_bit_exact(dev, rows, cols, mode):
    ld, c0 = cols + 5, 3
    x = (2.0 + O.randn(rows * ld, 70 + rows % 97)).astype(np.float32)
    want = np.full((rows + 1) * 2, np.nan, np.float32)
    O.rowstats(capi.rowstats_args(x=x.ctypes.data, x_ld=ld, x_c0=c0, rows=rows, cols=cols, mode=mode, eps=1e-5,
                                  st=want.ctypes.data, st_off=1))
    xb = capi.to_device(x)
    st = capi.Buffer(want.nbytes).fill_u32(NAN)
    capi.rowstats(capi.rowstats_args(x=xb, x_ld=ld, x_c0=c0, rows=rows, cols=cols, mode=mode, eps=1e-5, st=st,
                                     st_off=1))
    got = st.read(np.float32)
    print(f"rowstats rows {rows} cols {cols} mode {mode}: mismatches {int(np.sum(got.view(np.uint32) != want.view(np.uint32)))}",
          flush=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    xb.free(); st.free()


@pytest.mark.parametrize("D,M,nsrc,mode", [(2048, 1, 4, 0), (2048, 5, 1, 0), (3072, 2, 2, 1), (100, 3, 3, 0)])
def test_normadd_bit_exact(dev, D, M, nsrc, mode):
    ldp = M * D + 64
    t = O.randn(nsrc * ldp, D + M, 0.3).astype(np.float32)
    w = (0.5 + O.rng_uniform(D, D)).astype(np.float32)
    x0 = O.randn(M * D, D + 1).astype(np.float32)
    xw, sw = x0.copy(), np.full(M + 2, np.nan, np.float32)
    kw = dict(t_n=nsrc, t_ld=ldp, w_off=0, st_off=2, D=D, M=M, eps=1e-6, scale=0.9, mode=mode)
    O.normadd(capi.normadd_args(t=t.ctypes.data, w=w.ctypes.data, x=xw.ctypes.data, st=sw.ctypes.data, **kw))
    tb, wb, xb = capi.to_device(t), capi.to_device(w), capi.to_device(x0)
    sb = capi.Buffer(sw.nbytes).fill_u32(NAN)
    capi.normadd(capi.normadd_args(t=tb, w=wb, x=xb, st=sb, **kw))
    gx, gs = xb.read(np.float32), sb.read(np.float32)
    assert np.array_equal(gx.view(np.uint32), xw.view(np.uint32))
    assert np.array_equal(gs.view(np.uint32), sw.view(np.uint32))
    for b in (tb, wb, xb, sb):
        b.free()


@pytest.mark.parametrize("n,M", [(4096, 1), (4096, 5), (1, 1), (257, 3), (0, 1)])
def test_argmax_exact(dev, n, M):
    rng = np.random.default_rng(n + M)
    mx = np.zeros(2 * max(n, 1) * M, np.float32)
    vals = rng.integers(-50, 50, n * M).astype(np.float32)   # ties everywhere
    mx[0:2 * n * M:2] = vals
    mx[1:2 * n * M:2] = rng.integers(0, 1 << 24, n * M).astype(np.uint32).view(np.float32)
    want = O.argmaxM(mx, n, M)
    mb = capi.to_device(mx)
    out = capi.Buffer(8 * M).fill_u32(0)
    if M == 1:
        capi.argmax(mb, n, out)
    else:
        capi.argmaxM(mb, n, M, out)
    got = out.read(np.uint32)
    assert np.array_equal(got, want)
    mb.free(); out.free()


def test_argmax_of_a_softcap_gemv(dev):
    """the pipeline the reference runs at the end of a decode step: head GEMV (rms + softcap, per-tile max/argmax),
    then argmax over the tiles = the argmax of the softcapped logits (ties to the lower row)"""
    N, K = 8192, 512
    w, _ = O.pack_q4(O.randn(N * K, 81, 0.05), N, K)
    x = O.randn(K, 82)
    nw = np.ones(K, np.float32)
    NT = N // 64
    mx = np.zeros(2 * NT + 4, np.float32)
    mx[2 * NT + 1] = 1.0   # rstd slot
    wb, xb, nb, mb = (capi.to_device(a) for a in (w, x, nw, mx))
    y = capi.Buffer(N * 4)
    capi.q4_gemv(capi.gemv_args(w=wb, w_rows=N, w_cols=K, x=xb, N=N, K=K, pro=capi.PRO["rms"], epi=capi.EPI["softcap"],
                                y=y, stat=mb, stat_off=2 * NT + 1, norm=nb, mx=mb, cap=30.0))
    out = capi.Buffer(8).fill_u32(0)
    capi.argmax(mb, NT, out)
    logits = y.read(np.float32)
    got = out.read(np.uint32)
    assert got[0] == int(np.argmax(logits)) and got[1] == logits.max().view(np.uint32)
    for b in (wb, xb, nb, mb, y, out):
        b.free()
