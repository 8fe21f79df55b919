"""GPU parity of the q8g64s.t64 GEMV (p0pc0rn_amd/csrc/gemv_q8.hip) through the C ABI.

Every q8 shape the reference ships (engine/tune/kshipped.js:14, run as kshipped.js:17-41 runs it: 128 rows at the real
K, its kPer rule, seeds 33 + K / 34 + K / 35 + K) under the reference's own acceptance (cos > 0.99999, the tile argmax)
and this build's bars (relative L2 <= 1e-3 and <= 2e-5), the expected rows in float64 from numpy over the decoded
records (tests/test_q8_oracle.py pins the packer and the decode); gemvM with M rows against the oracle; and a chain that
holds a q8 op is refused."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import cos_sim, rel_l2
from tests.test_q8_oracle import np_decode_q8

pytestmark = pytest.mark.gpu

Q8 = [("rms", "store", 1536, 0), ("raw", "store", 2048, 2048), ("raw", "store", 4096, 2048), ("rms", "geglu", 1536, 0),
      ("raw", "store", 6144, 2048), ("raw", "store", 1536, 0), ("pleg", "store", 256, 0)]


def _gelu(v):
    return v * 0.5 * (1.0 + np.tanh(np.clip(0.7978845608028654 * (v + 0.044715 * v * v * v), -15.0, 15.0)))


def nw_of(K):   # engine/tune/kshipped.js:19
    return np.array([0.9 + 0.2 * ((i * 7919) % 100) / 100 for i in range(K)], np.float32)


@pytest.mark.parametrize("pro,epi,K,kPer", Q8)
def test_q8_kshipped_shapes(dev, pro, epi, K, kPer):
    N, NT = 128, 2
    rows = 2 * N if epi == "geglu" else N
    w, _ = O.pack_q8(O.randn(rows * K, 33 + K, 0.05), rows, K)
    x, ev, nw = O.randn(K, 34 + K), O.randn(K, 35 + K, 0.5), nw_of(K)
    rstd = np.float32(1 / math.sqrt(float(np.sum(x.astype(np.float64) ** 2)) / K + 1e-6))
    xd = x.astype(np.float64)
    xp = xd if pro == "raw" else xd * float(rstd) * nw.astype(np.float64) if pro == "rms" else _gelu(xd) * ev
    dots = np_decode_q8(w, rows, K).astype(np.float64) @ xp
    want = _gelu(dots[:N]) * dots[N:] if epi == "geglu" else dots
    nsplit = -(-K // kPer) if kPer else 1
    st = np.array([0, rstd, 0, 0], np.float32)
    b = {k: capi.to_device(v) for k, v in dict(w=w, x=x, nw=nw, st=st, ev=ev).items()}
    yN = nsplit * N if epi == "store" else N
    yb = capi.Buffer(yN * 4).fill_u32(0x7FC00000)
    f = dict(w=b["w"], w_enc=2, w_rows=rows, w_cols=K, x=b["x"], N=N, K=K, kPer=kPer, pro=capi.PRO[pro],
             epi=capi.EPI[epi], y=yb)
    if pro == "rms":
        f.update(norm=b["nw"], stat=b["st"], stat_off=1)
    if pro == "pleg":
        f.update(src_n=1, src_ld=K, ev=b["ev"])
    assert capi.q4_gemv(capi.gemv_args(**f)) == nsplit
    y = yb.read(np.float32).reshape(-1, N).astype(np.float64).sum(axis=0)   # kshipped.js:32
    c, r = cos_sim(y, want), rel_l2(y, want)
    print(f"q8 {pro}.{epi} K {K} kPer {kPer}: cos {c:.8f} rel_l2 {r:.3e}", flush=True)
    assert np.all(np.isfinite(y)) and c > 0.99999 and r <= 1e-3 and r <= 2e-5
    for v in list(b.values()) + [yb]:
        v.free()


@pytest.mark.parametrize("M,epi", [(5, "store"), (16, "store"), (3, "softcap")])
def test_q8_gemvM_matches_oracle(dev, M, epi):
    N, K = 256, 2048
    w, _ = O.pack_q8(O.randn(N * K, 71, 0.05), N, K)
    x = O.randn(M * K, 72)
    NT = N // 64
    mx_len = M * NT * 2
    want = np.full(M * N, np.nan, np.float32)
    wmx = np.zeros(mx_len, np.float32)
    O.q4_gemvM(capi.gemvm_args(w=w.ctypes.data, w_enc=2, w_rows=N, w_cols=K, x=x.ctypes.data, x_ldx=K, M=M, N=N, K=K,
                               epi=capi.EPI[epi], y=want.ctypes.data, y_ldm=N, mx=wmx.ctypes.data, cap=30.0))
    wb, xb = capi.to_device(w), capi.to_device(x)
    yb = capi.Buffer(M * N * 4).fill_u32(0x7FC00000)
    mb = capi.Buffer(mx_len * 4).fill_u32(0)
    capi.q4_gemvM(capi.gemvm_args(w=wb, w_enc=2, w_rows=N, w_cols=K, x=xb, x_ldx=K, M=M, N=N, K=K, epi=capi.EPI[epi],
                                  y=yb, y_ldm=N, mx=mb, cap=30.0))
    got = yb.read(np.float32)
    r = rel_l2(got, want)
    print(f"q8 gemvM M {M} {epi}: rel_l2 {r:.3e}", flush=True)
    assert np.all(np.isfinite(got)) and r <= 2e-5
    if epi == "softcap":
        gm = mb.read(np.float32)
        assert np.allclose(gm[0::2], wmx[0::2], rtol=1e-5, atol=1e-5)
        assert np.mean(gm[1::2].view(np.uint32) == wmx[1::2].view(np.uint32)) > 0.99
    for v in (wb, xb, yb, mb):
        v.free()


def test_q8_ops_cannot_join_a_chain(dev):
    N, K = 128, 256
    w, _ = O.pack_q8(O.randn(N * K, 5, 0.05), N, K)
    wb, xb, yb = capi.to_device(w), capi.Buffer(K * 4), capi.Buffer(N * 4)
    with pytest.raises(capi.P0Error, match="q8g64s.t64 ops cannot join a chain"):
        capi.chain(lambda: capi.q4_gemv(capi.gemv_args(w=wb, w_enc=2, w_rows=N, w_cols=K, x=xb, N=N, K=K, y=yb)))
    for v in (wb, xb, yb):
        v.free()
