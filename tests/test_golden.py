"""The reference's own kernel checks, restated with committed fixtures (tests/golden/, written by make_golden.py: a numpy
restatement that shares no code with the C oracle).

CPU: the oracle reproduces every fixture (rng/randn and the packer bit-exact, dequant by digest, GEMV/GEMM values to
float64 rounding). GPU: the HIP kernels against the fixtures, under the reference's own acceptance (cosine > 0.9995
for the kcheck GEMM, > 0.9999 for the kcheck GEMV, > 0.99999 plus the tile argmax for every kshipped shape) AND this
build's bar (relative L2 <= 1e-3, the BASELINE north star, and the fp32 bar of 2e-5; 1e-5 for a GEMM with fp32 out).
"""
import hashlib
import math
import os

import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import cos_sim, rel_l2

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KSHIPPED = [("rms", "softcap", 1536), ("rms", "geglu", 1536), ("pleg", "store", 256)]


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, "<f4").tobytes()).hexdigest()


def nw_of(K):
    return np.array([0.9 + 0.2 * ((i * 7919) % 100) / 100 for i in range(K)], np.float32)


# ------------------------------------------------------------------------------------------------ the oracle (CPU)
def test_oracle_reproduces_kcheck_gemm_fixture():
    d = load("kcheck_gemm.npz")
    M, N, K = (int(v) for v in d["shape"])
    x = O.randn(M * K, 7)
    x16 = x.astype(np.float16)                                     # rf16: engine/kcheck.js:12
    assert np.array_equal(x16.view(np.uint16), d["x16"])
    w, deq = O.pack_q4(O.randn(N * K, 11, 0.05), N, K)
    assert np.array_equal(w, d["w"])
    assert np.array_equal(deq.reshape(-1).view(np.uint32), d["deq"].reshape(-1).view(np.uint32))
    y = np.zeros(M * N, np.float32)
    O.q4_gemm(capi.gemm_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=x16.ctypes.data, M=M, N=N, K=K,
                             epi=capi.GEPI["f32"], y=y.ctypes.data))
    assert rel_l2(y, d["y_tile16"]) < 1e-7                        # float64 sums over fp16 tiles, rounded once
    assert cos_sim(y, d["y"]) > 0.9995                             # kcheck's bar against the fp32 dequant product


def test_oracle_reproduces_kcheck_gemv_fixture():
    d = load("kcheck_gemv.npz")
    N, K = (int(v) for v in d["shape"])
    x = O.randn(K, 31)
    assert np.array_equal(x.view(np.uint32), d["x"].view(np.uint32))
    w, deq = O.pack_q4(O.randn(N * K, 32, 0.05), N, K)
    assert np.array_equal(w, d["w"])
    assert digest(deq) == str(d["deq_sha256"][0])
    y = np.zeros(N, np.float32)
    O.q4_gemv(capi.gemv_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, N=N, K=K, y=y.ctypes.data))
    assert rel_l2(y, d["y"]) < 1e-7


@pytest.mark.parametrize("pro,epi,K", KSHIPPED)
def test_oracle_reproduces_kshipped_fixture(pro, epi, K):
    d = load("kshipped_%s_%s_%d.npz" % (pro, epi, K))
    N = 128
    rows = 2 * N if epi == "geglu" else N
    w, deq = O.pack_q4(O.randn(rows * K, 33 + K, 0.05), rows, K)
    assert np.array_equal(w, d["w"]) and digest(deq) == str(d["deq_sha256"][0])
    x, ev = O.randn(K, 34 + K), O.randn(K, 35 + K, 0.5)
    assert np.array_equal(x, d["x"]) and np.array_equal(ev, d["ev"]) and np.array_equal(nw_of(K), d["nw"])
    ss = float(np.sum(x.astype(np.float64) ** 2))
    assert np.float32(1 / math.sqrt(ss / K + 1e-6)) == d["rstd"][0]
    got, mx = run_kshipped(d, pro, epi, K, host=True)
    assert rel_l2(got, d["y"]) < 1e-6
    if epi == "softcap":
        assert np.array_equal(mx[1:2 * (N // 64):2].view(np.uint32), d["tile_arg"])


# ------------------------------------------------------------------------------------------------ shared runner
def run_kshipped(d, pro, epi, K, host):
    """engine/tune/kshipped.js:17-41: one gemv call as the engine makes it; returns (rows summed over splits, mx)"""
    N = 128
    NT = N // 64
    rows = 2 * N if epi == "geglu" else N
    rstd = d["rstd"][0]
    mx = np.zeros(NT * 2 + 4, np.float32)
    mx[NT * 2] = rstd
    st = np.array([0, rstd, 0, 0], np.float32)
    arrays = dict(w=d["w"], x=d["x"], norm=d["nw"], ev=d["ev"], stat=st, mx=mx)
    y = np.full(N, np.nan, np.float32)
    if host:
        b = {k: v.ctypes.data for k, v in arrays.items()}
        yb = y.ctypes.data
    else:
        b = {k: capi.to_device(v) for k, v in arrays.items()}
        yb = capi.Buffer(N * 4).fill_u32(0x7FC00000)
    f = dict(w=b["w"], w_rows=rows, w_cols=K, x=b["x"], N=N, K=K, pro=capi.PRO[pro], epi=capi.EPI[epi], y=yb)
    if pro == "rms":
        f.update(norm=b["norm"], stat=b["mx"] if epi == "softcap" else b["stat"], stat_off=NT * 2 if epi == "softcap" else 1)
    if pro == "pleg":
        f.update(src_n=1, src_ld=K, ev=b["ev"])
    if epi == "softcap":
        f.update(mx=b["mx"], cap=30.0)
    (O.q4_gemv if host else capi.q4_gemv)(capi.gemv_args(**f))
    if host:
        return y, mx
    got, mxg = yb.read(np.float32), b["mx"].read(np.float32)
    for v in list(b.values()) + [yb]:
        v.free()
    return got, mxg


def _bar(got, want, what, cos_min, tol_build=2e-5):
    c, r = cos_sim(got, want), rel_l2(got, want)
    print("%s: cos %.8f rel_l2 %.3e" % (what, c, r), flush=True)
    assert np.all(np.isfinite(got)), what
    assert c > cos_min, what + ": the reference's own acceptance"
    assert r <= 1e-3 and r <= tol_build, what


# ------------------------------------------------------------------------------------------------ the HIP path (GPU)
@pytest.mark.gpu
def test_gpu_kcheck_gemm(dev):
    d = load("kcheck_gemm.npz")
    M, N, K = (int(v) for v in d["shape"])
    wb, xb = capi.to_device(d["w"]), capi.to_device(d["x16"])
    for epi, dt, tol in (("f32", np.float32, 1e-5), ("f16", np.float16, 2e-3)):
        yb = capi.Buffer(M * N * 4).fill_u32(0x7FC00000)
        capi.q4_gemm(capi.gemm_args(w=wb, w_rows=N, w_cols=K, x=xb, M=M, N=N, K=K, epi=capi.GEPI[epi], y=yb))
        got = yb.read(dt, M * N).astype(np.float64)
        _bar(got, d["y_tile16"], "kcheck gemm %s out" % epi, 0.9995, tol)
        c = cos_sim(got, d["y"])
        assert c > 0.9995 and rel_l2(got, d["y"]) <= 1e-3, "kcheck's own expectation: cos %.6f" % c
        yb.free()
    o32 = capi.Buffer(N * K * 4)
    capi.q4_dequant(wb, N, K, out32=o32)
    assert np.array_equal(o32.read(np.uint32), d["deq"].reshape(-1).view(np.uint32))
    for b in (wb, xb, o32):
        b.free()


@pytest.mark.gpu
def test_gpu_kcheck_gemv(dev):
    d = load("kcheck_gemv.npz")
    N, K = (int(v) for v in d["shape"])
    wb, xb = capi.to_device(d["w"]), capi.to_device(d["x"])
    yb = capi.Buffer(N * 4).fill_u32(0x7FC00000)
    capi.q4_gemv(capi.gemv_args(w=wb, w_rows=N, w_cols=K, x=xb, N=N, K=K, y=yb))
    _bar(yb.read(np.float32), d["y"], "kcheck gemv", 0.9999)
    o32 = capi.Buffer(N * K * 4)
    capi.q4_dequant(wb, N, K, out32=o32)
    assert digest(o32.read(np.float32)) == str(d["deq_sha256"][0])
    for b in (wb, xb, yb, o32):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("pro,epi,K", KSHIPPED)
def test_gpu_kshipped_fixture(dev, pro, epi, K):
    d = load("kshipped_%s_%s_%d.npz" % (pro, epi, K))
    got, mx = run_kshipped(d, pro, epi, K, host=False)
    _bar(got, d["y"], "kshipped %s.%s K %d" % (pro, epi, K), 0.99999)
    if epi == "softcap":
        assert np.array_equal(mx[1:4:2].view(np.uint32), d["tile_arg"])


# every shape of the reference's PICK table (engine/llm/lopsx.js:312), as kshipped runs it: 128 rows at the real K and
# split. Weights from the oracle's packer (pinned above); the expected rows in float64 here, independently of the oracle.
PICK = ["rms.softcap.262144x1536", "rms.geglu.6144x1536", "raw.store.1536x6144", "rms.geglu.12288x1536",
        "raw.store.1536x12288", "raw.store.8960x1536", "rms.store.3072x2560", "raw.store.2560x2048",
        "rms.store.6144x2560", "raw.store.2560x4096", "rms.store.2048x2560", "rms.store.4096x2560",
        "rms.softcap.262144x2560", "rms.geglu.10240x2560", "raw.store.2560x10240", "raw.store.256x2560",
        "raw.store.10752x2560"]


def _gelu(v):
    return v * 0.5 * (1.0 + np.tanh(np.clip(0.7978845608028654 * (v + 0.044715 * v * v * v), -15.0, 15.0)))


@pytest.mark.gpu
@pytest.mark.parametrize("key", PICK)
def test_gpu_kshipped_pick_shapes(dev, key):
    pro, epi, nk = key.split(".")
    K = int(nk.split("x")[1])
    kPer = 2048 if (pro == "raw" and epi == "store" and K >= 2048 and K != 2560) else 0   # kshipped.js:15
    N, NT = 128, 2
    rows = 2 * N if epi == "geglu" else N
    w, deq = O.pack_q4(O.randn(rows * K, 33 + K, 0.05), rows, K)
    x = O.randn(K, 34 + K)
    nw = nw_of(K)
    rstd = np.float32(1 / math.sqrt(float(np.sum(x.astype(np.float64) ** 2)) / K + 1e-6))
    xd = x.astype(np.float64)
    xp = xd if pro == "raw" else xd * float(rstd) * nw.astype(np.float64)
    dots = deq.reshape(rows, K).astype(np.float64) @ xp
    want = _gelu(dots[:N]) * dots[N:] if epi == "geglu" else (
        30 * np.tanh(np.clip(dots / 30, -15, 15)) if epi == "softcap" else dots)
    nsplit = -(-K // kPer) if kPer else 1
    mx = np.zeros(NT * 2 + 4, np.float32)
    mx[NT * 2] = rstd
    st = np.array([0, rstd, 0, 0], np.float32)
    b = {k: capi.to_device(v) for k, v in dict(w=w, x=x, nw=nw, mx=mx, st=st).items()}
    yN = nsplit * N if epi == "store" else N
    yb = capi.Buffer(yN * 4).fill_u32(0x7FC00000)
    f = dict(w=b["w"], w_rows=rows, w_cols=K, x=b["x"], N=N, K=K, kPer=kPer, pro=capi.PRO[pro], epi=capi.EPI[epi], y=yb)
    if pro == "rms":
        f.update(norm=b["nw"], stat=b["mx"] if epi == "softcap" else b["st"], stat_off=NT * 2 if epi == "softcap" else 1)
    if epi == "softcap":
        f.update(mx=b["mx"], cap=30.0)
    assert capi.q4_gemv(capi.gemv_args(**f)) == nsplit
    y = yb.read(np.float32).reshape(-1, N).astype(np.float64).sum(axis=0)      # kshipped.js:32: splits summed in order
    _bar(y, want, "kshipped %s (nsplit %d)" % (key, nsplit), 0.99999)
    if epi == "softcap":                                                       # kshipped.js:36-39
        arg = b["mx"].read(np.uint32)[1:2 * NT:2]
        for t in range(NT):
            best = t * 64 + int(np.argmax(want[t * 64:(t + 1) * 64]))
            assert arg[t] == best or abs(want[arg[t]] - want[best]) <= 1e-5, key
    for v in list(b.values()) + [yb]:
        v.free()
