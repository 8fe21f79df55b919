"""GPU parity of the q4 dequant-GEMM (p0_q4_gemm) against the CPU oracle, through the C ABI.

Tolerance: relative L2 <= 1e-3 against the oracle's float64 sum over the same fp16 operands,
plus this build's bar of 1e-5 for fp32 outputs (MFMA accumulates in fp32; the operands are bit-identical fp16) and
2e-3 where the output itself is fp16 (half an fp16 ulp is 2^-11 relative).
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
NAN32, NAN16x2 = 0x7FC00000, 0x7E007E00


def _weights(rows, K, seed):
    return O.pack_q4(O.randn(rows * K, seed, 0.05), rows, K)[0]


def run(fields, arrays, out_dtype, out_len, init=None):
    """run the same call on the oracle (host pointers) and on the GPU (device copies); returns (oracle, gpu)"""
    y_host = np.full(out_len, np.nan, out_dtype) if init is None else init.astype(out_dtype).copy()
    host = {k: v.ctypes.data for k, v in arrays.items()}
    O.q4_gemm(capi.gemm_args(**fields, **host, y=y_host.ctypes.data))
    dev = {k: capi.to_device(v) for k, v in arrays.items()}
    if init is None:
        yb = capi.Buffer(max(y_host.nbytes, 16)).fill_u32(NAN32 if out_dtype == np.float32 else NAN16x2)
    else:
        yb = capi.to_device(init.astype(out_dtype))
    flops = capi.q4_gemm(capi.gemm_args(**fields, **dev, y=yb))
    assert flops == 2.0 * fields["M"] * fields["N"] * fields["K"]
    got = yb.read(out_dtype, out_len)
    for b in list(dev.values()) + [yb]:
        b.free()
    return y_host, got


def check(got, want, what, tol_build):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    r = rel_l2(got, want)
    print(f"{what}: rel_l2 {r:.3e}", flush=True)
    assert np.all(np.isfinite(got)), what + ": unwritten outputs"
    assert r <= TOL and r <= tol_build, what


@pytest.mark.parametrize("M,N,K", [(40, 128, 256), (128, 256, 512), (300, 200, 96), (1, 64, 32), (257, 384, 1024)])
def test_gemm_f16_f32(dev, M, N, K):
    Nw = -(-N // 64) * 64                      # records hold 64 rows; a ragged N reads the first N of them
    w = _weights(Nw, K, 11)
    x = O.randn(M * K, 7).astype(np.float16)
    f = dict(w_rows=Nw, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE["f16"], epi=capi.GEPI["f32"])
    want, got = run(f, dict(w=w, x=x), np.float32, M * N)
    check(got, want, f"gemm f16->f32 {M}x{N}x{K}", 1e-5)


def test_gemm_f16_out(dev):
    M, N, K = 96, 256, 256
    w = _weights(N, K, 12)
    x = O.randn(M * K, 8).astype(np.float16)
    f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE["f16"], epi=capi.GEPI["f16"])
    want, got = run(f, dict(w=w, x=x), np.float16, M * N)
    check(got, want, "gemm f16->f16", 2e-3)


@pytest.mark.parametrize("M,N,y_ld,y_n0", [(96, 251, 260, 4), (70, 131, 131, 0), (33, 128, 139, 3), (33, 128, 128, 1)])
def test_gemm_f16_out_layouts(dev, M, N, y_ld, y_n0):
    """fp16 outputs are stored two columns per 4-byte store when Y's rows allow it (even row stride, even first
    column) and one by one otherwise; ragged N (an odd last column) and offset rows, with every element outside the
    written block left untouched"""
    K = 256
    Nw = -(-N // 64) * 64
    w = _weights(Nw, K, 31)
    x = O.randn(M * K, 32).astype(np.float16)
    f = dict(w_rows=Nw, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE["f16"], epi=capi.GEPI["f16"], y_ld=y_ld, y_n0=y_n0)
    n_out = (M * y_ld + y_n0 + 9) // 2 * 2   # whole 4-byte words: the device buffer is NaN-filled by words
    want, got = run(f, dict(w=w, x=x), np.float16, n_out)
    idx = np.concatenate([y_n0 + m * y_ld + np.arange(N) for m in range(M)])
    check(got[idx], want[idx], f"gemm f16 out M={M} N={N} ld={y_ld} n0={y_n0}", 2e-3)
    untouched = np.setdiff1d(np.arange(n_out), idx)
    assert np.all(np.isnan(got[untouched].astype(np.float32)))


def test_gemm_bf16_activations(dev):
    M, N, K = 64, 128, 512
    w = _weights(N, K, 14)
    xf = O.randn(M * K, 9)
    xb = (xf.view(np.uint32) >> 16).astype(np.uint16)          # bf16 by truncation: exact bf16 values
    f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE["bf16"], epi=capi.GEPI["f32"])
    want, got = run(f, dict(w=w, x=xb), np.float32, M * N)
    check(got, want, "gemm bf16->f32", 1e-5)


@pytest.mark.parametrize("mode", ["lnmod", "rms"])
def test_gemm_fused_norm_prologues(dev, mode):
    """engine/ops/gemm.js:59-63: X f32, (mean, rstd) per row, scale / shift vectors (shift base = off + stride, u32)"""
    M, N, K = 72, 192, 256
    w = _weights(N, K, 15)
    x = O.randn(M * K, 10, 2.0)
    st = np.zeros(2 * (M + 3), np.float32)
    xr = x.reshape(M, K).astype(np.float64)
    st[6::2] = xr.mean(1)
    st[7::2] = 1 / np.sqrt(xr.var(1) + 1e-6)
    pv = O.randn(4 * K, 16, 0.1)
    f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE[mode], epi=capi.GEPI["f32"], stats_off=3,
             pv_off=2 * K, pv_stride=(1 << 32) - 2 * K)           # shift at off - 2K, the reference's neg(stride) wrap
    want, got = run(f, dict(w=w, x=x, stats=st, pv=pv), np.float32, M * N)
    check(got, want, f"gemm {mode}", 1e-5)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_gemm_swiglu_with_bias(dev, act):
    M, MLP, K = 80, 192, 256
    w = _weights(2 * MLP, K, 17)                                 # rows [gate | up]
    x = O.randn(M * K, 18).astype(np.float16)
    bv = O.randn(2 * MLP + 8, 19, 0.1)
    f = dict(w_rows=2 * MLP, w_cols=K, M=M, N=2 * MLP, K=K, x_mode=0, epi=capi.GEPI["swiglu"], wr0=0, wr1=MLP,
             y_ld=MLP, bv_off=4, bv_up=MLP, act=capi.ACT[act])
    want, got = run(f, dict(w=w, x=x, bv=bv), np.float16, M * MLP)
    check(got, want, f"gemm swiglu {act}", 2e-3)


@pytest.mark.parametrize("store", [0, 1])
def test_gemm_resadd_gate_bias(dev, store):
    M, N, K = 64, 256, 512
    w = _weights(N, K, 20)
    x = O.randn(M * K, 21).astype(np.float16)
    gate = O.randn(N, 22)
    bv = O.randn(N, 23, 0.1)
    resid = O.randn(M * N, 24)
    f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=0, epi=capi.GEPI["resadd"], store=store)
    want, got = run(f, dict(w=w, x=x, ev=gate, bv=bv), np.float32, M * N, init=resid)
    check(got, want, f"gemm resadd store={store}", 1e-5)


@pytest.mark.parametrize("epi,N,y_ld,y_n0", [("f32", 131, 140, 2), ("f32", 128, 133, 1), ("resadd", 131, 140, 2),
                                            ("resadd", 128, 133, 3), ("bias", 131, 140, 2), ("bias", 128, 129, 1)])
def test_gemm_output_layouts(dev, epi, N, y_ld, y_n0):
    """the f32, resadd (accumulating) and bias (with residual) epilogues read and write two adjacent columns per
    access when Y's rows allow it and element by element otherwise; ragged N, offset rows, elements outside the block
    keep their values"""
    M, K = 45, 256
    Nw = -(-N // 64) * 64
    w = _weights(Nw, K, 41)
    x = O.randn(M * K, 42).astype(np.float16)
    ev = O.randn(N, 43)
    bv = O.randn(N, 44, 0.1)
    n_out = (M * y_ld + y_n0 + 9) // 2 * 2
    f = dict(w_rows=Nw, w_cols=K, M=M, N=N, K=K, x_mode=0, epi=capi.GEPI[epi], y_ld=y_ld, y_n0=y_n0)
    arrays = dict(w=w, x=x, ev=ev)
    if epi == "resadd":
        f.update(store=0)
        arrays.update(bv=bv)
    if epi == "bias":
        f.update(res=1)
    dt = np.float16 if epi == "bias" else np.float32
    init = O.randn(n_out, 45)
    want, got = run(f, arrays, dt, n_out, init=init)
    idx = np.concatenate([y_n0 + m * y_ld + np.arange(N) for m in range(M)])
    check(got[idx], want[idx], f"gemm {epi} out N={N} ld={y_ld} n0={y_n0}", 2e-3 if dt == np.float16 else 1e-5)
    untouched = np.setdiff1d(np.arange(n_out), idx)
    assert np.array_equal(got[untouched], init.astype(dt)[untouched])


def test_gemm_bias_residual_in_place(dev):
    M, N, K = 48, 128, 128
    w = _weights(N, K, 25)
    x = O.randn(M * K, 26).astype(np.float16)
    b = O.randn(N, 27, 0.1)
    prev = O.randn(M * N, 28).astype(np.float16)
    f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=0, epi=capi.GEPI["bias"], res=1)
    want, got = run(f, dict(w=w, x=x, ev=b), np.float16, M * N, init=prev)
    check(got, want, "gemm bias res", 2e-3)


def test_gemm_offsets(dev):
    """a sub-block of a larger weight (wr0 rows, wk0 columns), x with a k offset and row stride, y with n0 and ld"""
    M, N, K, Nw, Kw = 50, 128, 128, 320, 256
    w = _weights(Nw, Kw, 29)
    ldx = 400
    x = O.randn(M * ldx + 64, 30).astype(np.float16)
    f = dict(w_rows=Nw, w_cols=Kw, M=M, N=N, K=K, wr0=64, wk0=128, x_mode=0, x_off=16, x_ld=ldx, x_k0=40,
             epi=capi.GEPI["f32"], y_off=32, y_ld=N + 40, y_n0=8)
    n_out = 8 + M * (N + 40) + 32
    want, got = run(f, dict(w=w, x=x), np.float32, n_out)
    idx = np.concatenate([8 + 8 + m * (N + 40) + np.arange(N) for m in range(M)])
    check(got[idx], want[idx], "gemm offsets", 1e-5)
    untouched = np.setdiff1d(np.arange(n_out), idx)
    assert np.all(np.isnan(got[untouched]))


def test_gemm_flux_shape_sampled_rows(dev):
    """FLUX.2-klein QKV at full size (M=4608, N=9216, K=3072): every row computed on the GPU, a sample checked"""
    M, N, K = 4608, 9216, 3072
    w = O.fill_q4_sym(N, K, 7, 0.02)
    x32, x16 = O.fill_randn(M * K, 8)
    wb, xb = capi.to_device(w), capi.to_device(x16)
    yb = capi.Buffer(M * N * 4).fill_u32(NAN32)
    capi.q4_gemm(capi.gemm_args(w=wb, w_rows=N, w_cols=K, x=xb, M=M, N=N, K=K, x_mode=0, epi=capi.GEPI["f32"], y=yb))
    rows = np.array([0, 1, 127, 128, 2047, 4095, 4096, 4607])
    y = yb.read(np.float32).reshape(M, N)
    assert np.all(np.isfinite(y))
    sub = np.ascontiguousarray(x16.reshape(M, K)[rows])
    ys = np.zeros(len(rows) * N, np.float32)
    O.q4_gemm(capi.gemm_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=sub.ctypes.data, M=len(rows), N=N, K=K, x_mode=0,
                             epi=capi.GEPI["f32"], y=ys.ctypes.data))
    check(y[rows].ravel(), ys, "FLUX QKV sampled rows", 1e-5)
    for b in (wb, xb, yb):
        b.free()
