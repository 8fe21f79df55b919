"""GPU parity of the dequant-GEMM at the BASELINE DiT configurations and with the heads epilogue, through the C ABI.

  * config D (FLUX.2-klein block, M = 4608): qkv, out, mlp_up and mlp_down with bf16 activations and fp16 outputs, as
    bench.py runs them, plus the block's real calls: the lnmod + heads qkv of engine/pocketflux-engine.js:2341-2344,
    the gated resadd out projection and the lnmod + swiglu MLP with the resadd down projection (:2325-2335, 2349);
  * config E (SANA-Video, M = 32760): qkv, glu_up (swiglu) and down with bf16 activations;
  * the heads epilogue (engine/ops/gemm.js:212-250) in both RoPE modes, query / key / value heads, a row offset into
    Ltot rows, and rows past M left untouched;
  * a recording that captured a staged GEMM still replays correctly after a larger GEMM grew the staging workspace.
Full-size outputs are computed whole on the GPU and checked on sampled rows against the oracle (the oracle on the
sampled rows' inputs; bit-identical operands), plus finiteness everywhere. Tolerance: relative L2 <= 1e-3 (BASELINE),
and this build's bars: 1e-5 for fp32 outputs, 2e-3 for fp16 outputs (half an fp16 ulp is 2^-11 relative).
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

pytestmark = pytest.mark.gpu
NAN32, NAN16x2 = 0x7FC00000, 0x7E007E00
ROWS = np.array([0, 1, 255, 256, 2047, 2048, 4095, 4607])


def check(got, want, what, tol_build):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    r = rel_l2(got, want)
    print(f"{what}: rel_l2 {r:.3e}", flush=True)
    assert np.all(np.isfinite(got)), what + ": unwritten outputs"
    assert r <= 1e-3 and r <= tol_build, (what, r)


def bf16_rows(M, K, seed):
    x = np.random.default_rng(seed).standard_normal(M * K, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def oracle_rows(w, N, K, rows, xrows, **kw):
    """the oracle over the sampled rows only (their activations `xrows`)"""
    out_f32 = kw.pop("out_f32", False)
    epi = kw.pop("epi", capi.GEPI["f32"] if out_f32 else capi.GEPI["f16"])
    ncol = N // 2 if epi == capi.GEPI["swiglu"] else N
    y = np.zeros(len(rows) * ncol, np.float32 if out_f32 else np.float16)
    O.q4_gemm(capi.gemm_args(w=w.ctypes.data, w_rows=kw.pop("w_rows", N), w_cols=K, x=xrows.ctypes.data,
                             M=len(rows), N=N, K=K, epi=epi, y=y.ctypes.data, y_ld=ncol, **kw))
    return y.reshape(len(rows), ncol)


@pytest.mark.parametrize("name,M,N,K,epi", [
    ("flux qkv", 4608, 9216, 3072, "f16"), ("flux out", 4608, 3072, 3072, "f16"),
    ("flux mlp_up", 4608, 9216, 3072, "f16"), ("flux mlp_down", 4608, 3072, 9216, "f16"),
    ("sana qkv", 32760, 9216, 3072, "f16"), ("sana glu_up", 32760, 16384, 3072, "swiglu"),
    ("sana down", 32760, 3072, 8192, "f16"),
])
def test_dit_gemm_bf16_at_baseline_shapes(dev, name, M, N, K, epi):
    """configs D and E as bench.py runs them: symmetric BASELINE weights, bf16 N(0,1) activations, fp16 outputs"""
    print("case", name, M, N, K, epi, flush=True)
    w = O.fill_q4_sym(N, K, 100 + N % 97, 0.02)
    xb = bf16_rows(M, K, 3)
    ncol = N // 2 if epi == "swiglu" else N
    extra = dict(wr0=0, wr1=N // 2) if epi == "swiglu" else {}
    wb, xd = capi.to_device(w), capi.to_device(xb)
    yb = capi.Buffer(M * ncol * 2).fill_u32(NAN16x2)
    capi.q4_gemm(capi.gemm_args(w=wb, w_rows=N, w_cols=K, x=xd, x_ld=K, x_mode=capi.XMODE["bf16"], M=M, N=N, K=K,
                                epi=capi.GEPI[epi], y=yb, y_ld=ncol, **extra))
    y = yb.read(np.float16).reshape(M, ncol)
    assert np.all(np.isfinite(y)), name
    rows = np.unique(np.concatenate([ROWS[ROWS < M], [M - 1, M // 2]]))
    sub = np.ascontiguousarray(xb.reshape(M, K)[rows])
    want = oracle_rows(w, N, K, rows, sub, x_mode=capi.XMODE["bf16"], epi=capi.GEPI[epi], **extra)
    check(y[rows].astype(np.float32), want.astype(np.float32), name + " sampled rows", 2e-3)
    for b in (wb, xd, yb):
        b.free()


def rope_table(L, seed, mode):
    """a RoPE table [L][64][cos, sin] shaped as the callers build it (engine/pocketflux-engine.js:2271-2300)"""
    rng = np.random.default_rng(seed)
    pos = rng.integers(0, 64, (L, 4)).astype(np.float64)
    ang = np.zeros((L, 64))
    for p in range(64):
        ang[:, p] = pos[:, p >> 4] * 2000.0 ** (-(p & 15) / 16) if mode == "inter" else pos[:, 0] * 1e6 ** (-2 * p / 128)
    t = np.zeros((L, 128), np.float32)
    t[:, 0::2], t[:, 1::2] = np.cos(ang), np.sin(ang)
    return t


@pytest.mark.parametrize("mode,M,Hq,Hkv,Ltot,row0,xmode", [
    ("inter", 300, 2, 2, 520, 200, "lnmod"),     # FLUX: Hq = Hkv, lnmod prologue, img rows after txt rows
    ("half", 257, 4, 1, 257, 0, "rms"),          # Qwen3 TE: 4 query heads per kv head, rms prologue
    ("inter", 64, 1, 0, 64, 0, "f16"),           # one query head, no key / value heads
    ("half", 64, 1, 0, 64, 0, "f16"),            # odd head counts: the last column tile holds one real head
    ("half", 100, 1, 1, 120, 20, "f16"),         # H = 3
    ("inter", 130, 3, 1, 150, 10, "lnmod"),      # H = 5
])
def test_heads_epilogue_vs_oracle(dev, mode, M, Hq, Hkv, Ltot, row0, xmode):
    H = Hq + 2 * Hkv
    N, K = H * 128, 384
    print("case heads", mode, M, Hq, Hkv, Ltot, row0, xmode, flush=True)
    w = O.pack_q4(O.randn(N * K, 51, 0.05), N, K)[0]
    ev = (1.0 + 0.3 * O.randn(256 + 5, 52)).astype(np.float32)
    rope = rope_table(Ltot, 53, mode)
    arrays = dict(w=w, ev=ev, rope=rope)
    f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, epi=capi.GEPI["heads"], ev_off=5, heads_ltot=Ltot,
             heads_row_off=row0, heads_hq=Hq, heads_hkv=Hkv, heads_eps=1.1920928955078125e-7 if mode == "inter" else 1e-6,
             heads_rope=capi.ROPE[mode], x_mode=capi.XMODE[xmode])
    if xmode == "f16":
        arrays["x"] = O.randn(M * K, 54).astype(np.float16)
    else:
        x = (2.0 + O.randn(M * K, 54)).astype(np.float32)
        xr = x.reshape(M, K).astype(np.float64)
        st = np.zeros(2 * M, np.float32)
        st[0::2] = xr.mean(1)
        st[1::2] = 1 / np.sqrt(xr.var(1) + 1e-6)
        pv = O.randn(3 * K, 55, 0.2)
        arrays.update(x=x, stats=st, pv=pv)
        f.update(pv_off=K, pv_stride=(1 << 32) - K)
    n_out = H * Ltot * 128
    want = np.full(n_out, np.nan, np.float16)
    O.q4_gemm(capi.gemm_args(**f, **{k: v.ctypes.data for k, v in arrays.items()}, y=want.ctypes.data))
    devb = {k: capi.to_device(v) for k, v in arrays.items()}
    # Y with a tail of one more head's rows: a head past N / 128 (a 256-column tile's second head when H is odd) must
    # not be written
    tail = Ltot * 128
    yb = capi.Buffer((n_out + tail) * 2).fill_u32(NAN16x2)
    capi.q4_gemm(capi.gemm_args(**f, **devb, y=yb))
    full = yb.read(np.uint16)
    assert np.all(full[n_out:] == 0x7E00), "the heads epilogue wrote past the last head"
    got = full[:n_out].view(np.float16).reshape(H, Ltot, 128)
    want = want.reshape(H, Ltot, 128)
    inside = got[:, row0:row0 + M].astype(np.float32)
    check(inside, want[:, row0:row0 + M].astype(np.float32), f"heads {mode}", 2e-3)
    for h in range(H):   # per head: the norm and the rotation act per head, so each head must agree on its own
        r = rel_l2(inside[h], want[h, row0:row0 + M].astype(np.float32))
        assert r <= 2e-3, (h, r)
    outside = np.ones(Ltot, bool)
    outside[row0:row0 + M] = False
    assert np.all(np.isnan(got[:, outside].astype(np.float32)))
    for b in list(devb.values()) + [yb]:
        b.free()


def test_flux_block_qkv_lnmod_heads_at_full_size(dev):
    """config D's qkv exactly as klein_blocks calls it (engine/pocketflux-engine.js:2341-2344, ditSingle :2362-2364):
    L = 4608 rows of the fp32 residual, lnmod prologue with the modulation's scale at mo + 3072 and shift at mo
    (stride neg(3072)), heads epilogue with 24 + 24 + 24 heads, QK eps = fp32 epsilon, FLUX interleaved RoPE"""
    L, D, NH = 4608, 3072, 24
    N = 3 * D
    w = O.fill_q4_sym(N, D, 61, 0.02)
    x = (0.5 + np.random.default_rng(62).standard_normal(L * D, dtype=np.float32)).astype(np.float32)
    xr = x.reshape(L, D)
    st = np.zeros(2 * L, np.float32)
    st[0::2] = xr.mean(1)
    st[1::2] = 1 / np.sqrt(xr.var(1) + 1e-6)
    mo = 1000
    mod = O.randn(mo + 2 * D, 63, 0.3)
    ev = (1 + 0.2 * O.randn(256, 64)).astype(np.float32)
    rope = rope_table(L, 65, "inter")
    f = dict(w_rows=N, w_cols=D, M=L, N=N, K=D, x_mode=capi.XMODE["lnmod"], pv_off=mo + D, pv_stride=(1 << 32) - D,
             epi=capi.GEPI["heads"], heads_ltot=L, heads_hq=NH, heads_hkv=NH, heads_eps=1.1920928955078125e-7,
             heads_rope=capi.ROPE["inter"])
    d = {k: capi.to_device(v) for k, v in dict(w=w, x=x, stats=st, pv=mod, ev=ev, rope=rope).items()}
    yb = capi.Buffer(3 * NH * L * 128 * 2).fill_u32(NAN16x2)
    capi.q4_gemm(capi.gemm_args(**f, **d, y=yb))
    got = yb.read(np.float16).reshape(3 * NH, L, 128)
    assert np.all(np.isfinite(got.astype(np.float32)))
    rows = ROWS
    sub = dict(w=w, x=np.ascontiguousarray(xr[rows]), stats=np.ascontiguousarray(st.reshape(L, 2)[rows]), pv=mod,
               ev=ev, rope=np.ascontiguousarray(rope[rows]))
    want = np.zeros(3 * NH * len(rows) * 128, np.float16)
    O.q4_gemm(capi.gemm_args(**dict(f, M=len(rows), heads_ltot=len(rows)), **{k: v.ctypes.data for k, v in sub.items()},
                             y=want.ctypes.data))
    check(got[:, rows].astype(np.float32), want.reshape(3 * NH, len(rows), 128).astype(np.float32),
          "FLUX qkv lnmod+heads sampled rows", 2e-3)
    for b in list(d.values()) + [yb]:
        b.free()


def test_flux_block_out_and_mlp_calls(dev):
    """the rest of a FLUX double block as klein_blocks calls it at M = 4608: the gated resadd projection
    (engine/pocketflux-engine.js:2349-2350) and mlpChunks' lnmod + swiglu then gated resadd down (:2325-2335), here
    in one chunk of 4608 rows"""
    L, D, MLP = 4608, 3072, 9216
    rng = np.random.default_rng(71)
    w_proj = O.fill_q4_sym(D, D, 72, 0.02)
    w_up = O.fill_q4_sym(2 * MLP, D, 73, 0.02)
    w_dn = O.fill_q4_sym(D, MLP, 74, 0.02)
    o16 = rng.standard_normal(L * D, dtype=np.float32).astype(np.float16)
    resid = rng.standard_normal(L * D, dtype=np.float32)
    xr = resid.reshape(L, D).astype(np.float64)
    st = np.zeros(2 * L, np.float32)
    st[0::2] = xr.mean(1)
    st[1::2] = 1 / np.sqrt(xr.var(1) + 1e-6)
    mod = O.randn(6 * D, 75, 0.3)
    gate = O.randn(D, 76, 0.5)
    d = {k: capi.to_device(v) for k, v in dict(wp=w_proj, wu=w_up, wd=w_dn, o=o16, st=st, mod=mod, g=gate).items()}
    r1 = capi.to_device(resid)
    m16 = capi.Buffer(L * MLP * 2).fill_u32(NAN16x2)
    r2 = capi.to_device(resid)
    capi.q4_gemm(capi.gemm_args(w=d["wp"], w_rows=D, w_cols=D, x=d["o"], M=L, N=D, K=D, epi=capi.GEPI["resadd"],
                                y=r1, ev=d["g"]))
    capi.q4_gemm(capi.gemm_args(w=d["wu"], w_rows=2 * MLP, w_cols=D, x=r2, x_mode=capi.XMODE["lnmod"], stats=d["st"],
                                pv=d["mod"], pv_off=4 * D, pv_stride=(1 << 32) - D, M=L, N=2 * MLP, K=D, wr0=0,
                                wr1=MLP, epi=capi.GEPI["swiglu"], y=m16, y_ld=MLP))
    capi.q4_gemm(capi.gemm_args(w=d["wd"], w_rows=D, w_cols=MLP, x=m16, M=L, N=D, K=MLP, epi=capi.GEPI["resadd"],
                                y=r2, ev=d["g"]))
    g_r1 = r1.read(np.float32).reshape(L, D)
    g_m = m16.read(np.float16).reshape(L, MLP)
    g_r2 = r2.read(np.float32).reshape(L, D)
    rows = ROWS
    rr = np.ascontiguousarray(resid.reshape(L, D)[rows])
    want1 = rr.copy()
    orow = np.ascontiguousarray(o16.reshape(L, D)[rows])   # bound to a name: ctypes takes its address
    O.q4_gemm(capi.gemm_args(w=w_proj.ctypes.data, w_rows=D, w_cols=D, x=orow.ctypes.data, M=len(rows), N=D, K=D,
                             epi=capi.GEPI["resadd"], y=want1.ctypes.data, ev=gate.ctypes.data))
    check(g_r1[rows], want1, "FLUX proj resadd", 1e-5)
    want_m = np.zeros((len(rows), MLP), np.float16)
    st_s = np.ascontiguousarray(st.reshape(L, 2)[rows])
    O.q4_gemm(capi.gemm_args(w=w_up.ctypes.data, w_rows=2 * MLP, w_cols=D, x=rr.ctypes.data, x_mode=capi.XMODE["lnmod"],
                             stats=st_s.ctypes.data, pv=mod.ctypes.data, pv_off=4 * D, pv_stride=(1 << 32) - D,
                             M=len(rows), N=2 * MLP, K=D, wr0=0, wr1=MLP, epi=capi.GEPI["swiglu"],
                             y=want_m.ctypes.data, y_ld=MLP))
    check(g_m[rows].astype(np.float32), want_m.astype(np.float32), "FLUX mlp lnmod+swiglu", 2e-3)
    want2 = rr.copy()   # the down projection reads the GPU's own MLP rows: the check isolates this GEMM
    mrow = np.ascontiguousarray(g_m[rows])
    O.q4_gemm(capi.gemm_args(w=w_dn.ctypes.data, w_rows=D, w_cols=MLP, x=mrow.ctypes.data, M=len(rows), N=D, K=MLP,
                             epi=capi.GEPI["resadd"], y=want2.ctypes.data, ev=gate.ctypes.data))
    check(g_r2[rows], want2, "FLUX mlp down resadd", 1e-5)
    for b in list(d.values()) + [r1, r2, m16]:
        b.free()


def test_recording_keeps_its_staging_workspace(dev):
    """a recorded bf16 GEMM (staged through the activation workspace) replays correctly after a larger staged GEMM
    grew the workspace: the recording holds the buffer it captured (the growth would otherwise free it under it)"""
    M, N, K = 256, 256, 512
    w = O.pack_q4(O.randn(N * K, 81, 0.05), N, K)[0]
    xb = bf16_rows(M, K, 82)
    want = np.zeros(M * N, np.float32)
    O.q4_gemm(capi.gemm_args(w=w.ctypes.data, w_rows=N, w_cols=K, x=xb.ctypes.data, x_mode=capi.XMODE["bf16"], M=M,
                             N=N, K=K, epi=capi.GEPI["f32"], y=want.ctypes.data))
    wb, xd = capi.to_device(w), capi.to_device(xb)
    yb = capi.Buffer(M * N * 4)
    args = capi.gemm_args(w=wb, w_rows=N, w_cols=K, x=xd, x_mode=capi.XMODE["bf16"], M=M, N=N, K=K,
                          epi=capi.GEPI["f32"], y=yb)
    capi.q4_gemm(args)   # sizes the workspace outside the recording
    capi.done()
    rec = capi.record(lambda: capi.q4_gemm(args))
    # a staged GEMM whose activations need more than the workspace holds (> 256 MiB of fp16 rows): it grows
    Mb, Kb = 33024, 4096
    big_x = capi.Buffer(Mb * Kb * 2).fill_u32(0x3F803F80)   # bf16 1.0
    big_w = capi.Buffer(64 // 64 * Kb // 32 * 1280)
    capi.fill_q4_sym(big_w, 64, Kb, 83, 0.02)
    big_y = capi.Buffer(Mb * 64 * 2)
    capi.q4_gemm(capi.gemm_args(w=big_w, w_rows=64, w_cols=Kb, x=big_x, x_mode=capi.XMODE["bf16"], M=Mb, N=64, K=Kb,
                                epi=capi.GEPI["f16"], y=big_y))
    capi.done()
    for b in (big_x, big_w, big_y):
        b.free()
    for i in range(3):
        yb.fill_u32(NAN32)
        rec.replay()
        got = yb.read(np.float32)
        check(got, want, f"replay {i} after the workspace grew", 1e-5)
    rec.free()
    for b in (wb, xd, yb):
        b.free()


def test_chain_refuses_other_ops(dev):
    """gemv / gemvM, copy, argmax, rowstats and normadd calls join a chain: a GEMM called while one is being built is
    refused instead of running out of order"""
    w = capi.Buffer(1280)
    x = capi.Buffer(256)
    y = capi.Buffer(256)
    capi.check(capi.lib().p0_chain_begin())
    try:
        a = capi.gemm_args(w=w, w_rows=64, w_cols=32, x=x, M=1, N=64, K=32, epi=capi.GEPI["f32"], y=y)
        fl = capi.C.c_double()
        assert capi.lib().p0_q4_gemm(capi.C.byref(a), capi.C.byref(fl)) == capi.P0_EINVAL
        assert "calls join a chain" in capi.last_error()
    finally:
        h = capi.vp()
        capi.lib().p0_chain_end(capi.C.byref(h))   # an empty chain: refused, nothing to free
    for b in (w, x, y):
        b.free()
