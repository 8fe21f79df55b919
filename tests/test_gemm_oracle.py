"""Pins the oracle's dequant-GEMM prologues and epilogues (oracle/q4oracle.c p0o_q4_gemm) against numpy closed forms.

Each case is computed twice: by the oracle (the C restatement of engine/ops/gemm.js) and here by numpy from the
formulas' mathematical statement, written independently of the reference's loop structure (float64 matmuls over the
fp16 operands, RoPE as a complex rotation / rotate_half, RMSNorm by its definition). The data is chosen so that the
plausible misreadings fail:
  * lnmod: activations centred far from zero (mean 5), so a missed centring or a swapped (mean, rstd) is off by ~100%;
    the shift vector sits BEFORE the scale vector, reached through a negative pv stride (a u32 wrap, the way
    klein_blocks passes neg(3072)), so a missed wrap reads past the buffer and a wrong base reads the scale vector;
  * rms: a norm weight far from 1, so a dropped factor shows;
  * resadd / bias: a bias large against the accumulator, so gate * (acc + bias) vs gate * acc + bias differ, and the
    fp16 rounding of the bias epilogue is checked at the bit level (one rounding of acc + bias + residual);
  * bf16: values across the fp16 normal / subnormal / underflow boundaries, converted bf16 -> fp32 -> fp16 (RNE);
  * heads: both RoPE pairings, query / key / value heads, eps that matters (tiny rows), norm weights per column.
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import rel_l2

F16 = np.float16


def _weights(N, K, seed):
    w, deq = O.pack_q4(O.randn(N * K, seed, 0.05), N, K)
    return w, deq.astype(np.float16).astype(np.float64)   # the GEMM's fp16 tile value fl16(fl32(q s + m))


def _run(**kw):
    O.q4_gemm(capi.gemm_args(**kw))


def _fp16_close(got_bits, want, max_frac=0.01):
    """got (fp16 bits) vs want (float64): every element within one fp16 ulp of want's fp16 rounding, and almost all
    exactly equal"""
    w16 = want.astype(np.float16)
    g = got_bits.view(np.float16).astype(np.float64)
    ulp = np.abs(np.spacing(w16.astype(np.float16))).astype(np.float64)
    diff = np.abs(g - w16.astype(np.float64))
    assert np.all(diff <= ulp * 1.0001), float(np.max(diff / ulp))
    assert np.mean(got_bits != w16.view(np.uint16)) <= max_frac


def test_lnmod_prologue_with_wrapped_shift():
    M, N, K, ldx, k0, st_off = 24, 128, 96, 160, 32, 3
    w, wt = _weights(N, K, 31)
    rng = np.random.default_rng(1)
    x = (5.0 + rng.standard_normal((M, ldx))).astype(np.float32)
    stats = np.zeros((M + st_off, 2), np.float32)
    stats[st_off:, 0] = x[:, k0:k0 + K].mean(1) + 0.05          # mean (slightly off: any value works)
    stats[st_off:, 1] = 1.0 / (x[:, k0:k0 + K].std(1) + 0.1)   # rstd
    D = 512
    mod = rng.standard_normal(3 * D).astype(np.float32) * 0.5  # [shift | scale | ...] as the modulation vector
    pv_off, pv_stride = D, (1 << 32) - D                        # scale at D, shift at D - D = 0 (u32 wrap)
    y = np.zeros((M, N), np.float32)
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, x_ld=ldx, x_k0=k0, x_mode=capi.XMODE["lnmod"], M=M,
         N=N, K=K, epi=capi.GEPI["f32"], y=y.ctypes.data, stats=stats.ctypes.data, stats_off=st_off,
         pv=mod.ctypes.data, pv_off=pv_off, pv_stride=pv_stride)
    xs, mean, rstd = x[:, k0:k0 + K], stats[st_off:, 0:1], stats[st_off:, 1:2]
    scale, shift = mod[pv_off + k0:pv_off + k0 + K], mod[k0:k0 + K]
    xp = (((xs - mean) * rstd) * (np.float32(1) + scale) + shift).astype(np.float32).astype(np.float16)
    want = xp.astype(np.float64) @ wt.T
    assert rel_l2(y, want) <= 1e-7
    # the misreadings this data tells apart
    bad_center = (((xs * rstd) * (1 + scale) + shift).astype(np.float16).astype(np.float64)) @ wt.T
    bad_shift = ((((xs - mean) * rstd) * (1 + scale) + mod[pv_off + pv_off + k0:][:K]).astype(np.float16)
                 .astype(np.float64)) @ wt.T
    assert rel_l2(bad_center, want) > 0.5 and rel_l2(bad_shift, want) > 0.1


def test_rms_prologue():
    M, N, K = 16, 64, 128
    w, wt = _weights(N, K, 32)
    rng = np.random.default_rng(2)
    x = (3.0 + rng.standard_normal((M, K))).astype(np.float32)
    stats = np.zeros((M, 2), np.float32)
    stats[:, 0] = 123.0                                      # the rms prologue ignores the mean slot
    stats[:, 1] = 1.0 / np.sqrt((x * x).mean(1) + 1e-6)
    nw = (2.0 + rng.standard_normal(K)).astype(np.float32)
    y = np.zeros((M, N), np.float32)
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, x_mode=capi.XMODE["rms"], M=M, N=N, K=K,
         epi=capi.GEPI["f32"], y=y.ctypes.data, stats=stats.ctypes.data, pv=nw.ctypes.data)
    xp = ((x * stats[:, 1:2]) * nw).astype(np.float32).astype(np.float16)
    want = xp.astype(np.float64) @ wt.T
    assert rel_l2(y, want) <= 1e-7
    assert rel_l2(((x * nw).astype(np.float16).astype(np.float64)) @ wt.T, want) > 0.5   # rstd dropped


def test_bf16_activations_convert_to_fp16_rne():
    M, N, K = 8, 64, 64
    w, wt = _weights(N, K, 33)
    rng = np.random.default_rng(3)
    # rows 0-3 normal, rows 4-5 in fp16's subnormal range, rows 6-7 around its underflow (fp16 rounding is visible there)
    mags = np.concatenate([rng.standard_normal(M * K // 2), rng.standard_normal(M * K // 4) * 1e-5,
                           rng.standard_normal(M * K // 4) * 3e-8])
    xf = mags.astype(np.float32)
    xb = (xf.view(np.uint32) >> 16).astype(np.uint16)                 # bf16 bits (truncated)
    y = np.zeros((M, N), np.float32)
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=xb.ctypes.data, x_mode=capi.XMODE["bf16"], M=M, N=N, K=K,
         epi=capi.GEPI["f32"], y=y.ctypes.data)
    x32 = (xb.astype(np.uint32) << 16).view(np.float32).reshape(M, K)
    want = x32.astype(np.float16).astype(np.float64) @ wt.T
    assert rel_l2(y, want) <= 1e-7
    for r in range(M):
        assert rel_l2(y[r], want[r]) <= 1e-7
    # bf16 read as fp16 bits, or as fp32 without the fp16 rounding, would differ
    assert rel_l2(xb.view(np.float16).reshape(M, K).astype(np.float64) @ wt.T, want) > 0.5
    no16 = x32.astype(np.float64) @ wt.T
    assert rel_l2(no16[4:6], want[4:6]) > 1e-4 and rel_l2(no16[6:], want[6:]) > 1e-2


@pytest.mark.parametrize("store", [0, 1])
def test_resadd_gate_times_acc_plus_bias(store):
    M, N, K, ldy, n0 = 12, 128, 64, 200, 40
    w, wt = _weights(N, K, 34)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((M, K)).astype(np.float16)
    ev = rng.standard_normal(N + 5).astype(np.float32)       # gate at ev_off = 5
    bv = (10.0 + rng.standard_normal(N + 7)).astype(np.float32)  # bias at bv_off = 7, large against acc
    y0 = rng.standard_normal((M, ldy)).astype(np.float32)
    y = y0.copy()
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, M=M, N=N, K=K, epi=capi.GEPI["resadd"],
         y=y.ctypes.data, y_ld=ldy, y_n0=n0, ev=ev.ctypes.data, ev_off=5, bv=bv.ctypes.data, bv_off=7, store=store)
    acc = x.astype(np.float64) @ wt.T
    g, b = ev[5:5 + N].astype(np.float64), bv[7:7 + N].astype(np.float64)
    want = y0.astype(np.float64).copy()
    want[:, n0:n0 + N] = (0 if store else want[:, n0:n0 + N]) + g * (acc + b)
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=2e-5)
    wrong = (0 if store else y0[:, n0:n0 + N]) + g * acc + b
    assert np.max(np.abs(wrong - want[:, n0:n0 + N])) > 1.0
    assert np.array_equal(y[:, :n0], y0[:, :n0]) and np.array_equal(y[:, n0 + N:], y0[:, n0 + N:])


@pytest.mark.parametrize("res", [0, 1])
def test_bias_epilogue_rounds_once(res):
    M, N, K = 32, 128, 64
    w, wt = _weights(N, K, 35)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((M, K)).astype(np.float16)
    ev = rng.standard_normal(N).astype(np.float32) * 3
    y0 = (rng.standard_normal((M, N)) * 4).astype(np.float16)
    y = y0.copy()
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, M=M, N=N, K=K, epi=capi.GEPI["bias"],
         y=y.ctypes.data, ev=ev.ctypes.data, res=res)
    acc = (x.astype(np.float64) @ wt.T).astype(np.float32)   # the fp32 accumulator
    t = acc + ev
    if res:
        t = t + y0.astype(np.float32)
    _fp16_close(y.view(np.uint16), t.astype(np.float64))
    if res:   # rounding acc + bias to fp16 before the residual is a different function
        two = ((acc + ev).astype(np.float16).astype(np.float32) + y0.astype(np.float32)).astype(np.float16)
        assert np.mean(two.view(np.uint16) != y.view(np.uint16)) > 0.05


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_swiglu_gate_up_rows_and_bias(act):
    M, NH, K, wr0, wr1 = 8, 64, 64, 64, 192    # gate rows 64.., up rows 192.. of a 256-row weight
    N = 2 * NH
    w, wt = _weights(256, K, 36)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((M, K)).astype(np.float16)
    bv = rng.standard_normal(300).astype(np.float32)
    y = np.zeros((M, NH), np.float16)
    _run(w=w.ctypes.data, w_rows=256, w_cols=K, x=x.ctypes.data, M=M, N=N, K=K, wr0=wr0, wr1=wr1,
         epi=capi.GEPI["swiglu"], y=y.ctypes.data, y_ld=NH, bv=bv.ctypes.data, bv_off=3, bv_up=100, act=capi.ACT[act])
    xf = x.astype(np.float64)
    g = (xf @ wt[wr0:wr0 + NH].T).astype(np.float32).astype(np.float64) + bv[3:3 + NH]
    u = (xf @ wt[wr1:wr1 + NH].T).astype(np.float32).astype(np.float64) + bv[103:103 + NH]
    if act == "gelu":
        a = 0.5 * g * (1 + np.tanh(np.clip(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3), -15, 15)))
    else:
        a = g / (1 + np.exp(-g))
    _fp16_close(y.view(np.uint16), a * u)


def _rope_table(L, seed):
    ang = np.random.default_rng(seed).uniform(-3, 3, (L, 64))
    t = np.zeros((L, 128), np.float32)
    t[:, 0::2], t[:, 1::2] = np.cos(ang), np.sin(ang)
    return t


@pytest.mark.parametrize("mode", ["inter", "half"])
def test_heads_qk_rmsnorm_rope_head_major(mode):
    M, K, Hq, Hkv, Ltot, row0 = 20, 64, 3, 2, 40, 11
    H = Hq + 2 * Hkv
    N = H * 128
    w, wt = _weights(N, K, 37)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((M, K)).astype(np.float16)
    x[3] *= np.float16(1e-3)                                 # a row whose sum of squares is small: eps matters
    ev = (1.0 + 0.5 * rng.standard_normal(256 + 9)).astype(np.float32)   # q norm at 9, k norm at 9 + 128
    rope = _rope_table(Ltot, 8)
    eps = 1e-4
    y = np.full(H * Ltot * 128, 0x7E00, np.uint16)
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, M=M, N=N, K=K, epi=capi.GEPI["heads"],
         y=y.ctypes.data, ev=ev.ctypes.data, ev_off=9, heads_ltot=Ltot, heads_row_off=row0, heads_hq=Hq,
         heads_hkv=Hkv, heads_eps=eps, heads_rope=capi.ROPE[mode], rope=rope.ctypes.data)
    acc = (x.astype(np.float64) @ wt.T).astype(np.float32).astype(np.float64).reshape(M, H, 128)
    cs, sn = rope[row0:row0 + M, 0::2].astype(np.float64), rope[row0:row0 + M, 1::2].astype(np.float64)
    want = np.zeros((H, M, 128))
    for h in range(H):
        v = acc[:, h, :]
        if h >= Hq + Hkv:
            want[h] = v
            continue
        nw = ev[9 + (128 if h >= Hq else 0):][:128].astype(np.float64)
        t = v / np.sqrt((v * v).mean(1, keepdims=True) + eps) * nw
        if mode == "inter":   # consecutive pairs as complex numbers, rotated by e^{i angle}
            z = (t[:, 0::2] + 1j * t[:, 1::2]) * (cs + 1j * sn)
            r = np.empty_like(t)
            r[:, 0::2], r[:, 1::2] = z.real, z.imag
        else:                 # rotate_half: t cos + [-t2, t1] sin, the angle of entry d for both d and d + 64
            c2, s2 = np.concatenate([cs, cs], 1), np.concatenate([sn, sn], 1)
            r = t * c2 + np.concatenate([-t[:, 64:], t[:, :64]], 1) * s2
        want[h] = r
    got = y.reshape(H, Ltot, 128)
    _fp16_close(got[:, row0:row0 + M].copy().view(np.uint16).ravel(), want.ravel())
    untouched = np.ones(Ltot, bool)
    untouched[row0:row0 + M] = False
    assert np.all(got[:, untouched].view(np.uint16) == 0x7E00)


def test_heads_without_norm_or_rotation_differs():
    """sanity of the pins above: the value heads are a plain fp16 store, the query heads are not"""
    M, K = 4, 64
    N = 3 * 128
    w, wt = _weights(N, K, 38)
    x = np.random.default_rng(9).standard_normal((M, K)).astype(np.float16)
    ev = np.ones(256, np.float32)
    rope = _rope_table(M, 10)
    y = np.zeros(3 * M * 128, np.uint16)
    _run(w=w.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, M=M, N=N, K=K, epi=capi.GEPI["heads"],
         y=y.ctypes.data, ev=ev.ctypes.data, heads_ltot=M, heads_hq=1, heads_hkv=1, heads_rope=0,
         rope=rope.ctypes.data)
    acc = (x.astype(np.float64) @ wt.T).astype(np.float32).reshape(M, 3, 128)
    got = y.view(np.float16).reshape(3, M, 128)
    assert np.array_equal(got[2], acc[:, 2].astype(np.float16))
    assert not np.array_equal(got[0], acc[:, 0].astype(np.float16))
