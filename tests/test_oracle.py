"""Pins the CPU oracle (oracle/q4oracle.c) against textbook routines, closed forms and independent decodings.

The reference ships no golden vectors for this path (its checks run in a browser against a CPU reference,
engine/kcheck.js:67-137, engine/tune/kshipped.js:17-61), so each oracle function is pinned here by something that a
plausible mistake (a dropped min term, a swapped nibble, a transposed operand, a wrong split index) would fail.
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi
from tests.conftest import cos_sim, rel_l2


# ------------------------------------------------------------------------------------------------ fp16 conversion
def test_h2f_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.h2f(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_vs_numpy_rne():
    rng = np.random.default_rng(0)
    # random bit patterns over the whole f32 range, plus every half value, every midpoint between neighbours
    # (ties to even), midpoints +- 1 f32 ulp, the subnormal range and the overflow boundary
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    vals = [bits.view(np.float32)]
    halves = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (halves[:-1] + halves[1:]) / 2
    vals += [halves.astype(np.float32), mids.astype(np.float32)]
    m32 = mids.astype(np.float32)
    vals += [np.nextafter(m32, np.float32(np.inf)), np.nextafter(m32, np.float32(-np.inf))]
    vals += [np.float32([65504, 65519, 65519.996, 65520, 65536, 1e9, np.inf, -np.inf, 0.0, -0.0, 2**-24, 2**-25,
                         1.5 * 2**-25, 2**-26, 6.1e-5, -6.1e-5])]
    x = np.concatenate([v.astype(np.float32) for v in vals])
    x = np.concatenate([x, -x])
    got = O.f2h(x)
    want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7fff) == 0x7e00)


# ------------------------------------------------------------------------------------------------ RNG (kcheck.js:10-11)
def _js_xorshift(seed, n):
    """The recurrence evaluated with JavaScript's number semantics: ToInt32 on <<, >>, ^ and ToUint32 on >>>= 0."""
    def to_i32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v & 0x80000000 else v

    s = (seed & 0xFFFFFFFF) or 1
    out = []
    for _ in range(n):
        s = to_i32(s) ^ to_i32(to_i32(s) << 13)
        s &= 0xFFFFFFFF
        s = to_i32(s) ^ (to_i32(s) >> 17)      # arithmetic shift of the int32 view
        s = to_i32(s) ^ to_i32(to_i32(s) << 5)
        s &= 0xFFFFFFFF
        out.append(s / 4294967296)
    return out


@pytest.mark.parametrize("seed", [1, 7, 11, 31, 0x9E3779B9, 0xFFFFFFFF])
def test_rng_matches_js_semantics(seed):
    assert np.array_equal(O.rng_uniform(seed, 200), np.array(_js_xorshift(seed, 200)))


def test_rng_sign_extension_is_observable():
    # a logical-shift xorshift32 would differ from the JS recurrence on this seed within a few steps
    s, logical = 0x80000001, []
    for _ in range(8):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        logical.append(s / 4294967296)
    assert not np.array_equal(O.rng_uniform(0x80000001, 8), np.array(logical))


def test_randn_moments():
    x = O.randn(400_000, 7, 0.05).astype(np.float64)
    assert abs(x.mean()) < 0.05 * 0.01
    assert abs(x.std() / 0.05 - 1) < 0.01
    # Box-Muller pairs: the first two values from the first two uniforms
    u = O.rng_uniform(7, 2)
    m = np.sqrt(-2 * np.log(max(u[0], 1e-9))) * 0.05
    assert x[0] == np.float32(m * np.cos(2 * np.pi * u[1]))
    assert x[1] == np.float32(m * np.sin(2 * np.pi * u[1]))


# ------------------------------------------------------------------------------------------------ packQ4 / dequant
def np_decode(w, N, K):
    """q4g32a.t64 decoded by the KERNELS' rule (u32 word w of row r, nibble i -> k = 32 g + 8 w + i; u32 256 + r =
    f16 scale | f16 min << 16; engine/llm/lops.js:67-71), independent of the packer's byte rule."""
    rec = np.ascontiguousarray(w, np.uint8).reshape(N // 64, K // 32, 1280)
    words = rec[:, :, :1024].copy().view(np.uint32).reshape(N // 64, K // 32, 64, 4)
    sm = rec[:, :, 1024:].copy().view(np.uint32).reshape(N // 64, K // 32, 64)
    q = (words[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    q = q.reshape(N // 64, K // 32, 64, 32).astype(np.float32)
    s = (sm & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    m = (sm >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    deq = q * s[..., None] + m[..., None]      # q * s exact in f32, then one rounding
    return deq.transpose(0, 2, 1, 3).reshape(N, K), q.transpose(0, 2, 1, 3).reshape(N, K), s, m


@pytest.mark.parametrize("N,K,seed", [(64, 32, 1), (128, 256, 11), (192, 96, 5)])
def test_pack_q4_decodes_by_kernel_rule(N, K, seed):
    W = O.randn(N * K, seed, 0.05).reshape(N, K)
    b, deq = O.pack_q4(W, N, K)
    d2, q, s, m = np_decode(b, N, K)
    assert np.array_equal(deq.view(np.uint32), d2.view(np.uint32))   # packQ4's own deq == the kernels' decode
    assert q.min() >= 0 and q.max() <= 15
    # |deq - W| <= s / 2 (round to nearest code) + fp16 rounding of min; the per (row, group) scale
    s_full = np.repeat(s.transpose(0, 2, 1).reshape(N, K // 32), 32, axis=1)
    assert np.all(np.abs(deq - W) <= s_full * 0.5 + 1e-3 * np.abs(W).max())
    # the recorded min is fl16(min of the group), the scale fl16((max - min) / 15) (engine/kcheck.js:28-30)
    g = W.reshape(N, K // 32, 32)
    mn = g.min(-1).astype(np.float16).astype(np.float64)
    sc = ((g.max(-1) - mn) / 15).astype(np.float32).astype(np.float16).astype(np.float32)
    assert np.array_equal(m.transpose(0, 2, 1).reshape(N, K // 32), mn.astype(np.float32))
    assert np.array_equal(s.transpose(0, 2, 1).reshape(N, K // 32), np.where(sc == 0, 1, sc))


def test_pack_q4_symmetric_roundtrip():
    """codes q in [0, 15] with scale s and min -8 s: a group holding both 0 and 15 packs back to itself exactly"""
    N, K = 128, 128
    rng = np.random.default_rng(3)
    q = rng.integers(0, 16, size=(N, K))
    q[:, ::32] = 0
    q[:, 1::32] = 15
    s = np.abs(rng.normal(0, 0.02, size=(N, K // 32))).astype(np.float16).astype(np.float32)
    m = (-8 * s).astype(np.float16).astype(np.float32)
    assert np.array_equal(m, -8 * s)                          # exact in fp16
    W = q * np.repeat(s, 32, 1) + np.repeat(m, 32, 1)
    b, deq = O.pack_q4(W.astype(np.float32), N, K)
    d2, q2, s2, m2 = np_decode(b, N, K)
    assert np.array_equal(q2, q.astype(np.float32))
    assert np.array_equal(deq, W.astype(np.float32))


def test_dequant_q4_is_pack_deq_and_fp16_tile():
    N, K = 128, 192
    W = O.randn(N * K, 21, 0.05).reshape(N, K)
    b, deq = O.pack_q4(W, N, K)
    o32, o16 = O.dequant_q4(b, N, K)
    assert np.array_equal(o32.view(np.uint32), deq.view(np.uint32))
    assert np.array_equal(o16, o32.astype(np.float16).view(np.uint16))


def test_fill_q4_sym_is_symmetric_baseline_data():
    N, K = 128, 256
    w = O.fill_q4_sym(N, K, 123, 0.02)
    deq, q, s, m = np_decode(w, N, K)
    assert np.array_equal(m, -8 * s)                  # min = -8 scale: symmetric codes q - 8 in [-8, 7]
    assert np.all(s > 0)
    assert abs(np.sqrt((s.astype(np.float64) ** 2).mean()) / 0.02 - 1) < 0.05   # |N(0, 0.02)|: E s^2 = sigma^2
    hist = np.bincount(q.astype(np.int64).ravel(), minlength=16) / q.size
    assert np.all(np.abs(hist - 1 / 16) < 0.01)
    assert np.array_equal(deq, ((q - 8) * np.repeat(s.transpose(0, 2, 1).reshape(N, K // 32), 32, 1)).astype(np.float32))
    assert O.lib().p0o_hash(0) == 129708002        # the published PCG hash's value at 0 (pcg_hash in JCGT 2020)


# ------------------------------------------------------------------------------------------------ GEMV / GEMV-M
def _gelu(v):
    v = np.asarray(v, np.float64)
    return v * 0.5 * (1 + np.tanh(np.clip(0.7978845608028654 * (v + 0.044715 * v ** 3), -15, 15)))


def _weights(N, K, seed):
    W = O.randn(N * K, seed, 0.05).reshape(N, K)
    b, deq = O.pack_q4(W, N, K)
    return b, deq.astype(np.float64)


def _gemv_case(pro, epi, N, K, kPer, seed=1):
    rows = 2 * N if epi == "geglu" else N
    b, deq = _weights(rows, K, seed)
    x = O.randn(3 * K, seed + 1)          # several producer rows (sum / pleg partials)
    nw = (0.9 + 0.2 * ((np.arange(K) * 7919) % 100) / 100).astype(np.float32)
    ev = O.randn(K, seed + 2, 0.5)
    rs = np.float32(1 / np.sqrt((x[:K].astype(np.float64) ** 2).mean() + 1e-6))
    NT = N // 64
    stat = np.zeros(NT * 2 + 4, np.float32)
    stat[NT * 2] = rs
    kch = ((K + 255) // 256) * 256 if (not kPer and K > 2048) else 2048
    kp = min(kch, kPer or K)
    nsplit = -(-K // kp)
    y = np.full(nsplit * N, np.nan, np.float32)
    mx = stat.copy()
    a = capi.gemv_args(w=b.ctypes.data, w_rows=rows, w_cols=K, x=x.ctypes.data, x_rowB=0, N=N, K=K, kPer=kPer,
                       pro=capi.PRO[pro], epi=capi.EPI[epi], y=y.ctypes.data, ldy=N,
                       stat=(mx if epi == "softcap" else stat).ctypes.data, stat_off=NT * 2,
                       norm=nw.ctypes.data, norm_off=0, src_n=2, src_ld=K, ev=ev.ctypes.data, ev_off=0,
                       mx=mx.ctypes.data, cap=30.0)
    ns = O.q4_gemv(a)
    assert ns == nsplit
    xs = x.astype(np.float64)
    if pro == "raw":
        xp = x[:K].astype(np.float32)
    elif pro == "rms":
        xp = (x[:K] * rs).astype(np.float32) * nw
    else:
        sm = (x[:K] + x[K:2 * K]).astype(np.float32)
        xp = sm if pro == "sum" else (_gelu(sm).astype(np.float32) * ev)
    return dict(y=y, mx=mx, deq=deq, xp=xp.astype(np.float64), nsplit=nsplit, kp=kp, N=N, K=K, xs=xs)


@pytest.mark.parametrize("pro", ["raw", "rms", "sum", "pleg"])
def test_gemv_store_vs_numpy(pro):
    c = _gemv_case(pro, "store", 128, 256, 0)
    want = c["deq"] @ c["xp"]
    assert rel_l2(c["y"], want) < 1e-6


def test_gemv_split_partials_sum_to_whole():
    N, K = 128, 8192
    c = _gemv_case("raw", "store", N, K, 2048)
    assert c["nsplit"] == 4
    parts = c["y"].reshape(4, N).astype(np.float64)
    for s in range(4):   # each partial is its own k range
        want = c["deq"][:, s * 2048:(s + 1) * 2048] @ c["xp"][s * 2048:(s + 1) * 2048]
        assert rel_l2(parts[s], want) < 1e-6
    assert rel_l2(parts.sum(0), c["deq"] @ c["xp"]) < 1e-6


def test_gemv_ragged_last_split():
    c = _gemv_case("raw", "store", 64, 2048 + 96, 1024)
    assert c["nsplit"] == 3
    parts = c["y"].reshape(3, 64).astype(np.float64)
    assert rel_l2(parts[2], c["deq"][:, 2048:] @ c["xp"][2048:]) < 1e-6


def test_gemv_geglu_vs_closed_form():
    c = _gemv_case("rms", "geglu", 128, 256, 0)
    d = c["deq"] @ c["xp"]
    want = _gelu(d[:128].astype(np.float32)) * d[128:]
    assert rel_l2(c["y"][:128], want) < 1e-6


def test_gemv_softcap_and_tile_argmax():
    c = _gemv_case("rms", "softcap", 256, 256, 0)
    d = c["deq"] @ c["xp"]
    want = 30 * np.tanh(np.clip(d / 30, -15, 15))
    assert rel_l2(c["y"][:256], want) < 1e-6
    mx = c["mx"]
    for t in range(4):
        seg = c["y"][t * 64:(t + 1) * 64]
        assert mx[2 * t] == seg.max()
        assert mx[2 * t + 1:2 * t + 2].view(np.uint32)[0] == t * 64 + int(np.argmax(seg))   # first max = lowest index


def test_gemvM_rows_vs_numpy():
    M, N, K = 5, 128, 512
    b, deq = _weights(N, K, 4)
    x = O.randn(M * K, 9)
    nw = np.linspace(0.5, 1.5, K).astype(np.float32)
    st = np.zeros(2 * M, np.float32)
    st[1::2] = np.linspace(0.7, 1.3, M)
    y = np.full(M * N, np.nan, np.float32)
    a = capi.gemvm_args(w=b.ctypes.data, w_rows=N, w_cols=K, x=x.ctypes.data, M=M, N=N, K=K, pro=capi.PRO["rms"],
                        epi=capi.EPI["store"], y=y.ctypes.data, stat=st.ctypes.data, stat_off=1, stat_ld=2,
                        norm=nw.ctypes.data)
    assert O.q4_gemvM(a) == 1
    for m in range(M):
        xp = (x[m * K:(m + 1) * K] * st[1 + 2 * m]).astype(np.float32) * nw
        assert rel_l2(y[m * N:(m + 1) * N], deq @ xp.astype(np.float64)) < 1e-6


# ------------------------------------------------------------------------------------------------ GEMM
def test_gemm_vs_numpy_fp16_operands():
    M, N, K = 40, 128, 256
    b, deq = _weights(N, K, 11)
    X = O.randn(M * K, 7).reshape(M, K)
    x16 = X.astype(np.float16)
    y = np.zeros(M * N, np.float32)
    a = capi.gemm_args(w=b.ctypes.data, w_rows=N, w_cols=K, x=x16.ctypes.data, x_mode=capi.XMODE["f16"], M=M, N=N,
                       K=K, epi=capi.GEPI["f32"], y=y.ctypes.data)
    O.q4_gemm(a)
    want = x16.astype(np.float64) @ deq.astype(np.float32).astype(np.float16).astype(np.float64).T
    assert rel_l2(y, want) < 1e-6
    # the kcheck.js:72-88 criterion against the unrounded product
    assert cos_sim(y, X.astype(np.float64) @ deq.T) > 0.9995


def test_gemm_swiglu_interleave():
    M, N2, K = 8, 128, 128           # N2 ws columns = 64 gate + 64 up rows, interleaved
    b, deq = _weights(128, K, 13)
    X = O.randn(M * K, 17).reshape(M, K).astype(np.float16)
    y = np.zeros(M * N2 // 2, np.float16)
    a = capi.gemm_args(w=b.ctypes.data, w_rows=128, w_cols=K, x=X.ctypes.data, M=M, N=N2, K=K, wr0=0, wr1=64,
                       epi=capi.GEPI["swiglu"], y=y.ctypes.data, y_ld=64)
    O.q4_gemm(a)
    d16 = deq.astype(np.float32).astype(np.float16).astype(np.float64)
    acc = X.astype(np.float64) @ d16.T
    g, u = acc[:, :64].astype(np.float32).astype(np.float64), acc[:, 64:].astype(np.float32).astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    assert rel_l2(y.astype(np.float64), want) < 2e-3     # fp16 output


def test_lgemv_f32_cpu_baseline_matches_kcheck_criterion():
    """engine/kcheck.js:126-135: gemv N=256, K=1536, seeds 31 (x) / 32 (W x0.05), cos > 0.9999 vs the deq product"""
    N, K = 256, 1536
    x = O.randn(K, 31)
    b, deq = O.pack_q4(O.randn(N * K, 32, 0.05), N, K)
    y = O.lgemv_f32(b, x, N, K, threads=2)
    want = deq.astype(np.float64) @ x.astype(np.float64)
    assert cos_sim(y, want) > 0.9999
    assert rel_l2(y, want) < 1e-5


def test_gemm_f32_cpu_baseline():
    M, N, K = 16, 64, 256
    b, deq = _weights(N, K, 3)
    x16 = O.randn(M * K, 5).astype(np.float16)
    y = O.gemm_f32(b, x16.view(np.uint16), M, N, K, threads=2)
    want = x16.reshape(M, K).astype(np.float64) @ deq.astype(np.float32).astype(np.float16).astype(np.float64).T
    assert rel_l2(y, want) < 1e-5
