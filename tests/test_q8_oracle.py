"""CPU pins of the q8g64s.t64 oracle (packQ8, engine/kcheck.js:39-52; the record reader, engine/llm/lops.js:74-80):
an independent numpy decode of the record bytes (row r's 64 int8 codes at 64 r, the fp16 scale at 4096 + 2 r), the
quantiser's rules (s = fl16(absmax / 127), 1 when the group is zero; q = clamp(round-half-even(w / s), -128, 127)),
and the oracle's q8 GEMV against a float64 numpy matmul of the decoded weights."""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi


def np_decode_q8(b, N, K):
    rec = b.reshape(N // 64, K // 64, 4224)
    codes = rec[:, :, :4096].reshape(N // 64, K // 64, 64, 64).view(np.int8).astype(np.float32)
    s = rec[:, :, 4096:].copy().view(np.float16).astype(np.float32)          # [tile][group][64 rows]
    w = codes * s[:, :, :, None]                                               # [tile][group][row][k]
    return w.transpose(0, 2, 1, 3).reshape(N, K)


def test_pack_q8_rules_and_layout():
    N, K = 128, 256
    W = O.randn(N * K, 7, 0.05).reshape(N, K)
    W[3, 64:128] = 0.0                                       # a zero group: scale 1, codes 0
    b, deq = O.pack_q8(W, N, K)
    dec = np_decode_q8(b, N, K)
    assert np.array_equal(dec.ravel(), deq)                 # the byte layout decodes to packQ8's own dequant
    assert np.array_equal(O.dequant_q8(b, N, K), deq)       # the oracle's record reader agrees
    rec = b.reshape(N // 64, K // 64, 4224)
    s = rec[:, :, 4096:].copy().view(np.float16).astype(np.float64)
    for n in range(N):
        for g in range(K // 64):
            grp = W[n, 64 * g:64 * g + 64].astype(np.float64)
            am = np.abs(grp).max()
            want_s = np.float16(np.float32(am / 127)) if am > 0 else np.float16(1.0)
            got_s = s[n // 64, g, n % 64]
            assert got_s == np.float64(want_s)
            q = dec[n, 64 * g:64 * g + 64] / got_s
            assert np.all(np.abs(q) <= 128) and np.array_equal(q, np.round(q))
            assert np.all(np.abs(dec[n, 64 * g:64 * g + 64] - grp) <= got_s / 2 + 1e-7)
    assert np.all(dec[3, 64:128] == 0.0) and s[0, 1, 3] == 1.0


@pytest.mark.parametrize("pro", ["raw", "rms"])
def test_q8_gemv_oracle_vs_numpy(pro):
    N, K = 128, 512
    W = O.randn(N * K, 9, 0.05)
    b, deq = O.pack_q8(W, N, K)
    x = O.randn(K, 10)
    nw = np.linspace(0.8, 1.2, K).astype(np.float32)
    st = np.array([0.0, 0.8], np.float32)
    y = np.full(N, np.nan, np.float32)
    O.q4_gemv(capi.gemv_args(w=b.ctypes.data, w_enc=2, w_rows=N, w_cols=K, x=x.ctypes.data, N=N, K=K,
                             pro=capi.PRO[pro], y=y.ctypes.data, stat=st.ctypes.data, stat_off=1, norm=nw.ctypes.data))
    # the prologue in fp32, as the reference computes it (engine/llm/lops.js:52)
    xp = (x if pro == "raw" else (x * np.float32(0.8) * nw).astype(np.float32)).astype(np.float64)
    want = np_decode_q8(b, N, K).astype(np.float64) @ xp
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))
