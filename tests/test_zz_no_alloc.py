"""p0_q4_gemm_noalloc, the GEMM entry point that allocates nothing, against p0_q4_gemm through the C ABI.

The staging the no-allocation call needs (bf16 / lnmod / rms / unaligned fp16 activations -> fp16 rows) goes to the
library's static device scratch instead of the context's growable workspace; the kernels are the same, so its outputs
must be bit-identical to p0_q4_gemm's. Two calls in a row, the second smaller (the scratch keeps the first call's
contents, which the second must not depend on), in a staged mode and with the heads epilogue; a size past the scratch
is refused with an error before anything runs.
"""
import numpy as np
import pytest

from oracle import oracle as O
from p0pc0rn_amd import capi

pytestmark = pytest.mark.gpu
SCRATCH = 32 << 20


def _pair(fields, arrays, out_bytes, tail=0):
    """the same call through both entry points -> (gemm output bytes, noalloc output bytes, noalloc flops); Y is
    allocated with `tail` more bytes after the output, which neither call may write"""
    d = {k: capi.to_device(v) for k, v in arrays.items()}
    ya = capi.Buffer(out_bytes + tail).fill_u32(0x7FC00000)
    yb = capi.Buffer(out_bytes + tail).fill_u32(0x7FC00000)
    capi.q4_gemm(capi.gemm_args(**fields, **d, y=ya))
    fl = capi.q4_gemm_noalloc(capi.gemm_args(**fields, **d, y=yb))
    a, b = ya.read(np.uint8), yb.read(np.uint8)
    for buf in list(d.values()) + [ya, yb]:
        buf.free()
    for out in (a, b):
        assert np.all(out[out_bytes:].view(np.uint32) == 0x7FC00000), "written past the output"
    return a[:out_bytes], b[:out_bytes], fl


def test_noalloc_matches_gemm_two_calls_second_smaller(dev):
    for M, N, K, seed in ((1536, 1024, 3072, 1), (200, 256, 512, 2)):   # 9.4 MB of staging, then 0.2 MB
        print("case bf16", M, N, K, flush=True)
        w = O.pack_q4(O.randn(N * K, seed, 0.05), N, K)[0]
        xf = np.random.default_rng(seed).standard_normal(M * K, dtype=np.float32)
        xb = (xf.view(np.uint32) >> 16).astype(np.uint16)
        f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE["bf16"], epi=capi.GEPI["f32"])
        a, b, fl = _pair(f, dict(w=w, x=xb), M * N * 4)
        assert fl == 2.0 * M * N * K
        assert np.all(np.isfinite(b.view(np.float32)))
        assert np.array_equal(a, b), "noalloc output differs from p0_q4_gemm's"


def test_noalloc_lnmod_heads_two_calls(dev):
    """the FLUX qkv call shape (lnmod prologue, heads epilogue), twice, the second smaller"""
    for M, H, K, seed in ((768, 6, 1024, 3), (130, 3, 256, 4)):
        print("case lnmod+heads", M, H, K, flush=True)
        N = H * 128
        w = O.pack_q4(O.randn(N * K, seed, 0.05), N, K)[0]
        x = (1.0 + O.randn(M * K, seed + 10)).astype(np.float32)
        xr = x.reshape(M, K).astype(np.float64)
        st = np.zeros(2 * M, np.float32)
        st[0::2], st[1::2] = xr.mean(1), 1 / np.sqrt(xr.var(1) + 1e-6)
        pv = O.randn(3 * K, seed + 20, 0.2)
        ev = (1 + 0.2 * O.randn(256, seed + 30)).astype(np.float32)
        rope = np.random.default_rng(seed).uniform(-1, 1, (M, 128)).astype(np.float32)
        f = dict(w_rows=N, w_cols=K, M=M, N=N, K=K, x_mode=capi.XMODE["lnmod"], pv_off=K, pv_stride=(1 << 32) - K,
                 epi=capi.GEPI["heads"], heads_ltot=M, heads_hq=H // 3, heads_hkv=H // 3, heads_rope=0)
        a, b, _ = _pair(f, dict(w=w, x=x, stats=st, pv=pv, ev=ev, rope=rope), N * M * 2, tail=M * 128 * 2)
        assert np.all(np.isfinite(b.view(np.float16).astype(np.float32)))
        assert np.array_equal(a, b), "noalloc heads output differs from p0_q4_gemm's"


def test_noalloc_refuses_more_than_its_scratch(dev):
    """M K fp16 values past the scratch: an error, nothing launched (no buffer is read or written)"""
    M, K = SCRATCH // (2 * 1024) + 64, 1024
    a = capi.gemm_args(w=16, w_rows=64, w_cols=K, x=16, x_mode=capi.XMODE["bf16"], M=M, N=64, K=K,
                       epi=capi.GEPI["f32"], y=16)
    fl = capi.C.c_double()
    assert capi.lib().p0_q4_gemm_noalloc(capi.C.byref(a), capi.C.byref(fl)) == capi.P0_EINVAL
    assert capi.last_error().startswith("gemm_noalloc: the activations need")
