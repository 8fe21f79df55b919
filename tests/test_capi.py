"""The C-ABI boundary on the CPU: the library loads, exports every symbol include/p0pc0rn.h declares, and rejects bad
arguments with the reference's own error text before touching a device (engine/llm/lops.js:114-124,
engine/llm/lops_spec.js:166-173, engine/ops/gemm.js:266-278)."""
import os
import re
import subprocess

import numpy as np
import pytest

from p0pc0rn_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "p0pc0rn.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(p0_[a-zA-Z0-9_]+)\s*\(", src)))


def test_library_exports_every_header_symbol():
    names = header_functions()
    assert len(names) >= 20
    assert sorted(capi.HEADER_SYMBOLS) == names
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (p0_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(capi.lib(), n)


def test_library_is_built_for_gfx950_only():
    blob = open(capi.LIB_PATH, "rb").read()   # the embedded code-object bundle names its targets
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"--gfx942", b"--gfx90a", b"--gfx1100"):
        assert other not in blob


def _err(fn, args):
    rc = fn(args)
    return rc


def gemv_err(**kw):
    base = dict(w=16, w_rows=64, w_cols=64, x=16, N=64, K=64, y=16)
    base.update(kw)
    a = capi.gemv_args(**base)
    n = capi.i32()
    rc = capi.lib().p0_q4_gemv(capi.C.byref(a), capi.C.byref(n))
    return rc, capi.last_error()


@pytest.mark.parametrize("kw,msg", [
    (dict(N=100), "gemv: N % 64"),
    (dict(K=5000, w_cols=5000), "gemv: K 5000 needs a kPer"),
    (dict(K=4096, w_cols=4096, kPer=100), "gemv: kPer must be a multiple of 32"),
    (dict(K=4096, w_cols=4096, kPer=2048, epi=1), "gemv: geglu needs one split"),
    (dict(K=4096, w_cols=4096, kPer=2048, epi=2, mx=16), "gemv: softcap needs one split"),
    (dict(w_off=2), "gemv: weight offset"),
    (dict(w_enc=2, K=4096, w_cols=4096, kPer=2016), "gemv: kPer must be a multiple of 64"),   # q8: groups of 64
    (dict(w_enc=2, K=96, w_cols=96), "gemv: kPer must be a multiple of 64"),
    (dict(w_enc=7), "gemv: encoding 7"),
    (dict(K=48, w_cols=48), "gemv: kPer must be a multiple of 32"),
    (dict(N=128), "gemv: weight has 64 rows < N 128"),
    (dict(epi=1), "gemv: weight has 64 rows < 2N 128"),
])
def test_gemv_argument_errors(kw, msg):
    rc, err = gemv_err(**kw)
    assert rc == capi.P0_EINVAL
    assert err == msg


def _device_open():
    d = capi.DeviceInfo()
    return capi.lib().p0_device_info(capi.C.byref(d)) == capi.P0_OK


def test_gemv_kper_defaults_follow_the_reference():
    # K in (2048, 3072] without a kPer is ONE split (engine/llm/lops.js:116-117); validation passes, then needs a device.
    # The call's buffers are fake addresses: with a device open it would launch on them, so it runs without one only.
    if _device_open():
        pytest.skip("a device context is open in this process: the fake buffers must not reach a kernel")
    rc, err = gemv_err(K=2560, w_cols=2560)
    assert rc == capi.P0_ENODEV and "no device" in err


def gemvm_err(**kw):
    base = dict(w=16, w_rows=64, w_cols=64, x=16, M=2, N=64, K=64, y=16)
    base.update(kw)
    a = capi.gemvm_args(**base)
    n = capi.i32()
    rc = capi.lib().p0_q4_gemvM(capi.C.byref(a), capi.C.byref(n))
    return rc, capi.last_error()


@pytest.mark.parametrize("kw,msg", [
    (dict(N=96), "gemvM: N % 64"),
    (dict(pro=2), "gemvM: prologue sum"),
    (dict(K=4096, w_cols=4096, kPer=48), "gemvM: kPer must be a multiple of 32"),
    (dict(K=4096, w_cols=4096, kPer=1024, epi=1), "gemvM: geglu needs one split"),
    (dict(w_off=6), "gemvM: weight offset"),
    (dict(M=17), "gemvM: M 17 (this build: 1..16)"),
    (dict(N=128), "gemvM: weight has 64 rows < N 128"),
    (dict(epi=1), "gemvM: weight has 64 rows < 2N 128"),
])
def test_gemvM_argument_errors(kw, msg):
    rc, err = gemvm_err(**kw)
    assert rc == capi.P0_EINVAL
    assert err == msg


def test_gemvM_kper_caps_at_2048():
    # kPer above 2048 is capped at KCH (engine/llm/lops_spec.js:170): 4096 / 2048 = 2 splits -> geglu refused
    rc, err = gemvm_err(K=4096, w_cols=4096, kPer=4096, epi=1)
    assert err == "gemvM: geglu needs one split"


def gemm_err(**kw):
    base = dict(w=16, w_rows=64, w_cols=64, x=16, M=4, N=64, K=64, y=16)
    base.update(kw)
    a = capi.gemm_args(**base)
    fl = capi.C.c_double()
    rc = capi.lib().p0_q4_gemm(capi.C.byref(a), capi.C.byref(fl))
    return rc, capi.last_error()


@pytest.mark.parametrize("kw,msg", [
    (dict(K=40), "gemm: K must be a multiple of 32"),
    (dict(w_enc=9), "gemm: unsupported weight encoding 9"),
    (dict(epi=3, N=63), "gemm: swiglu needs an even N"),
    (dict(x_mode=1), "gemm: lnmod needs stats and pv"),
    (dict(epi=4), "gemm: bias needs ev"),
    (dict(N=128), "gemm: weight rows 0 + 128 past the 64 rows of the weight"),
    (dict(wr0=32), "gemm: weight rows 32 + 64 past the 64 rows of the weight"),
    (dict(wr0=-64), "gemm: negative weight row"),
    (dict(w_rows=128, epi=3, N=128, wr0=0, wr1=96), "gemm: weight rows 96 + 64 past the 128 rows of the weight"),
    (dict(w_rows=128, epi=3, N=128, wr0=96, wr1=0), "gemm: weight rows 96 + 64 past the 128 rows of the weight"),
    (dict(w_rows=128, N=128, epi=5), "gemm: heads needs ev (the norm weights) and heads.rope"),
    (dict(w_rows=192, epi=5, N=192, ev=16, rope=16), "gemm: heads needs N a multiple of 128"),
    (dict(w_rows=128, epi=5, N=128, ev=16, rope=16, heads_ltot=3), "gemm: heads rows 0 + 4 past Ltot 3"),
    (dict(w_rows=128, epi=5, N=128, ev=16, rope=16, heads_ltot=8, heads_row_off=5),
     "gemm: heads rows 5 + 4 past Ltot 8"),
    (dict(w_rows=128, epi=5, N=128, ev=16, rope=16, heads_ltot=8, heads_rope=2), "gemm: heads rope mode 2"),
    (dict(epi=6), "gemm: epilogue 6"),
])
def test_gemm_argument_errors(kw, msg):
    rc, err = gemm_err(**kw)
    assert rc == capi.P0_EINVAL
    assert err == msg


def test_ops_without_a_device_fail_loudly():
    if _device_open():
        pytest.skip("a device context is open in this process")
    rc, err = gemv_err()
    assert rc == capi.P0_ENODEV and "no device" in err
    p = capi.vp()
    assert capi.lib().p0_buffer(64, capi.C.byref(p)) == capi.P0_ENODEV
    assert capi.lib().p0_copy(None, 0, None, 0, 16) == capi.P0_ENODEV
    assert capi.lib().p0_chain_begin() == capi.P0_ENODEV


def test_chain_tune_knobs_round_trip():
    """chain knobs answer queries without a device and clamp the waves knob to 8 or 16"""
    old = capi.chain_tune(0, 0)
    assert old in (8, 16)
    assert capi.chain_tune(0, 9) == old and capi.chain_tune(0, -1) == 8
    assert capi.chain_tune(0, 16) == 8 and capi.chain_tune(0, -1) == 16
    capi.chain_tune(0, old)
    assert capi.chain_tune(9, -1) == 3 and capi.chain_tune(9, 6) == 3 and capi.chain_tune(9, -1) == 6
    capi.chain_tune(9, 3)
    assert capi.chain_tune(3, -1) == 0 and capi.chain_tune(15, 1) == -1
    assert capi.chain_tune(12, -1) == 1 and capi.chain_tune(12, 0) == 1 and capi.chain_tune(12, 1) == 0
    assert capi.chain_tune(13, -1) == 2 and capi.chain_tune(13, 1) == 2 and capi.chain_tune(13, 2) == 1
    assert capi.chain_tune(14, -1) == 1 and capi.chain_tune(14, 0) == 1 and capi.chain_tune(14, 1) == 0
    assert capi.chain_tune(10, -1) == 1 and capi.chain_tune(10, 0) == 1 and capi.chain_tune(10, -1) == 0
    assert capi.chain_tune(10, 1) == 0 and capi.chain_tune(10, -1) == 1
    assert capi.chain_tune(4, -1) == 1 and capi.chain_tune(4, 0) == 1 and capi.chain_tune(4, -1) == 0
    assert capi.chain_tune(4, 1) == 0 and capi.chain_tune(4, -1) == 1
    assert capi.chain_tune(5, -1) == 2 and capi.chain_tune(5, 9) == 2 and capi.chain_tune(5, 2) == 4
    assert capi.chain_tune(6, -1) == 2 and capi.chain_tune(6, 1) == 2 and capi.chain_tune(6, 2) == 1
    assert capi.chain_tune(11, -1) == 1 and capi.chain_tune(11, 2) == 1 and capi.chain_tune(11, 1) == 2
    assert capi.chain_tune(7, -1) == 1 and capi.chain_tune(7, 0) == 1 and capi.chain_tune(7, -1) == 0
    assert capi.chain_tune(7, 1) == 0 and capi.chain_tune(7, -1) == 1
    assert capi.chain_tune(8, -1) == 1 and capi.chain_tune(8, 0) == 1 and capi.chain_tune(8, -1) == 0
    assert capi.chain_tune(8, 1) == 0 and capi.chain_tune(8, -1) == 1


def test_gemv_tune_q8_slices_knob():
    """knob 5 (q8 K-slices) answers without a device: 0 = planned, a positive count sets it, a negative value restores
    the plan; knob 6 does not exist"""
    old = capi.gemv_tune(5)
    assert old >= 0
    assert capi.gemv_tune(5, 3) == old and capi.gemv_tune(5) == 3
    assert capi.gemv_tune(5, -1) == 3 and capi.gemv_tune(5) == 0
    if old > 0:
        capi.gemv_tune(5, old)
    assert capi.gemv_tune(6, 1) == -1
