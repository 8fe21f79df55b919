"""GPU parity of the q8g64s.t64 GEMV (p0pc0rn_amd/csrc/gemv_q8.hip) through the C ABI.

Every q8 shape the reference ships (engine/tune/kshipped.js:14, run as kshipped.js:17-41 runs it: 128 rows at the real
K, its kPer rule, seeds 33 + K / 34 + K / 35 + K) under the reference's own acceptance (cos > 0.99999, the tile argmax)
and this build's bars (relative L2 <= 1e-3 and <= 2e-5), the expected rows in float64 from numpy over the decoded
records (tests/test_q8_oracle.py pins the packer and the decode); gemvM with M rows against the oracle; q8 ops inside
pipelined chains of M = 1 (decode) and M = 3, 5, 8 (verify) rows, mixed with q4 ops, against the oracle; and a chain
holding a q8 op is refused where only the general chain kernel would run it."""
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



@pytest.mark.parametrize("slices", [1, 2, 5, 24])
@pytest.mark.parametrize("pro,epi,K,kPer", [("rms", "geglu", 1536, 0), ("raw", "store", 6144, 2048),
                                            ("raw", "store", 5120, 2048)])
def test_q8_k_slices_across_workgroups(dev, slices, pro, epi, K, kPer):
    """the 16-wave q8 GEMV with each split's K cut into slices across workgroups (p0_gemv_tune knob 5: one workgroup
    per split, two, five uneven slices, two groups a slice), the last arriving workgroup adding the slices' partials
    through the uncached workspace: the same checks as the shipped shapes. K = 5120 in splits of 2048 leaves a last
    split of 16 groups, whose trailing slices hold no group (they add zeros and still count their arrival)"""
    old = capi.gemv_tune(5, slices)
    try:
        test_q8_kshipped_shapes(dev, pro, epi, K, kPer)
    finally:
        capi.gemv_tune(5, old if old > 0 else -1)


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


def _q8(rows, K, seed):
    return O.pack_q8(O.randn(rows * K, seed, 0.05), rows, K)[0]


def _q4(rows, K, seed):
    return O.pack_q4(O.randn(rows * K, seed, 0.05), rows, K)[0]


def test_q8_ops_in_a_pipelined_chain(dev):
    """A decode-like chain of q4g32a.t64 and q8g64s.t64 ops (the real E2B pack is balanced 4/8-bit) as one pipelined
    launch: q8 ops with every prologue the chain sees (rms, raw through a mailbox, raw with 2 K-splits), a geglu, a
    softcap and a large share per workgroup (one wave per unit). Each op is checked against the oracle run on the input
    it read on the GPU (the previous op's output, read back), to this build's fp32 bar; every intermediate is NaN-filled
    before the run. Two more runs reproduce the bits."""
    D = 256
    x0 = O.randn(2048, 501)
    nw = nw_of(2048)
    st = np.array([0, 0.7, 0, 0], np.float32)
    ops = [   # (name, enc, w rows, N, K, kPer, pro, epi, input, input offset)
        ("a", "q4", 512, 512, D, 0, "rms", "store", "x", 0),
        ("b", "q8", D, D, 512, 0, "raw", "store", "a", 0),          # mailbox from a q4 op into a q8 op
        ("c", "q8", 768, 384, D, 0, "rms", "geglu", "b", 0),      # mailbox into an rms q8 op
        ("d", "q4", D, D, 384, 0, "rms", "store", "c", 0),        # the geglu output's mailbox into a q4 op
        ("e", "q8", D, D, D, 128, "raw", "store", "d", 0),         # mailbox into a 2-split q8 op
        ("f", "q8", 32768, 32768, 2048, 0, "rms", "store", "x", 0),  # 8 units x 4 slots per workgroup: per-wave mode
        ("g", "q8", 4096, 4096, D, 0, "rms", "softcap", "x", 0),
    ]
    host = {n: (_q8 if enc == "q8" else _q4)(rows, K, 510 + i)
            for i, (n, enc, rows, N, K, kPer, pro, epi, src, off) in enumerate(ops)}
    dw = {n: capi.to_device(w) for n, w in host.items()}
    x, nwb, stb = capi.to_device(x0), capi.to_device(nw), capi.to_device(st)
    nsplit = {n: (-(-K // kPer) if kPer else 1) for (n, enc, rows, N, K, kPer, pro, epi, src, off) in ops}
    out = {n: capi.Buffer(4 * N * nsplit[n]) for (n, enc, rows, N, K, kPer, pro, epi, src, off) in ops}
    NTg = 4096 // 64
    mx0 = np.zeros(NTg * 2 + 8, np.float32)
    mx0[NTg * 2 + 1] = 0.9
    mx = capi.to_device(mx0)
    bufs = dict(out, x=x)

    def fields(n, enc, rows, N, K, kPer, pro, epi, src, off, b):
        f = dict(w=b["w"][n], w_enc=1 if enc == "q4" else 2, w_rows=rows, w_cols=K, x=b[src], x_rowB=off, N=N, K=K,
                 kPer=kPer, pro=capi.PRO[pro], epi=capi.EPI[epi], y=b[n])
        if pro == "rms":
            f.update(norm=b["nw"], stat=b["st"], stat_off=1)
        if epi == "softcap":
            f.update(mx=b["mx"], stat=b["mx"], stat_off=NTg * 2 + 1)
        return f

    dev_b = dict(bufs, w=dw, nw=nwb, st=stb, mx=mx)

    def enqueue():
        for o in ops:
            capi.q4_gemv(capi.gemv_args(**fields(*o, dev_b)))

    ch = capi.chain(enqueue)
    info = ch.info()
    print("mixed chain", info, flush=True)
    if info["waves_per_workgroup"] != 12:
        pytest.skip("this device plans the general chain kernel")
    # b, c, d and e take their x from the previous op's mailbox (raw or rms prologue, x inside one split of that op's
    # store or geglu output); f and g read the chain input x
    assert info["mailboxes"] == 4
    runs = []
    for r in range(3):
        for n in out:
            out[n].fill_u32(0x7FC00000)
        mx.upload(mx0)
        ch.run()
        assert not ch.status()
        runs.append({n: out[n].read(np.float32) for n in out} | {"mx": mx.read(np.float32)})
    for r in runs[1:]:
        for k in r:
            assert np.array_equal(runs[0][k].view(np.uint32), r[k].view(np.uint32)), k
    got = runs[0]
    mxh = mx0.copy()
    for o in ops:
        n, enc, rows, N, K, kPer, pro, epi, src, off = o
        xin = np.ascontiguousarray(x0 if src == "x" else got[src], np.float32)
        y = np.full(N * nsplit[n], np.nan, np.float32)
        f = fields(n, enc, rows, N, K, kPer, pro, epi, "x", off,
                   dict(w={n: host[n].ctypes.data}, x=xin.ctypes.data, nw=nw.ctypes.data, st=st.ctypes.data,
                        mx=mxh.ctypes.data, **{n: y.ctypes.data}))
        O.q4_gemv(capi.gemv_args(**f))
        r = rel_l2(got[n], y)
        print(f"op {n} ({enc} {pro}.{epi} {N}x{K} kPer {kPer}): rel_l2 {r:.3e}", flush=True)
        assert np.all(np.isfinite(got[n])) and r <= 2e-5, n
    gm, om = got["mx"][:2 * NTg:2], mxh[:2 * NTg:2]
    assert np.allclose(gm, om, rtol=1e-5, atol=1e-5)
    assert np.mean(got["mx"][1:2 * NTg:2].view(np.uint32) == mxh[1:2 * NTg:2].view(np.uint32)) > 0.99
    ch.free()
    for v in list(dw.values()) + [x, nwb, stb, mx] + list(out.values()):
        v.free()


@pytest.mark.parametrize("M", [3, 5, 8])
def test_q8_ops_in_a_verify_chain(dev, M):
    """A verify-pass chain (gemvM, M rows) mixing q4g32a.t64 and q8g64s.t64 ops as the real E2B pack does
    (p0pc0rn.config.json:207, its q8 shapes at engine/tune/tunecore.js:17-21): q8 ops with raw and rms prologues, a q8
    geglu, a q8 op reading one K-split of a q4 op, a large q8 softcap share (one wave per unit) and argmaxM after it;
    M = 3 and 5 as one pipelined launch, M = 8 as pipelined row-group passes. Each op against the oracle on the input it
    read on the GPU, every intermediate NaN-filled before the run."""
    ops = [   # (name, enc, w rows, N, K, kPer, pro, epi, input, x row stride)
        ("a", "q4", 768, 768, 512, 0, "rms", "store", "x", 512),
        ("b", "q8", 512, 512, 512, 0, "raw", "store", "a", 768),      # the first 512 of a's 768 outputs per row
        ("c", "q8", 2048, 1024, 512, 0, "rms", "geglu", "b", 512),
        ("d", "q4", 512, 512, 1024, 512, "raw", "store", "c", 1024),  # 2 K-splits
        ("e", "q8", 512, 512, 512, 0, "rms", "store", "d", 512),      # d's first split
        ("f", "q8", 32768, 32768, 512, 0, "rms", "softcap", "e", 512),
    ]
    host = {n: (_q8 if enc == "q8" else _q4)(rows, K, 610 + i)
            for i, (n, enc, rows, N, K, kPer, pro, epi, src, ld) in enumerate(ops)}
    x0 = O.randn(M * 512, 620)
    nw = nw_of(1024)
    st = np.zeros(2 * M, np.float32)
    st[1::2] = 0.8
    NT = 32768 // 64
    mx0 = np.zeros(M * NT * 2 + 2 * M, np.float32)
    mx0[M * NT * 2 + 1::2] = 0.9
    nsplit = {o[0]: (-(-o[4] // o[5]) if o[5] else 1) for o in ops}
    olen = {o[0]: M * o[3] * (nsplit[o[0]] if o[7] == "store" else 1) for o in ops}
    dw = {n: capi.to_device(w) for n, w in host.items()}
    d = {"x": capi.to_device(x0), "nw": capi.to_device(nw), "st": capi.to_device(st), "mx": capi.to_device(mx0),
         "arg": capi.Buffer(8 * M)}
    out = {n: capi.Buffer(4 * olen[n]) for n in olen}

    def fields(o, b, w):
        n, enc, rows, N, K, kPer, pro, epi, src, ld = o
        f = dict(w=w[n], w_enc=1 if enc == "q4" else 2, w_rows=rows, w_cols=K, x=b[src], x_ldx=ld, M=M, N=N, K=K,
                 kPer=kPer, pro=capi.PRO[pro], epi=capi.EPI[epi], y=b[n], y_ldm=N, y_ldy=M * N, norm=b["nw"],
                 stat=b["st"], stat_off=1, stat_ld=2)
        if epi == "softcap":
            f.update(mx=b["mx"], stat=b["mx"], stat_off=M * NT * 2 + 1, cap=30.0)
        return f

    def token():
        for o in ops:
            capi.q4_gemvM(capi.gemvm_args(**fields(o, {**d, **out}, dw)))
        capi.argmaxM(d["mx"], NT, M, d["arg"])

    ch = capi.chain(token)
    info = ch.info()
    print("mixed q4 / q8 verify chain", info, flush=True)
    assert info["workgroups"] == capi.device_info()["cu_count"] and info["passes"] == (1 if M <= 5 else 2)
    for b in out.values():
        b.fill_u32(0x7FC00000)
    d["arg"].fill_u32(0x7FC00000)
    ch.run()
    assert not ch.status()
    got = {n: out[n].read(np.float32) for n in out}
    gmx = d["mx"].read(np.float32)
    mxh = mx0.copy()
    for o in ops:
        n, src = o[0], o[8]
        xin = np.ascontiguousarray(x0 if src == "x" else got[src], np.float32)
        y = np.full(olen[n], np.nan, np.float32)
        hb = {"x": xin.ctypes.data, src: xin.ctypes.data, n: y.ctypes.data, "nw": nw.ctypes.data,
              "st": st.ctypes.data, "mx": mxh.ctypes.data}
        O.q4_gemvM(capi.gemvm_args(**fields(o, hb, {n: host[n].ctypes.data})))
        r = rel_l2(got[n], y)
        print(f"M={M} op {n} ({o[1]} {o[6]}.{o[7]} {o[3]}x{o[4]}): rel_l2 {r:.3e}", flush=True)
        assert np.all(np.isfinite(got[n])) and r <= 2e-5, n
    assert np.allclose(gmx[:2 * M * NT:2], mxh[:2 * M * NT:2], rtol=1e-5, atol=1e-5)
    want = np.asarray(O.argmaxM(gmx, NT, M), np.uint32).ravel()
    assert np.array_equal(d["arg"].read(np.uint32), want)
    ch.free()
    for v in list(dw.values()) + list(d.values()) + list(out.values()):
        v.free()


def test_q8_ops_join_only_pipelined_chains(dev):
    """q8 ops need the pipelined kernel: with it switched off (p0_chain_tune knob 4) a chain holding one is refused at
    p0_chain_end"""
    N, K, M = 128, 256, 2
    wb, xb, yb = capi.to_device(_q8(N, K, 5)), capi.Buffer(M * K * 4), capi.Buffer(M * N * 4)
    old = capi.chain_tune(4, 0)
    try:
        with pytest.raises(capi.P0Error, match="q8g64s.t64 ops join only pipelined chains"):
            capi.chain(lambda: capi.q4_gemvM(capi.gemvm_args(w=wb, w_enc=2, w_rows=N, w_cols=K, x=xb, M=M, N=N, K=K,
                                                             y=yb)))
    finally:
        capi.chain_tune(4, old)
    for v in (wb, xb, yb):
        v.free()
