#!/usr/bin/env python3
"""Benchmark of the q4g32a.t64 matmul hot path on one MI355X (BASELINE.json's metric and configs).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemm] [--json-only]

Headline (`value`): tokens/s of the Gemma-4-E2B-shaped decode token at M=1 (config B): 30 layers x {qkv 3072x2048
rms, o 2048x2048 raw kPer 2048, gate_up 2x8192x2048 rms+geglu, down 2048x8192 raw kPer 2048} + the token's tail as
engine/llm/gemma4.js:503-511 and engine/llm/drunner.js:82-90 run it: the rstd copy into the head's stat slot, the
lm_head 262144x2048 rms+softcap (tile max/argmax), the argmax over the 4096 tile maxima and the copy of the result
words into the staging buffer = 121 GEMV ops + 3 others. Run per token both ways the library offers (the
DecodeRunner analogue): planned once into a chain that runs as ONE persistent launch, and recorded as a graph of 124
launches; the faster is the headline and both are reported (also the 121 GEMVs alone).
Attention, norms and the PLE projections are not part of the step (config B counts the linears only).

Also reported: the step's weight-streaming GB/s, config A (one 8192x2048 GEMV, weight ring of 32 copies), the
verify pass at M = 5 and the M sweep {1, 2, 4, 8, 16} (config C), and the FLUX.2-klein (M=4608, config D) and
SANA-Video (M=32760, config E) dequant-GEMM TFLOP/s. All weights are synthetic symmetric int4 (codes uniform,
scale |N(0, 0.02)| fp16, min = -8 scale) filled on the device; activations fp16-valued N(0, 1). The decode and verify
layers take weight scales that keep each op's output at its input's magnitude, and each timed path runs on rstd slots
calibrated from its own activations (Step.calibrate), so every layer computes on O(1) values.

Timing: HIP events on the library's stream around back-to-back replays, inputs already resident in HBM.
CPU baseline: the oracle's fp32 port of the reference's lgemv kernel (engine/llm/lops.js:60-88) on the host cores,
over a bounded sample of the same step (one layer + 1/16 of the head), scaled to tokens/s.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0     # MI355X dense fp16 MFMA
Q4_BYTES_PER_W = 0.625        # 1280 B per 64 rows x 32 k (engine/kcheck.js:23)

D, LAYERS, QKV, MLP, VOCAB = 2048, 30, 3072, 8192, 262144


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Step:
    """The decode step's weights and buffers (device), and its op sequence for M rows."""

    def __init__(self, capi, seed=0, baseline_scales=False):
        self.c = capi
        c = capi
        self.layers = []
        # Bounded activations. The weight scales keep each op's output at its input's magnitude (codes q - 8 have mean
        # square 21.5; the down projection makes up for the geglu's ~0.65), and the norm weights alternate in sign, so
        # that the codes' mean of -0.5 s does not pile up a common-mode component op after op. The rstd slots are
        # inputs of the step (the model's RMSNorm sits outside it); calibrate() sets them before each timed path from
        # that path's own activations, as the norm would, so every layer and the head compute on O(1) values (with
        # fixed slots the geglu's square makes the magnitude collapse towards 0 within a few layers, and the later
        # layers would compute on zeros). An M > 1 verify pass keeps its matrix-core path (it falls back to the VALU
        # for |x'| >= 255) and every path runs what a model's step runs.
        # baseline_scales: BASELINE's |N(0, 0.02)| scales for every layer instead (the activations then grow ~4x per op,
        # and x' leaves the range of the matrix cores' fixed 2^8 staging from the second layer on)
        sigma = {"qkv": 1 / np.sqrt(21.5 * D), "o": 1 / np.sqrt(21.5 * D), "gu": 1 / np.sqrt(21.5 * D),
                 "down": 1.55 / np.sqrt(21.5 * MLP)}
        if baseline_scales:
            sigma = {k: 0.02 for k in sigma}
        for l in range(LAYERS):
            t = {}
            for name, (n, k) in (("qkv", (QKV, D)), ("o", (D, D)), ("gu", (2 * MLP, D)), ("down", (D, MLP))):
                b = c.Buffer(n // 64 * k // 32 * 1280)
                c.fill_q4_sym(b, n, k, seed * 7919 + l * 16 + len(t), float(sigma[name]))
                t[name] = (b, n, k)
            self.layers.append(t)
        self.head = c.Buffer(VOCAB // 64 * D // 32 * 1280)
        c.fill_q4_sym(self.head, VOCAB, D, seed * 7919 + 999, 0.02)
        self.weight_bytes = sum(b.nbytes for t in self.layers for (b, n, k) in t.values()) + self.head.nbytes
        nw = np.linspace(0.8, 1.2, D) * (1 if baseline_scales else 1 - 2 * (np.arange(D) % 2))
        self.nw = c.to_device(nw.astype(np.float32))
        self.M = 0

    def alloc(self, M):
        """activation buffers for M rows (fp16-valued N(0,1) inputs), and the rstd slots"""
        c = self.c
        self.M = M
        self.x = c.Buffer(M * D * 4)
        c.fill_randn(self.x, M * D, 12345)
        # rstd slots: a (pad, rstd) pair per row for each of the 2 per layer rms ops (qkv, gate_up), all 1 / sqrt(1 + eps)
        st = np.zeros(2 * M * 2 * LAYERS + 4, np.float32)
        st[1::2] = 1.0 / np.sqrt(1.0 + 1e-6)
        self.st_host = st
        self.st = c.to_device(st)
        # the activations, one set shared by every layer (as the model's step reuses its buffers), and per-layer twins
        # that calibrate() runs the same ops on
        self.qkvp = c.Buffer(M * QKV * 4)
        self.obuf = c.Buffer(M * D * 4)
        self.mbuf = c.Buffer(M * MLP * 4)
        self.dpart = c.Buffer(4 * M * D * 4)
        self.shared = {"qkvp": self.qkvp, "obuf": self.obuf, "mbuf": self.mbuf, "dpart": self.dpart}
        self.twin = [{"qkvp": c.Buffer(M * QKV * 4), "obuf": c.Buffer(M * D * 4), "mbuf": c.Buffer(M * MLP * 4),
                      "dpart": c.Buffer(4 * M * D * 4)} for _ in range(LAYERS)]
        self.logits = c.Buffer(M * VOCAB * 4)
        mx = np.zeros(M * (VOCAB // 64) * 2 + 2 * M + 4, np.float32)
        mx[M * (VOCAB // 64) * 2 + 1::2] = 1.0
        self.mx_host = mx
        self.mx = c.to_device(mx)
        self.rstd_head = np.ones(M, np.float32)
        self.mx_stat_off = M * (VOCAB // 64) * 2 + 1
        # the token's tail: the final norm's rstd per row (what the token copies into the head's stat slot), the
        # argmax words and the staging buffer the result is copied to
        self.rsrc = c.to_device(np.tile(np.array([0.0, 1.0], np.float32), M))
        self.arg = c.Buffer(max(16, 8 * M))
        self.stage = c.Buffer(max(16, 8 * M))

    def free_weights(self):
        for t in self.layers:
            for (b, n, k) in t.values():
                b.free()
        self.head.free()
        self.nw.free()

    def rms_off(self, j):
        """stat_off of rms op j (qkv of layer l: j = 2 l, gate_up: 2 l + 1)"""
        return 2 * self.M * j + 1

    def calibrate(self, graph=False, token=False):
        """sets every rms op's rstd slots, the head's included (in the mx buffer and in the token's rsrc), to
        1 / sqrt(mean(x^2) + 1e-6) over each row that op reads, as the model's RMSNorm computes them. They are computed
        on a twin of the path about to be timed (a chain, or a recording if graph; with the token's tail if token)
        whose ops write per-layer buffers, so that every op's input can be read after a run; the arithmetic does not
        depend on the buffers' addresses, so the twin computes the timed path's values bit for bit. One slot per run
        of the twin: a run reproduces every op before the slot just set, and the next slot is computed from its
        output. Returns the rstd values set."""
        c, M = self.c, self.M

        def rstd(buf):
            x = buf.read(np.float32, M * D).reshape(M, D).astype(np.float64)
            return (1.0 / np.sqrt(np.mean(x * x, axis=1) + 1e-6)).astype(np.float32)

        got = [rstd(self.x)]
        self.st_host[self.rms_off(0)::2][:M] = got[0]
        self.st.upload(self.st_host)
        tw = (c.record if graph else c.chain)(lambda: self.ops(token=token, twin=True))
        try:
            for j in range(1, 2 * LAYERS + 1):
                if graph:
                    tw.replay()
                else:
                    tw.run()
                    if tw.status():
                        raise RuntimeError("a chain wait gave up during the rstd calibration")
                # gate_up reads o's output; the next qkv, and the head, the first K-split partial of down
                got.append(rstd(self.twin[(j - 1) // 2]["obuf"] if j % 2 else self.twin[j // 2 - 1]["dpart"]))
                if j < 2 * LAYERS:
                    self.st_host[self.rms_off(j)::2][:M] = got[-1]
                    self.st.upload(self.st_host)
        finally:
            tw.free()
        self.rstd_head = got[-1]
        self.mx_host[self.mx_stat_off::2][:M] = got[-1]
        self.mx.upload(self.mx_host)
        r = np.zeros(2 * M, np.float32)
        r[1::2] = got[-1]
        self.rsrc.upload(r)
        return np.concatenate(got)

    def head_input_norm(self):
        """per row, the rms of the head's input (the last layer's first down partial, in the shared buffer) times its
        rstd slot after a timed path's runs: ~1 when the calibration carried over to the path"""
        x = self.dpart.read(np.float32, self.M * D).reshape(self.M, D).astype(np.float64)
        return [round(float(v), 4) for v in np.sqrt(np.mean(x * x, axis=1)) * self.rstd_head]

    def free_acts(self):
        for b in (self.x, self.st, self.qkvp, self.obuf, self.mbuf, self.dpart, self.logits, self.mx, self.rsrc,
                  self.arg, self.stage):
            b.free()
        for t in self.twin:
            for b in t.values():
                b.free()

    # one projection, M = 1 through gemv, M > 1 through gemvM (the reference's decode / verify call pairs)
    def proj(self, w, n, k, x, y, pro="raw", epi="store", kPer=0, stat=None, stat_off=0, mx=None, ldx=0):
        c, M = self.c, self.M
        N = n // 2 if epi == "geglu" else n   # a geglu's weight holds the gate rows, then the up rows
        if M == 1:
            a = c.gemv_args(w=w, w_rows=n, w_cols=k, x=x, N=N, K=k, kPer=kPer, pro=c.PRO[pro], epi=c.EPI[epi], y=y,
                            stat=stat, stat_off=stat_off, norm=self.nw, mx=mx)
            return c.q4_gemv(a)
        a = c.gemvm_args(w=w, w_rows=n, w_cols=k, x=x, x_ldx=ldx or k, M=M, N=N, K=k, kPer=kPer, pro=c.PRO[pro],
                         epi=c.EPI[epi], y=y, stat=stat, stat_off=stat_off, stat_ld=2, norm=self.nw, mx=mx)
        return c.q4_gemvM(a)

    def ops(self, only=None, token=False, twin=False):
        """enqueue the step (or only one projection kind over all layers). Every op reads its predecessor's output:
        o the q rows of qkv, gate_up o's output, down gate_up's, the next layer's qkv (and the head) the first K-split
        partial of down. In the model a norm sits between some of them (normadd / rowstats, not part of the step);
        their rstd slots are inputs here (calibrate). token: the whole token, with the tail of
        engine/llm/gemma4.js:503-511 (the rstd copy into the head's stat slot before the head, the argmax after it) and
        DecodeRunner.end's copy of the result words (engine/llm/drunner.js:82-90). twin: the layers write their own
        buffers instead of the shared ones."""
        c, M = self.c, self.M
        for li in range(LAYERS):
            self.ops_layer(li, ("qkv", "o", "gu", "down") if only is None else (only,), twin)
        if only in (None, "head"):
            if token:
                for m in range(M):
                    c.copy(self.rsrc, (2 * m + 1) * 4, self.mx, (self.mx_stat_off + 2 * m) * 4, 4)
            # the head's rms slot lives in the mx buffer past the tile maxima (engine/llm/gemma4.js:505-508)
            self.proj(self.head, VOCAB, D, (self.twin[-1] if twin else self.shared)["dpart"], self.logits, "rms",
                      "softcap", stat=self.mx,
                      stat_off=self.mx_stat_off, mx=self.mx)
            if token:
                if M == 1:
                    c.argmax(self.mx, VOCAB // 64, self.arg)
                else:
                    c.argmaxM(self.mx, VOCAB // 64, M, self.arg)
                c.copy(self.arg, 0, self.stage, 0, 8 * M)

    def ops_layer(self, li, kinds, twin=False):
        """enqueue the projections `kinds` of layer li (twin: on the layer's own buffers)"""
        t = self.layers[li]
        a = self.twin[li] if twin else self.shared
        xin = self.x if li == 0 else (self.twin[li - 1] if twin else self.shared)["dpart"]
        if "qkv" in kinds:
            b, n, k = t["qkv"]
            self.proj(b, n, k, xin, a["qkvp"], "rms", stat=self.st, stat_off=self.rms_off(2 * li))
        if "o" in kinds:
            b, n, k = t["o"]
            self.proj(b, n, k, a["qkvp"], a["obuf"], "raw", kPer=2048, ldx=QKV)
        if "gu" in kinds:
            b, n, k = t["gu"]
            self.proj(b, n, k, a["obuf"], a["mbuf"], "rms", "geglu", stat=self.st, stat_off=self.rms_off(2 * li + 1))
        if "down" in kinds:
            b, n, k = t["down"]
            self.proj(b, n, k, a["mbuf"], a["dpart"], "raw", kPer=2048)

    def step_bytes(self, only=None, token=False):
        M = self.M
        tot = 0
        if token:   # the tail: the rstd copies, the argmax's read of the tile maxima, its words and their copy
            tot += M * 8 + M * (VOCAB // 64) * 8 + M * 8 + M * 16
        shapes = {"qkv": (QKV, D), "o": (D, D), "gu": (2 * MLP, D), "down": (D, MLP)}
        for kind, (n, k) in shapes.items():
            if only in (None, kind):
                out = (n // 2 if kind == "gu" else n) * (4 if kind == "down" else 1)
                tot += LAYERS * (n * k * Q4_BYTES_PER_W + M * k * 4 + M * out * 4)
        if only in (None, "head"):
            tot += VOCAB * D * Q4_BYTES_PER_W + M * D * 4 + M * VOCAB * 4 + M * (VOCAB // 64) * 8
        return tot


def time_runs(c, run, warmup, reps):
    """ms per run(): HIP events on the library's stream around `reps` back-to-back runs"""
    for _ in range(warmup):
        run()
    c.done()
    c.timer_start()
    for _ in range(reps):
        run()
    return c.timer_stop() / reps


def time_chain(c, ops, warmup, reps):
    """ops planned into one chain (p0_chain_*), timed per run; raises if any run's wait gave up"""
    ch = c.chain(ops)
    try:
        ms = time_runs(c, ch.run, warmup, reps)
        if ch.status():
            raise RuntimeError("a chain wait gave up during the benchmark")
        return ms, ch.info()
    finally:
        ch.free()


def time_recording(c, ops, warmup, reps):
    """ops recorded as one launch per op (HIP graph), timed per replay"""
    rec = c.record(ops)
    try:
        return time_runs(c, rec.replay, warmup, reps)
    finally:
        rec.free()


def bench_decode(c, step, steps, warmup, breakdown=True):
    """the M=1 token two ways, both product paths: one chain launch per token (p0_chain_*) and a recording of 124
    launches (p0_record_*); the faster is the headline. The per-projection breakdown and the 121 GEMVs alone run first:
    the chain's first dispatches after the weight fill run slower (the clock and the address translation caches settle
    over ~50 dispatches), and the headline is the steady state."""
    step.alloc(1)
    # O(1) values in every shared buffer before the one-kind chains below read them: the token chain calibrated and
    # run once
    step.calibrate(token=True)
    time_chain(c, lambda: step.ops(token=True), 1, 1)
    by_kind = {}
    for kind in ("qkv", "o", "gu", "down", "head") if breakdown else ():
        kms, _ = time_chain(c, lambda: step.ops(kind), 3, 20)
        kms_graph = time_recording(c, lambda: step.ops(kind), 3, 20)
        launches = 1 if kind == "head" else LAYERS
        by_kind[kind] = {"us_per_op_chain": round(kms * 1e3 / launches, 2),
                         "us_per_launch": round(kms_graph * 1e3 / launches, 2),
                         "GBps_chain": round(step.step_bytes(kind) / (kms * 1e-3) / 1e9, 1),
                         "GBps": round(step.step_bytes(kind) / (kms_graph * 1e-3) / 1e9, 1)}
    # each timed path on its own calibrated rstd slots (calibrate); after it, the head's input rows times their rstd
    # (~1: the calibration carried over to the timed path)
    step.calibrate(graph=True, token=True)
    ms_graph = time_recording(c, lambda: step.ops(token=True), warmup, steps)
    norm = {"graph": step.head_input_norm()}
    step.calibrate()
    ms_gemv, _ = time_chain(c, step.ops, warmup, steps)   # the 121 GEMVs alone, as one chain
    norm["gemv_chain"] = step.head_input_norm()
    r = step.calibrate(token=True)
    ms_chain, info = time_chain(c, lambda: step.ops(token=True), warmup, steps)
    norm["chain"] = step.head_input_norm()
    log("rstd slots of the token chain: %.3g - %.3g; head input x rstd after each timed path: %s"
        % (r.min(), r.max(), norm))
    mode = "chain" if ms_chain <= ms_graph else "graph"
    out = {"ms": min(ms_chain, ms_graph), "mode": mode, "ms_chain": ms_chain, "ms_graph": ms_graph,
           "ms_gemv_chain": ms_gemv, "bytes": step.step_bytes(token=True), "by_kind": by_kind, "chain": info,
           "rstd_range": [round(float(r.min()), 4), round(float(r.max()), 4)], "head_input_x_rstd": norm}
    step.free_acts()
    return out


def bench_verify(c, step, Ms=(1, 2, 4, 5, 8, 16), graph=True, calibrate=True):
    """a verify pass of M rows per M, as one chain launch and as a recording; calibrate: each path on rstd slots set
    from its own activations (Step.calibrate), else on the fixed 1 / sqrt(1 + eps)"""
    res = {}
    for M in Ms:
        step.alloc(M)
        norm = {}
        if calibrate:
            step.calibrate()
        ms_chain, _ = time_chain(c, step.ops, 3, 10)
        if calibrate:
            norm["chain"] = step.head_input_norm()
        ms_graph = float("inf")
        if graph:
            if calibrate:
                step.calibrate(graph=True)
            ms_graph = time_recording(c, step.ops, 3, 10)
            if calibrate:
                norm["graph"] = step.head_input_norm()
        ms = min(ms_chain, ms_graph)
        res[str(M)] = {"ms_per_pass": round(ms, 4), "tok_per_s": round(M / (ms * 1e-3), 1),
                       "GBps": round(step.step_bytes() / (ms * 1e-3) / 1e9, 1),
                       "ms_chain": round(ms_chain, 4), "ms_graph": round(ms_graph, 4) if graph else None}
        if calibrate:
            res[str(M)]["head_input_x_rstd"] = norm
        step.free_acts()
    return res


def bench_config_a(c, reps=8):
    """one M=1 GEMV N=8192 K=2048 over a ring of 32 weight copies (336 MB > the 256 MB last-level cache)"""
    N, K, R = 8192, 2048, 32
    ws = []
    for i in range(R):
        b = c.Buffer(N // 64 * K // 32 * 1280)
        c.fill_q4_sym(b, N, K, i, 0.02)
        ws.append(b)
    x = c.Buffer(K * 4)
    c.fill_randn(x, K, 0)
    y = c.Buffer(N * 4)

    def ops():
        for b in ws:
            c.q4_gemv(c.gemv_args(w=b, w_rows=N, w_cols=K, x=x, N=N, K=K, y=y))

    ms = time_recording(c, ops, 2, reps) / R
    for b in ws + [x, y]:
        b.free()
    byts = N * K * Q4_BYTES_PER_W + K * 4 + N * 4
    return {"us_per_launch": round(ms * 1e3, 2), "GBps": round(byts / (ms * 1e-3) / 1e9, 1), "bytes": int(byts)}


# the 8-bit GEMV shapes of Gemma-4-E2B's balanced pack, as the reference's tuner lists them with their calls per token
# (engine/tune/tunecore.js:17-21): prologue, epilogue, N, K, kPer, calls per token
Q8_E2B = [("rms", "store", 2560, 1536, 0, 12), ("rms", "store", 5120, 1536, 0, 3), ("rms", "store", 2048, 1536, 0, 16),
          ("rms", "store", 4096, 1536, 0, 4), ("raw", "store", 1536, 2048, 2048, 28),
          ("raw", "store", 1536, 4096, 2048, 7), ("rms", "geglu", 6144, 1536, 0, 4),
          ("raw", "store", 1536, 6144, 2048, 4), ("raw", "store", 256, 1536, 0, 35), ("pleg", "store", 1536, 256, 0, 35)]
Q8_REC = 4224   # one q8g64s.t64 record: 64 rows x 64 k of byte codes, then 64 fp16 scales


def q8_records(rows, K, seed):
    """synthetic q8g64s.t64 weights: uniform byte codes (stored + 128) and fp16 scales |N(0, 0.02)| / 127"""
    rng = np.random.default_rng(seed)
    nrec = (rows // 64) * (K // 64)
    rec = np.empty((nrec, Q8_REC), np.uint8)
    rec[:, :4096] = rng.integers(0, 256, (nrec, 4096), dtype=np.uint8)
    sc = (np.abs(rng.standard_normal((nrec, 64))) * 0.02 / 127).astype(np.float16)
    rec[:, 4096:] = sc.view(np.uint8)
    return rec.ravel()


def bench_q8(c, reps=4):
    """the q8g64s.t64 GEMV at the E2B balanced pack's 8-bit shapes, standalone launches replayed from a recording
    over a ring of weight copies (256 MB or more where at most 256 copies reach it, so the weights come from HBM as in a
    token): us per launch and GB/s of algorithmic bytes (records + x in + y out). Launch-bound like config A."""
    res = {}
    for pro, epi, N, K, kPer, calls in Q8_E2B:
        rows = 2 * N if epi == "geglu" else N
        wbytes = (rows // 64) * (K // 64) * Q8_REC
        R = int(min(256, max(8, -(-(256 << 20) // wbytes))))
        host = q8_records(rows, K, N + K)
        ws = [c.to_device(host) for _ in range(R)]
        x = c.Buffer(K * 4)
        c.fill_randn(x, K, 0)
        nw = c.to_device(np.linspace(0.9, 1.1, K).astype(np.float32))
        ev = c.to_device(np.linspace(-0.5, 0.5, K).astype(np.float32))
        st = c.to_device(np.array([0.0, 1.0, 0.0, 0.0], np.float32))
        nsplit = -(-K // kPer) if kPer else 1
        y = c.Buffer(nsplit * N * 4)
        kw = dict(w_enc=2, w_rows=rows, w_cols=K, x=x, N=N, K=K, kPer=kPer, pro=c.PRO[pro], epi=c.EPI[epi], y=y)
        if pro == "rms":
            kw.update(norm=nw, stat=st, stat_off=1)
        if pro == "pleg":
            kw.update(src_n=1, src_ld=K, ev=ev)

        def ops():
            for b in ws:
                c.q4_gemv(c.gemv_args(w=b, **kw))
        ms = time_recording(c, ops, 1, reps) / R
        byts = wbytes + K * 4 + nsplit * N * 4
        res[f"{pro}.{epi}.{N}x{K}"] = {"us_per_launch": round(ms * 1e3, 2), "GBps": round(byts / (ms * 1e-3) / 1e9, 1),
                                       "calls_per_token": calls, "ring_copies": R}
        for b in ws + [x, nw, ev, st, y]:
            b.free()
    return res


def bench_gemm(c, M, shapes, reps=5):
    """the dequant-GEMMs of one DiT block at M tokens: bf16 N(0,1) activations (converted to fp16 by a staging pass,
    exact for |x| >= 2^-17), fp16 output. The block figure times the block's GEMMs (each with its staging pass)
    recorded back to back and replayed; per_gemm times each GEMM replayed alone."""
    Kmax = max(k for (_, n, k) in shapes)
    Nmax = max(n for (_, n, k) in shapes)
    xf = np.random.default_rng(3).standard_normal(M * Kmax, dtype=np.float32)
    x = c.to_device((xf.view(np.uint32) >> 16).astype(np.uint16))
    del xf
    y = c.Buffer(M * Nmax * 2)
    ws = []
    for i, (name, n, k) in enumerate(shapes):
        b = c.Buffer(n // 64 * k // 32 * 1280)
        c.fill_q4_sym(b, n, k, 100 + i, 0.02)
        ws.append((name, b, n, k))
    res, tot_fl, all_args = {}, 0.0, []
    for name, b, n, k in ws:
        args = c.gemm_args(w=b, w_rows=n, w_cols=k, x=x, x_ld=k, x_mode=c.XMODE["bf16"], M=M, N=n, K=k,
                           epi=c.GEPI["f16"], y=y)
        c.q4_gemm(args)   # once eagerly: sizes the activation staging workspace outside the recording
        c.done()
        ms = time_recording(c, lambda: c.q4_gemm(args), 2, reps)   # one GEMM per replay (launch latency included)
        fl = 2.0 * M * n * k
        res[name] = {"ms": round(ms, 4), "TFLOPS": round(fl / (ms * 1e-3) / 1e12, 1)}
        tot_fl += fl
        all_args.append(args)

    def block():   # the block's linears back to back, as a DiT block runs them: one recording per block
        for a in all_args:
            c.q4_gemm(a)
    tot_ms = time_recording(c, block, 2, reps)
    for (_, b, _, _) in ws:
        b.free()
    x.free()
    y.free()
    return {"M": M, "GFLOP": round(tot_fl / 1e9, 2), "ms": round(tot_ms, 4),
            "TFLOPS": round(tot_fl / (tot_ms * 1e-3) / 1e12, 1),
            "frac_fp16_peak": round(tot_fl / (tot_ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4), "per_gemm": res}


CAL_COPY_BYTES = 256 << 20


def calibrate(c, reps=3):
    """a plain copy of known size, profiled beside the step to scale FETCH_SIZE / WRITE_SIZE: copy16_kernel reads and
    writes CAL_COPY_BYTES with 16-byte lane accesses, the same request shape as the GEMV's record loads"""
    a, b = c.Buffer(CAL_COPY_BYTES), c.Buffer(CAL_COPY_BYTES)
    a.fill_u32(0x3F800000)
    for _ in range(reps):
        c.copy(a, 0, b, 0, CAL_COPY_BYTES)
    c.done()
    a.free()
    b.free()
    log("calibration kernel: copy16_kernel reads and writes %d B" % CAL_COPY_BYTES)


READ_PROBE_BYTES = 1 << 30


def measured_peaks(c):
    """what this box sustains, reported beside the spec-sheet peaks the roofline uses: a 256 MiB device copy (bytes
    read + written per second), a 1 GiB read-only stream (p0_probe_read: the access the GEMV weights make) and the
    dense fp16 matrix-core rate (p0_probe_mfma: back-to-back MFMAs, no memory)"""
    a, b = c.Buffer(CAL_COPY_BYTES), c.Buffer(CAL_COPY_BYTES)
    a.fill_u32(0x3F800000)
    ms = time_runs(c, lambda: c.copy(a, 0, b, 0, CAL_COPY_BYTES), 2, 5)
    a.free()
    b.free()
    sink = c.Buffer(4096)
    r = c.Buffer(READ_PROBE_BYTES)
    r.fill_u32(0x3F800000)
    rms = time_runs(c, lambda: c.probe_read(r, READ_PROBE_BYTES, sink), 2, 5)
    r.free()
    fl = [0.0]

    def probe():
        fl[0] = c.probe_mfma(20000, sink)
    mms = time_runs(c, probe, 1, 3)
    sink.free()
    return {"copy_GBps": round(2 * CAL_COPY_BYTES / (ms * 1e-3) / 1e9, 1), "copy_bytes": CAL_COPY_BYTES,
            "read_GBps": round(READ_PROBE_BYTES / (rms * 1e-3) / 1e9, 1), "read_bytes": READ_PROBE_BYTES,
            "mfma_f16_dense_TFLOPS": round(fl[0] / (mms * 1e-3) / 1e12, 1),
            "spec_hbm_GBps": 8000.0, "spec_fp16_dense_TFLOPS": FP16_PEAK_TFLOPS}


def cpu_baseline(min_seconds=10.0):
    """the oracle's fp32 port of lgemv (engine/llm/lops.js:60-88) over one layer + 1/16 of the head"""
    from oracle import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    shapes = [(QKV, D), (D, D), (2 * MLP, D), (D, MLP)]
    ws = [(O.fill_q4_sym(n, k, 1 + i, 0.02), n, k) for i, (n, k) in enumerate(shapes)]
    head_rows = VOCAB // 16
    hw = O.fill_q4_sym(head_rows, D, 9, 0.02)
    x = {k: O.fill_randn(k, 5)[0] for k in (D, MLP)}
    for w, n, k in ws:   # warm-up
        O.lgemv_f32(w, x[k], n, k, threads)
    t_layer, t_head, reps, t0 = 0.0, 0.0, 0, time.time()
    while time.time() - t0 < min_seconds or reps < 2:
        a = time.perf_counter()
        for w, n, k in ws:
            O.lgemv_f32(w, x[k], n, k, threads)
        b = time.perf_counter()
        O.lgemv_f32(hw, x[D], head_rows, D, threads)
        t_layer += b - a
        t_head += time.perf_counter() - b
        reps += 1
    per_token = (t_layer / reps) * LAYERS + (t_head / reps) * 16
    return {"value": round(1.0 / per_token, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": "oracle lgemv_f32 (the reference lgemv's fp32 order) over one decoder layer's 4 GEMVs + "
                      "1/16 of the lm_head (16384x2048), %d repetitions in %.1f s; tokens/s = 1 / (30 x layer + "
                      "16 x head slice)" % (reps, time.time() - t0),
            "ms_per_token": round(per_token * 1e3, 2), "cpu": cpu_model(), "nproc": os.cpu_count()}


def cpu_model():
    """the host CPU's model name (/proc/cpuinfo), or '?'"""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "?"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-q8", action="store_true", help="leave out the q8g64s.t64 GEMV section")
    ap.add_argument("--no-extra", action="store_true", help="decode step only")
    ap.add_argument("--verify-m", default="1,2,4,5,8,12,16",
                    help="x rows of the verify passes timed (config C); empty: none")
    ap.add_argument("--verify-m-baseline", default="5,8,16",
                    help="x rows of the verify passes also timed on BASELINE's sigma 0.02 weight scales; empty: none")
    ap.add_argument("--no-config-a", action="store_true", help="skip the single-GEMV ring (config A)")
    ap.add_argument("--verify-chain-only", action="store_true",
                    help="time the verify passes as chains only (no recorded-graph timing)")
    ap.add_argument("--no-breakdown", action="store_true",
                    help="skip the per-projection timings (short runs under PMC counters)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a copy of known size (copy16_kernel, CAL_COPY_BYTES) to calibrate PMC byte "
                         "counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus %d is not supported (the hot path runs on one MI355X; "
              "sharding across GPUs is a design, not part of this build)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    from p0pc0rn_amd import capi as c
    c.open_device(0)
    info = c.device_info()
    log("device", info)

    t0 = time.time()
    step = Step(c)
    c.done()
    log("weights filled: %.2f GB in %.1f s" % (step.weight_bytes / 1e9, time.time() - t0))
    dec = bench_decode(c, step, args.steps, args.warmup, not args.no_breakdown)
    ms = dec["ms"]
    tok_s = 1e3 / ms
    step_gbps = dec["bytes"] / (ms * 1e-3) / 1e9
    log("decode step: %.4f ms -> %.1f tok/s, %.1f GB/s" % (ms, tok_s, step_gbps), dec["by_kind"])

    extra = {"decode_step": {"ms": round(ms, 4), "algorithmic_bytes": int(dec["bytes"]),
                             "GBps": round(step_gbps, 1), "frac_hbm_peak": round(step_gbps / HBM_PEAK_GBPS, 4),
                             "mode": dec["mode"], "ms_chain": round(dec["ms_chain"], 4),
                             "ms_graph": round(dec["ms_graph"], 4), "ms_gemv_chain": round(dec["ms_gemv_chain"], 4),
                             "chain": dec["chain"], "by_projection": dec["by_kind"],
                             "rstd_slots_range": dec["rstd_range"], "head_input_x_rstd": dec["head_input_x_rstd"]}}
    if not args.no_extra:
        if not args.no_config_a:
            extra["config_a_gemv"] = bench_config_a(c)
            log("config A", extra["config_a_gemv"])
        vm = tuple(int(v) for v in args.verify_m.split(",") if v.strip())
        if vm:
            extra["verify_sweep"] = bench_verify(c, step, vm, graph=not args.verify_chain_only)
            log("verify sweep", extra["verify_sweep"])
    step.free_weights()
    vb = () if args.no_extra else tuple(int(v) for v in args.verify_m_baseline.split(",") if v.strip())
    if vb:   # the same passes on BASELINE's weight scales (every layer |N(0, 0.02)|: activations grow ~4x per op)
        step = Step(c, baseline_scales=True)
        extra["verify_sweep_baseline_scales"] = bench_verify(c, step, vb, graph=False, calibrate=False)
        log("verify sweep, baseline scales", extra["verify_sweep_baseline_scales"])
        step.free_weights()
    if args.calibrate:
        calibrate(c)
    if not args.no_extra:
        extra["measured_peaks"] = measured_peaks(c)
        log("measured peaks", extra["measured_peaks"])
        if not args.no_q8:
            extra["q8_gemv_e2b_shapes"] = bench_q8(c)
            log("q8 GEMV", extra["q8_gemv_e2b_shapes"])
    if not args.no_gemm:
        extra["gemm_flux2_klein_M4608"] = bench_gemm(
            c, 4608, [("qkv", 9216, 3072), ("out", 3072, 3072), ("mlp_up", 9216, 3072), ("mlp_down", 3072, 9216)])
        log("gemm FLUX", extra["gemm_flux2_klein_M4608"])
        if not args.no_extra:
            extra["gemm_sana_video_M32760"] = bench_gemm(
                c, 32760, [("qkv", 9216, 3072), ("glu_up", 16384, 3072), ("down", 3072, 8192)], reps=2)
            log("gemm SANA", extra["gemm_sana_video_M32760"])

    # the dominant kernel, measured live with HIP events on the library's stream. Chain mode: the chain kernel is the
    # whole step (one launch per token), its algorithmic bytes the step's (weights + activations in and out). Graph
    # mode: the gate_up GEMV (mode-2 q4_gemv_kernel, 57% of a layer's bytes), 30 distinct weights back to back.
    if dec["mode"] == "chain":
        roofline = {"bound": "hbm", "achieved": round(step_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(step_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                    "kernel": ("q4_chain_pipe_kernel (the whole M=1 decode token: 121 GEMV ops, the rstd copy, the "
                               "argmax and the result copy, one launch)"),
                    "bytes_per_launch": int(dec["bytes"]), "us_per_launch": round(ms * 1e3, 2)}
        traffic_key = "decode_chain_bytes_per_launch"
    elif not dec["by_kind"]:
        roofline, traffic_key = None, None
    else:
        gu = dec["by_kind"]["gu"]
        gu_bytes = 2 * MLP * D * Q4_BYTES_PER_W + D * 4 + MLP * 4
        achieved = gu_bytes / (gu["us_per_launch"] * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                    "kernel": "q4_gemv_kernel<1,2> (gate_up 16384x2048 rms+geglu)",
                    "bytes_per_launch": int(gu_bytes), "us_per_launch": gu["us_per_launch"]}
        traffic_key = "gate_up_gemv_bytes_per_launch"
    prof = os.path.join(ROOT, "profiles", "traffic.json")
    if roofline and os.path.exists(prof):
        try:
            roofline["traffic"] = json.load(open(prof)).get(traffic_key)
        except Exception:
            pass

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline()
        log("cpu baseline", cpu)

    line = {
        "metric": "int4 GEMV HBM GB/s + decode tok/s (M=1); dequant-GEMM TFLOPS at M=4608",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "gemma4-e2b-shaped decode token, M=1: 30 x {qkv 3072x2048 rms, o 2048x2048, "
                               "gate_up 2x8192x2048 rms+geglu, down 2048x8192 kPer 2048} + rstd copy, lm_head "
                               "262144x2048 rms+softcap, argmax over 4096 tile maxima, result copy; q4g32a.t64 int4 "
                               "weights (0.625 B/weight), fp32 accumulate",
                   "weights_GB": round(step.weight_bytes / 1e9, 3),
                   "activations": "fp16-valued N(0,1) input rows; every rms op's rstd slot calibrated per timed path "
                                  "from that path's own activations, so all 30 layers and the head compute on O(1) "
                                  "values",
                   "launches_per_step": 1 if dec["mode"] == "chain" else 124, "gemv_ops_per_step": 121,
                   "ops_per_token": 124,
                   "decode_path": dec["mode"],
                   "gemv_GBps": round(step_gbps, 1),
                   "gemm_TFLOPS_M4608": extra.get("gemm_flux2_klein_M4608", {}).get("TFLOPS")},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
