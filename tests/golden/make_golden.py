#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from a pure-Python/numpy restatement of the reference's own check
helpers. It shares no code with oracle/ (a C restatement), so each pins the other.

    python tests/golden/make_golden.py

Restated (the reference's own checks: there are no committed golden vectors in the reference):
  rng / randn            engine/kcheck.js:10-11   xorshift32 with JS int32 semantics, Box-Muller in double -> f32
  rf16 / rhe             engine/kcheck.js:12,14   fp16 round trip (f32 then RNE fp16), round half to even
  packQ4                 engine/kcheck.js:22-38   q4g32a.t64 records and their fp32 dequant
  cpuGemm                engine/kcheck.js:53      double-precision dot products
  kcheck gemm            engine/kcheck.js:72-88   M=32 N=128 K=256, X = rf16(randn(M K, 7)), W = randn(N K, 11, 0.05)
  kcheck gemv            engine/kcheck.js:126-135 N=256 K=1536, x = randn(K, 31), W = randn(N K, 32, 0.05)
  kshipped one()         engine/tune/kshipped.js:17-48  rows 128 (256 for geglu), W = randn(rows K, 33+K, 0.05),
                         x = randn(K, 34+K), nw[i] = 0.9 + 0.2 ((7919 i) % 100) / 100, ev = randn(K, 35+K, 0.5),
                         rstd = fround(1 / sqrt(sum x^2 / K + 1e-6)); want in double, epilogue then f32

Fixture files (numpy .npz, no pickles):
  kcheck_gemm.npz       x16 (fp16 bits), w (records), deq (f32), y (f64, kcheck's fp32-dequant product),
                        y_tile16 (f64, the product over fp16 tiles that the GEMM kernel computes)
  kcheck_gemv.npz       x (f32), w (records), deq_sha256, y (f64)
  kshipped_<pro>_<epi>_<K>.npz   w, x, nw, ev, rstd, deq_sha256, y (f64, after the epilogue), tile_arg (u32, softcap)
deq_sha256 is the SHA-256 of the row-major fp32 dequant's little-endian bytes (the bit-exact contract, kept small).
"""
import hashlib
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def rng(seed):
    """engine/kcheck.js:10: `s ^= s << 13; s >>>= 0; s ^= s >> 17; s ^= s << 5; s >>>= 0; return s / 2^32`.
    `<<` and `>>` act on int32 in JS: `s >> 17` of a state >= 2^31 shifts in ones."""
    s = (seed & 0xFFFFFFFF) or 1

    def i32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v >= 1 << 31 else v

    def nxt():
        nonlocal s
        s = (i32(s) ^ i32(s << 13)) & 0xFFFFFFFF
        s = (i32(s) ^ (i32(s) >> 17)) & 0xFFFFFFFF
        s = (i32(s) ^ i32(s << 5)) & 0xFFFFFFFF
        return s / 4294967296.0

    return nxt


def randn(n, seed, scale=1.0):
    """engine/kcheck.js:11 (Box-Muller in double, stored to a Float32Array)"""
    r = rng(seed)
    o = np.empty(n, np.float64)
    for i in range(0, n, 2):
        u = max(1e-9, r())
        v = r()
        m = math.sqrt(-2.0 * math.log(u)) * scale
        o[i] = m * math.cos(2.0 * math.pi * v)
        if i + 1 < n:
            o[i + 1] = m * math.sin(2.0 * math.pi * v)
    return o.astype(np.float32)


def rf16(v):
    """engine/kcheck.js:12 h2f(f2h(x)): the double is stored to a Float32Array first, then rounded to fp16 (RNE)"""
    return np.asarray(v, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def pack_q4(W, N, K):
    """engine/kcheck.js:22-38, vectorised: records (tile, group) of 1280 B, and the fp32 dequant"""
    W = np.asarray(W, np.float32).astype(np.float64).reshape(N, K // 32, 32)
    mn = rf16(W.min(axis=2))
    s = rf16((W.max(axis=2) - mn) / 15.0)
    s = np.where(s == 0.0, 1.0, s)
    q = np.clip(np.rint((W - mn[..., None]) / s[..., None]), 0, 15).astype(np.uint8)   # rint: ties to even (rhe)
    deq = (q * s[..., None] + mn[..., None]).astype(np.float32).reshape(N, K)
    NT, G = N // 64, K // 32
    codes = (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)                       # [N][G][16]
    sm = (s.astype(np.float16).view(np.uint16).astype(np.uint32)
          | (mn.astype(np.float16).view(np.uint16).astype(np.uint32) << 16))            # [N][G]
    rec = np.zeros((NT, G, 1280), np.uint8)
    c = codes.reshape(NT, 64, G, 16).transpose(0, 2, 1, 3).reshape(NT, G, 1024)
    rec[:, :, :1024] = c
    rec[:, :, 1024:] = sm.reshape(NT, 64, G).transpose(0, 2, 1).astype('<u4').copy().view(np.uint8).reshape(NT, G, 256)
    return rec.reshape(-1), deq


def digest(deq):
    return np.array([hashlib.sha256(np.ascontiguousarray(deq, "<f4").tobytes()).hexdigest()])


def gelu(v):
    """engine/tune/kshipped.js:12 (and engine/llm/lops.js:26): tanh GELU, argument clamped to +-15"""
    return v * 0.5 * (1.0 + np.tanh(np.clip(0.7978845608028654 * (v + 0.044715 * v * v * v), -15.0, 15.0)))


def kshipped_case(pro, epi, K):
    """engine/tune/kshipped.js:17-48 for the q4 encoding: inputs and the double-precision expected rows"""
    N = 128
    rows = 2 * N if epi == "geglu" else N
    W0 = randn(rows * K, 33 + K, 0.05)
    w, deq = pack_q4(W0, rows, K)
    x = randn(K, 34 + K)
    nw = np.array([0.9 + 0.2 * ((i * 7919) % 100) / 100 for i in range(K)], np.float32)
    ev = randn(K, 35 + K, 0.5)
    ss = float(np.sum(x.astype(np.float64) ** 2))
    rstd = np.float32(1.0 / math.sqrt(ss / K + 1e-6))
    xd, nwd, evd = x.astype(np.float64), nw.astype(np.float64), ev.astype(np.float64)
    xp = xd if pro == "raw" else xd * float(rstd) * nwd if pro == "rms" else gelu(xd) * evd
    dots = deq.astype(np.float64) @ xp
    if epi == "geglu":
        y = gelu(dots[:N]) * dots[N:]
    elif epi == "softcap":
        y = 30.0 * np.tanh(np.clip(dots / 30.0, -15.0, 15.0))
    else:
        y = dots
    out = dict(w=w, x=x, nw=nw, ev=ev, rstd=np.array([rstd], np.float32), deq_sha256=digest(deq), y=y)
    if epi == "softcap":
        yt = y.astype(np.float32).reshape(-1, 64)
        out["tile_arg"] = (np.arange(yt.shape[0]) * 64 + np.argmax(yt, axis=1)).astype(np.uint32)   # first max wins
    return out


def main():
    # engine/kcheck.js:72-88: the q4 matrix multiply check
    M, N, K = 32, 128, 256
    X = rf16(randn(M * K, 7)).astype(np.float32)
    w, deq = pack_q4(randn(N * K, 11, 0.05), N, K)
    y = X.reshape(M, K).astype(np.float64) @ deq.astype(np.float64).T
    # the GEMM kernel multiplies fp16 tiles of the dequant (engine/ops/gemm.js:147-148): y_tile16 is that product in
    # double; kcheck's own expectation y uses the fp32 dequant (cpuGemm), hence its looser cosine bar
    y16 = X.reshape(M, K).astype(np.float64) @ deq.astype(np.float16).astype(np.float64).T
    np.savez_compressed(os.path.join(HERE, "kcheck_gemm.npz"), x16=X.astype(np.float16).view(np.uint16), w=w,
                        deq=deq, y=y.reshape(-1), y_tile16=y16.reshape(-1), shape=np.array([M, N, K]))
    # engine/kcheck.js:126-135: the assistant's q4 matrix-vector check
    N, K = 256, 1536
    x = randn(K, 31)
    w, deq = pack_q4(randn(N * K, 32, 0.05), N, K)
    y = deq.astype(np.float64) @ x.astype(np.float64)
    np.savez_compressed(os.path.join(HERE, "kcheck_gemv.npz"), x=x, w=w, deq_sha256=digest(deq), y=y,
                        shape=np.array([N, K]))
    # engine/tune/kshipped.js: the head (softcap + tile argmax), a gate/up pair (geglu) and the per-layer-input gate
    for pro, epi, K in (("rms", "softcap", 1536), ("rms", "geglu", 1536), ("pleg", "store", 256)):
        c = kshipped_case(pro, epi, K)
        np.savez_compressed(os.path.join(HERE, "kshipped_%s_%s_%d.npz" % (pro, epi, K)), **c)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
