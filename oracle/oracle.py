"""ctypes loader of the CPU oracle (oracle/libq4oracle.so). TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use it as the checker; the product never imports it."""
import ctypes as C
import os

import numpy as np

from p0pc0rn_amd.capi import GemmArgs, GemvArgs, GemvMArgs, NormaddArgs, RowstatsArgs

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "libq4oracle.so")
_o = None


def lib():
    global _o
    if _o is None:
        if not os.path.exists(PATH):
            raise RuntimeError("oracle not built: make -C oracle")
        o = C.CDLL(PATH)
        vp, i64 = C.c_void_p, C.c_int64
        o.p0o_f2h.argtypes, o.p0o_f2h.restype = [C.c_float], C.c_uint16
        o.p0o_h2f.argtypes, o.p0o_h2f.restype = [C.c_uint16], C.c_float
        o.p0o_f2h_n.argtypes = [vp, vp, i64]
        o.p0o_h2f_n.argtypes = [vp, vp, i64]
        o.p0o_rng_uniform.argtypes = [C.c_uint32, vp, i64]
        o.p0o_randn.argtypes = [C.c_uint32, C.c_double, vp, i64]
        o.p0o_pack_q4.argtypes = [vp, i64, i64, vp, vp]
        o.p0o_dequant_q4.argtypes = [vp, i64, i64, i64, vp, vp]
        o.p0o_pack_q8.argtypes = [vp, i64, i64, vp, vp]
        o.p0o_dequant_q8.argtypes = [vp, i64, i64, i64, vp]
        o.p0o_hash.argtypes, o.p0o_hash.restype = [C.c_uint32], C.c_uint32
        o.p0o_fill_q4_sym.argtypes = [vp, i64, i64, C.c_uint32, C.c_float]
        o.p0o_fill_randn.argtypes = [vp, vp, i64, C.c_uint32, C.c_float]
        o.p0o_q4_gemv.argtypes, o.p0o_q4_gemv.restype = [C.POINTER(GemvArgs)], C.c_int
        o.p0o_q4_gemvM.argtypes, o.p0o_q4_gemvM.restype = [C.POINTER(GemvMArgs)], C.c_int
        o.p0o_q4_gemm.argtypes, o.p0o_q4_gemm.restype = [C.POINTER(GemmArgs)], C.c_int
        o.p0o_lgemv_f32.argtypes = [vp, i64, vp, i64, i64, vp, C.c_int]
        o.p0o_gemm_f32.argtypes = [vp, i64, vp, i64, i64, i64, vp, C.c_int]
        o.p0o_max_threads.restype = C.c_int
        o.p0o_rowstats.argtypes = [C.POINTER(RowstatsArgs)]
        o.p0o_normadd.argtypes = [C.POINTER(NormaddArgs)]
        o.p0o_argmaxM.argtypes = [vp, i64, i64, vp]
        _o = o
    return _o


def _p(a):
    return a.ctypes.data if a is not None else None


def f2h(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().p0o_f2h_n(_p(x), _p(out), x.size)
    return out


def h2f(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().p0o_h2f_n(_p(h), _p(out), h.size)
    return out


def rng_uniform(seed, n):
    out = np.empty(n, np.float64)
    lib().p0o_rng_uniform(seed, _p(out), n)
    return out


def randn(n, seed, scale=1.0):
    """engine/kcheck.js randn(n, seed, scale)"""
    out = np.empty(n, np.float32)
    lib().p0o_randn(seed, scale, _p(out), n)
    return out


def pack_q4(W, N, K):
    """engine/kcheck.js packQ4 -> (bytes uint8 [N/64 * K/32 * 1280], deq float32 [N, K])"""
    W = np.ascontiguousarray(W, dtype=np.float32).reshape(N, K)
    out = np.zeros((N // 64) * (K // 32) * 1280, np.uint8)
    deq = np.empty((N, K), np.float32)
    lib().p0o_pack_q4(_p(W), N, K, _p(out), _p(deq))
    return out, deq


def dequant_q4(w, N, K, wG=None):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    o32 = np.empty((N, K), np.float32)
    o16 = np.empty((N, K), np.uint16)
    lib().p0o_dequant_q4(_p(w), N, K, wG or K // 32, _p(o32), _p(o16))
    return o32, o16


def fill_q4_sym(N, K, seed, sigma=0.02):
    w = np.empty((N // 64) * (K // 32) * 1280, np.uint8)
    lib().p0o_fill_q4_sym(_p(w), N, K, seed, sigma)
    return w


def fill_randn(n, seed, sigma=1.0):
    o32 = np.empty(n, np.float32)
    o16 = np.empty(n, np.uint16)
    lib().p0o_fill_randn(_p(o32), _p(o16), n, seed, sigma)
    return o32, o16


def q4_gemv(args):
    return lib().p0o_q4_gemv(C.byref(args))


def q4_gemvM(args):
    return lib().p0o_q4_gemvM(C.byref(args))


def q4_gemm(args):
    return lib().p0o_q4_gemm(C.byref(args))


def lgemv_f32(w, x, N, K, threads=0, wG=None):
    y = np.empty(N, np.float32)
    lib().p0o_lgemv_f32(_p(w), wG or K // 32, _p(np.ascontiguousarray(x, np.float32)), N, K, _p(y), threads or max_threads())
    return y


def gemm_f32(w, x16, M, N, K, threads=0):
    y = np.empty((M, N), np.float32)
    lib().p0o_gemm_f32(_p(w), K // 32, _p(np.ascontiguousarray(x16, np.uint16)), M, N, K, _p(y), threads or max_threads())
    return y


def max_threads():
    return lib().p0o_max_threads()


def rowstats(args):
    """engine/ops/misc.js:13-40 on host pointers (RowstatsArgs)"""
    lib().p0o_rowstats(C.byref(args))


def normadd(args):
    """engine/llm/lops.js:143-178 on host pointers (NormaddArgs)"""
    lib().p0o_normadd(C.byref(args))


def argmaxM(mx, n, M):
    """engine/llm/lops_spec.js:327-348 (M = 1: engine/llm/lops.js:416-436); returns uint32 [M][2]"""
    mx = np.ascontiguousarray(mx, np.float32)
    out = np.zeros(2 * M, np.uint32)
    lib().p0o_argmaxM(mx.ctypes.data, n, M, out.ctypes.data)
    return out


def pack_q8(W, N, K):
    """packQ8 (engine/kcheck.js:39-52): (record bytes uint8, exact dequantized f32 [N][K])"""
    W = np.ascontiguousarray(W, np.float32)
    out = np.zeros(N // 64 * K // 64 * 4224, np.uint8)
    deq = np.zeros(N * K, np.float32)
    lib().p0o_pack_q8(W.ctypes.data, N, K, out.ctypes.data, deq.ctypes.data)
    return out, deq


def dequant_q8(w, N, K, wG=None):
    out = np.zeros(N * K, np.float32)
    lib().p0o_dequant_q8(np.ascontiguousarray(w).ctypes.data, N, K, wG or K // 64, out.ctypes.data)
    return out
