"""ctypes binding of the C ABI (include/p0pc0rn.h) for Python callers: the tests and bench.py.

The Node host (p0pc0rn_amd/js) is the reference-shaped host; this module is a thin, faithful mirror of the same C
entry points. The library must be built (python -m p0pc0rn_amd.build); a missing library raises at import of `lib()`,
there is no fallback of any kind.
"""
import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libp0pc0rn_hip.so")

P0_OK, P0_EINVAL, P0_EHIP, P0_ENODEV, P0_ENOMEM = 0, 1, 2, 3, 4
ENC = {"q4g32a.t64": 1, "q8g64s.t64": 2, "f16": 3}
PRO = {"raw": 0, "rms": 1, "sum": 2, "pleg": 3}
EPI = {"store": 0, "geglu": 1, "softcap": 2}
XMODE = {"f16": 0, "lnmod": 1, "rms": 2, "bf16": 3}
GEPI = {"f16": 0, "f32": 1, "resadd": 2, "swiglu": 3, "bias": 4, "heads": 5}
ROPE = {"inter": 0, "half": 1}
ACT = {"silu": 0, "gelu": 1}

# every symbol the header declares (tests check the library exports each one)
HEADER_SYMBOLS = [
    "p0_last_error", "p0_version", "p0_open", "p0_close", "p0_device_info", "p0_set_stream", "p0_get_stream",
    "p0_buffer", "p0_free", "p0_upload", "p0_read", "p0_fill", "p0_copy", "p0_done", "p0_timer_start", "p0_timer_stop",
    "p0_q4_gemv", "p0_q4_gemvM", "p0_q4_gemm", "p0_q4_gemm_noalloc", "p0_q4_dequant", "p0_fill_q4_sym", "p0_fill_randn", "p0_gemv_tune",
    "p0_probe_mfma",
    "p0_probe_read",
    "p0_record_begin", "p0_record_end", "p0_replay", "p0_record_info", "p0_record_free",
    "p0_chain_begin", "p0_chain_end", "p0_chain_run", "p0_chain_status", "p0_chain_info", "p0_chain_free",
    "p0_chain_tune", "p0_rowstats", "p0_normadd", "p0_argmax", "p0_argmaxM", "p0_upload_file",
]

i64, i32, f32, vp = C.c_int64, C.c_int32, C.c_float, C.c_void_p


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("device", C.c_int), ("cu_count", C.c_int), ("xcd_count", C.c_int),
                ("hbm_bytes", i64), ("lds_bytes_per_cu", i64), ("clock_khz", C.c_int), ("workspace_bytes", i64)]


class ChainInfo(C.Structure):
    _fields_ = [("n_ops", i32), ("m", i32), ("workgroups", i32), ("waves_per_workgroup", i32), ("lds_bytes", i64),
                ("mailboxes", i32), ("staged", i32), ("passes", i32)]


class GemvArgs(C.Structure):
    _fields_ = [("w", vp), ("w_off", i64), ("w_enc", i32), ("w_rows", i64), ("w_cols", i64),
                ("x", vp), ("x_rowB", i64), ("N", i64), ("K", i64), ("kPer", i64), ("pro", i32), ("epi", i32),
                ("y", vp), ("ldy", i64), ("stat", vp), ("stat_off", i64), ("norm", vp), ("norm_off", i64),
                ("src_n", i64), ("src_ld", i64), ("ev", vp), ("ev_off", i64), ("mx", vp), ("cap", f32)]


class GemvMArgs(C.Structure):
    _fields_ = [("w", vp), ("w_off", i64), ("w_enc", i32), ("w_rows", i64), ("w_cols", i64),
                ("x", vp), ("x_ldx", i64), ("x_rowB", i64), ("M", i64), ("N", i64), ("K", i64), ("kPer", i64),
                ("pro", i32), ("epi", i32), ("y", vp), ("y_ldy", i64), ("y_ldm", i64),
                ("stat", vp), ("stat_off", i64), ("stat_ld", i64), ("norm", vp), ("norm_off", i64),
                ("src_n", i64), ("src_ld", i64), ("ev", vp), ("ev_off", i64), ("ev_ld", i64), ("mx", vp), ("cap", f32)]


class GemmArgs(C.Structure):
    _fields_ = [("w", vp), ("w_off", i64), ("w_enc", i32), ("w_rows", i64), ("w_cols", i64),
                ("x", vp), ("x_off", i64), ("x_ld", i64), ("x_k0", i64), ("x_mode", i32),
                ("M", i64), ("N", i64), ("K", i64), ("wr0", i64), ("wr1", i64), ("wk0", i64), ("epi", i32),
                ("y", vp), ("y_off", i64), ("y_ld", i64), ("y_n0", i64), ("ev", vp), ("ev_off", i64),
                ("stats", vp), ("stats_off", i64), ("pv", vp), ("pv_off", i64), ("pv_stride", i64),
                ("bv", vp), ("bv_off", i64), ("bv_up", i64), ("act", i32), ("store", i32), ("res", i32),
                ("heads_ltot", i64), ("heads_row_off", i64), ("heads_hq", i32), ("heads_hkv", i32),
                ("heads_eps", f32), ("heads_rope", i32), ("rope", vp)]


class RowstatsArgs(C.Structure):
    _fields_ = [("x", vp), ("x_off", i64), ("x_ld", i64), ("x_c0", i64), ("rows", i64), ("cols", i64), ("mode", i32),
                ("eps", f32), ("st", vp), ("st_off", i64)]


class NormaddArgs(C.Structure):
    _fields_ = [("t", vp), ("t_n", i64), ("t_ld", i64), ("w", vp), ("w_off", i64), ("x", vp), ("st", vp),
                ("st_off", i64), ("D", i64), ("M", i64), ("eps", f32), ("scale", f32), ("mode", i32)]


class P0Error(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


_lib = None


def lib():
    """The loaded C-ABI library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("p0pc0rn: %s is not built (python -m p0pc0rn_amd.build)" % LIB_PATH)
        L = C.CDLL(LIB_PATH)
        L.p0_last_error.restype = C.c_char_p
        L.p0_get_stream.restype = vp
        sig = {
            "p0_open": [C.c_int], "p0_close": [], "p0_device_info": [C.POINTER(DeviceInfo)], "p0_set_stream": [vp],
            "p0_buffer": [C.c_size_t, C.POINTER(vp)], "p0_free": [vp],
            "p0_upload": [vp, C.c_size_t, vp, C.c_size_t], "p0_read": [vp, vp, C.c_size_t, C.c_size_t],
            "p0_fill": [vp, C.c_size_t, C.c_uint32, C.c_size_t], "p0_done": [], "p0_timer_start": [],
            "p0_copy": [vp, C.c_size_t, vp, C.c_size_t, C.c_size_t],
            "p0_timer_stop": [C.POINTER(f32)],
            "p0_q4_gemv": [C.POINTER(GemvArgs), C.POINTER(i32)], "p0_q4_gemvM": [C.POINTER(GemvMArgs), C.POINTER(i32)],
            "p0_q4_gemm": [C.POINTER(GemmArgs), C.POINTER(C.c_double)],
            "p0_q4_gemm_noalloc": [C.POINTER(GemmArgs), C.POINTER(C.c_double)],
            "p0_q4_dequant": [vp, i64, i64, i64, vp, vp], "p0_fill_q4_sym": [vp, i64, i64, i64, C.c_uint32, f32],
            "p0_fill_randn": [vp, i64, i64, C.c_uint32, f32, i32], "p0_gemv_tune": [C.c_int, C.c_int],
            "p0_probe_mfma": [i64, vp, C.POINTER(C.c_double)],
            "p0_probe_read": [vp, i64, vp],
            "p0_record_begin": [], "p0_record_end": [C.POINTER(vp)], "p0_replay": [vp], "p0_record_free": [vp],
            "p0_record_info": [vp, C.POINTER(i32)],
            "p0_chain_begin": [], "p0_chain_end": [C.POINTER(vp)], "p0_chain_run": [vp],
            "p0_chain_status": [vp, C.POINTER(i32)], "p0_chain_info": [vp, C.POINTER(ChainInfo)], "p0_chain_free": [vp],
            "p0_chain_tune": [C.c_int, C.c_int],
            "p0_rowstats": [C.POINTER(RowstatsArgs)], "p0_normadd": [C.POINTER(NormaddArgs)],
            "p0_argmax": [vp, i64, vp], "p0_argmaxM": [vp, i64, i64, vp],
            "p0_upload_file": [C.c_char_p, i64, i64, vp, i64],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int
        _lib = L
    return _lib


def check(rc):
    if rc != P0_OK:
        raise P0Error(rc, lib().p0_last_error().decode())
    return rc


def last_error():
    return lib().p0_last_error().decode()


# ------------------------------------------------------------------------------------------------ device + buffers
class Buffer:
    """A device allocation made through p0_buffer (freed explicitly or when collected)."""

    def __init__(self, nbytes):
        p = vp()
        check(lib().p0_buffer(nbytes, C.byref(p)))
        self.ptr = p.value
        self.nbytes = nbytes

    def free(self):
        if self.ptr:
            lib().p0_free(self.ptr)
            self.ptr = 0

    def upload(self, arr, off=0):
        a = np.ascontiguousarray(arr)
        if off + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        check(lib().p0_upload(self.ptr, off, a.ctypes.data, a.nbytes))
        return self

    def read(self, dtype, count=None, off=0):
        dt = np.dtype(dtype)
        count = (self.nbytes - off) // dt.itemsize if count is None else count
        out = np.empty(count, dtype=dt)
        check(lib().p0_read(out.ctypes.data, self.ptr, off, out.nbytes))
        return out

    def fill_u32(self, value, words=None, off=0):
        words = (self.nbytes - off) // 4 if words is None else words
        check(lib().p0_fill(self.ptr, off, value & 0xFFFFFFFF, words))
        return self


def to_device(arr):
    a = np.ascontiguousarray(arr)
    return Buffer(max(a.nbytes, 16)).upload(a)


def open_device(device=0):
    check(lib().p0_open(device))


def close_device():
    lib().p0_close()


def device_info():
    d = DeviceInfo()
    check(lib().p0_device_info(C.byref(d)))
    return {"name": d.name.decode(), "device": d.device, "cu_count": d.cu_count, "xcd_count": d.xcd_count,
            "hbm_bytes": d.hbm_bytes, "lds_bytes_per_cu": d.lds_bytes_per_cu, "clock_khz": d.clock_khz,
            "workspace_bytes": d.workspace_bytes}


def done():
    check(lib().p0_done())


def copy(src, src_off, dst, dst_off, nbytes):
    """device-to-device copy on the library's stream (runner.copy)"""
    check(lib().p0_copy(_ptr(src), src_off, _ptr(dst), dst_off, nbytes))


def timer_start():
    check(lib().p0_timer_start())


def timer_stop():
    ms = f32()
    check(lib().p0_timer_stop(C.byref(ms)))
    return ms.value


class Recording:
    """A recorded op sequence (p0_record_begin ... p0_record_end), replayed with one launch."""

    def __init__(self, handle):
        self.handle = handle

    def replay(self):
        check(lib().p0_replay(self.handle))

    def launches(self):
        n = i32()
        check(lib().p0_record_info(self.handle, C.byref(n)))
        return n.value

    def free(self):
        if self.handle:
            lib().p0_record_free(self.handle)
            self.handle = None


def record(fn):
    """Record the ops fn() enqueues into a Recording (they do not run now)."""
    check(lib().p0_record_begin())
    try:
        fn()
    finally:
        h = vp()
        rc = lib().p0_record_end(C.byref(h))
    check(rc)
    return Recording(h.value)


def gemv_tune(knob, value=0):
    return lib().p0_gemv_tune(knob, value)


def probe_mfma(iters, sink):
    """enqueue the matrix-core probe (p0_probe_mfma); returns the flops enqueued"""
    fl = C.c_double()
    check(lib().p0_probe_mfma(iters, _ptr(sink), C.byref(fl)))
    return fl.value


def probe_read(buf, nbytes, sink):
    """enqueue one read pass over nbytes of buf (p0_probe_read)"""
    check(lib().p0_probe_read(_ptr(buf), nbytes, _ptr(sink)))


class Chain:
    """A GEMV chain (p0_chain_begin ... p0_chain_end): the recorded ops run as one persistent launch."""

    def __init__(self, handle):
        self.handle = handle

    def run(self):
        check(lib().p0_chain_run(self.handle))

    def status(self):
        """waits for the stream; True if a wait of an earlier run gave up (that run's results are invalid)"""
        t = i32()
        check(lib().p0_chain_status(self.handle, C.byref(t)))
        return bool(t.value)

    def info(self):
        d = ChainInfo()
        check(lib().p0_chain_info(self.handle, C.byref(d)))
        return {f: getattr(d, f) for f, _ in ChainInfo._fields_}

    def free(self):
        if self.handle:
            lib().p0_chain_free(self.handle)
            self.handle = None


def chain(fn):
    """Plan the gemv / gemvM calls fn() makes into a Chain (they do not run now)."""
    check(lib().p0_chain_begin())
    try:
        fn()
    finally:
        h = vp()
        rc = lib().p0_chain_end(C.byref(h))
    check(rc)
    return Chain(h.value)


def chain_tune(knob, value=0):
    return lib().p0_chain_tune(knob, value)


# ------------------------------------------------------------------------------------------------ ops
def _ptr(b):
    return None if b is None else (b.ptr if isinstance(b, Buffer) else int(b))


def gemv_args(**kw):
    """GemvArgs from keyword fields; Buffer objects are accepted where the header takes a pointer."""
    a = GemvArgs()
    a.w_enc = 1
    a.cap = 30.0
    for k, v in kw.items():
        setattr(a, k, _ptr(v) if k in ("w", "x", "y", "stat", "norm", "ev", "mx") else v)
    return a


def gemvm_args(**kw):
    a = GemvMArgs()
    a.w_enc = 1
    a.cap = 30.0
    for k, v in kw.items():
        setattr(a, k, _ptr(v) if k in ("w", "x", "y", "stat", "norm", "ev", "mx") else v)
    return a


def gemm_args(**kw):
    a = GemmArgs()
    a.w_enc = 1
    for k, v in kw.items():
        setattr(a, k, _ptr(v) if k in ("w", "x", "y", "ev", "stats", "pv", "bv", "rope") else v)
    return a


def q4_gemv(args):
    n = i32()
    check(lib().p0_q4_gemv(C.byref(args), C.byref(n)))
    return n.value


def q4_gemvM(args):
    n = i32()
    check(lib().p0_q4_gemvM(C.byref(args), C.byref(n)))
    return n.value


def q4_gemm(args):
    fl = C.c_double()
    check(lib().p0_q4_gemm(C.byref(args), C.byref(fl)))
    return fl.value


def q4_gemm_noalloc(args):
    """p0_q4_gemm_noalloc: the same GEMM, staging through the library's static scratch (allocates nothing)"""
    fl = C.c_double()
    check(lib().p0_q4_gemm_noalloc(C.byref(args), C.byref(fl)))
    return fl.value


def q4_dequant(w, N, K, out32=None, out16=None, w_off=0):
    check(lib().p0_q4_dequant(_ptr(w), w_off, N, K, _ptr(out32), _ptr(out16)))


def fill_q4_sym(w, N, K, seed, sigma=0.02, w_off=0):
    check(lib().p0_fill_q4_sym(_ptr(w), w_off, N, K, seed, sigma))


def fill_randn(dst, n, seed, sigma=1.0, as_f16=False, off_bytes=0):
    check(lib().p0_fill_randn(_ptr(dst), off_bytes, n, seed, sigma, 1 if as_f16 else 0))


# ------------------------------------------------------------------------------------------------ rowstats / normadd / argmax
def rowstats_args(**kw):
    a = RowstatsArgs()
    for k, v in kw.items():
        setattr(a, k, _ptr(v) if k in ("x", "st") else v)
    return a


def normadd_args(**kw):
    a = NormaddArgs()
    a.scale = 1.0
    for k, v in kw.items():
        setattr(a, k, _ptr(v) if k in ("t", "w", "x", "st") else v)
    return a


def rowstats(args):
    check(lib().p0_rowstats(C.byref(args)))


def normadd(args):
    check(lib().p0_normadd(C.byref(args)))


def argmax(mx, n, out):
    check(lib().p0_argmax(_ptr(mx), n, _ptr(out)))


def argmaxM(mx, n, M, out):
    check(lib().p0_argmaxM(_ptr(mx), n, M, _ptr(out)))


def upload_file(path, offset, nbytes, dst, dst_off=0):
    """bytes [offset, offset + nbytes) of a file -> device memory (the pack reader's I/O, engine/core/store.js:221-244)"""
    check(lib().p0_upload_file(os.fsencode(path), offset, nbytes, _ptr(dst), dst_off))
