"""CPU ORACLE — test infrastructure only.

numpy wrappers over liboracle.so (this repository's C++ restatement of the reference CPU attention, see
oracle.cpp) and, where it was built, _ref/libref.so (the reference's own cpu_kernels.cpp primitives
compiled in place). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; the product (libqwattn.so and its Python mirror) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _host_has_avx512():
    """The v4 builds need AVX-512 F/BW/DQ/VL/CD; otherwise the AVX2 (x86-64-v3) builds are loaded."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512dq", "avx512vl", "avx512cd"} <= flags
    except OSError:
        pass
    return False


_SUFFIX = "" if _host_has_avx512() else "_v3"
LIB = os.path.join(HERE, f"liboracle{_SUFFIX}.so")
REF_LIB = os.path.join(HERE, "_ref", f"libref{_SUFFIX}.so")
REF_SRC = "/root/reference/src/cpu_kernels.cpp"

_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_I = ctypes.c_int


def build(ref=True):
    """Compiles liboracle.so and, when the reference sources are present, _ref/libref.so."""
    targets = ["all"] + (["ref"] if ref and os.path.exists(REF_SRC) else [])
    subprocess.run(["make", "-s", "-C", HERE, "-j4", *targets], check=True)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a):
    return None if a is None else a.ctypes.data_as(_F)


def _dp(a):
    return None if a is None else a.ctypes.data_as(_D)


class Oracle:
    def __init__(self, path=LIB):
        if not os.path.exists(path):
            build(ref=False)
        lib = ctypes.CDLL(path)
        lib.orc_set_threads.argtypes = [_I]
        lib.orc_set_threads.restype = _I
        lib.orc_dot_f32.argtypes = [_F, _F, _I]
        lib.orc_dot_f32.restype = ctypes.c_float
        lib.orc_inv_freq.argtypes = [_F, _I, ctypes.c_double]
        lib.orc_rope_table.argtypes = [_F, _I, _I, ctypes.c_double]
        lib.orc_rms_mul.argtypes = [_F, _F, _F, _I, ctypes.c_float]
        lib.orc_rmsnorm_one_plus.argtypes = [_F, _F, _F, _I, ctypes.c_float]
        lib.orc_rope.argtypes = [_F, _I, _I, ctypes.c_double]
        lib.orc_qk_norm_rope.argtypes = [_F, _F, _F, _F, _F, _F, _F, _F, _I, _I, _I, _I, _I, _I, ctypes.c_double,
                                         ctypes.c_float]
        lib.orc_attention.argtypes = [_F, _I, _F, _F, _F, _F, _I, _I, _I, _I, _I]
        lib.orc_attention_split.argtypes = [_F, _I, _F, _F, _F, _F, _I, _I, _I, _I, _I, _I]
        lib.orc_attention_f64.argtypes = [_D, _I, _D, _D, _D, _D, _I, _I, _I, _I, _I]
        lib.orc_qk_norm_rope_f64.argtypes = [_D, _D, _D, _I, _I, _I, ctypes.POINTER(_I), ctypes.c_double,
                                             ctypes.c_double, _I]
        for f in ("orc_inv_freq", "orc_rope_table", "orc_rms_mul", "orc_rmsnorm_one_plus", "orc_rope",
                  "orc_qk_norm_rope", "orc_attention", "orc_attention_split", "orc_attention_f64",
                  "orc_qk_norm_rope_f64"):
            getattr(lib, f).restype = None
        self.lib = lib

    def set_threads(self, n):
        return self.lib.orc_set_threads(n)

    def dot(self, a, b):
        a, b = _f32(a), _f32(b)
        return float(self.lib.orc_dot_f32(_fp(a), _fp(b), a.size))

    def inv_freq(self, R, theta):
        out = np.zeros(R // 2, np.float32)
        self.lib.orc_inv_freq(_fp(out), R, theta)
        return out

    def rope_table(self, n_pos, R, theta):
        out = np.zeros((n_pos, R // 2, 2), np.float32)
        self.lib.orc_rope_table(_fp(out), n_pos, R, theta)
        return out

    def rms_mul(self, x, gamma, eps):
        x, gamma = _f32(x), _f32(gamma)
        out = np.zeros_like(x)
        self.lib.orc_rms_mul(_fp(x), _fp(gamma), _fp(out), x.size, eps)
        return out

    def rmsnorm_one_plus(self, x, w, eps):
        x, w = _f32(x), _f32(w)
        out = np.zeros_like(x)
        self.lib.orc_rmsnorm_one_plus(_fp(x), _fp(w), _fp(out), x.size, eps)
        return out

    def rope(self, v, p, R, theta):
        v = _f32(v).copy()
        self.lib.orc_rope(_fp(v), p, R, theta)
        return v

    def qk_norm_rope(self, qg, k, v, q_gamma, k_gamma, pos, R, theta, eps, cache_rows=None):
        """qg [n,NH,2D], k/v [n,NKV,D], folded gammas [D] -> (q_out [n,NH,D], kcache, vcache) with fp32
        caches of cache_rows (default pos+n) rows whose rows [pos, pos+n) are written."""
        qg, k, v = _f32(qg), _f32(k), _f32(v)
        n, NH, D2 = qg.shape
        D = D2 // 2
        NKV = k.shape[1]
        rows = cache_rows or pos + n
        q_out = np.zeros((n, NH, D), np.float32)
        kc = np.zeros((rows, NKV, D), np.float32)
        vc = np.zeros((rows, NKV, D), np.float32)
        self.lib.orc_qk_norm_rope(_fp(qg), _fp(k), _fp(v), _fp(_f32(q_gamma)), _fp(_f32(k_gamma)), _fp(q_out),
                                  _fp(kc), _fp(vc), pos, n, NH, NKV, D, R, theta, eps)
        return q_out, kc, vc

    def attention(self, q, kcache, vcache, pos, qg=None):
        """q [n,NH,D] (or a [n,NH,2D] qg whose first half is the query), caches [rows,NKV,D] fp32,
        qg for the gate (None = no gate) -> out [n,NH,D]."""
        q = _f32(q)
        n, NH, QS = q.shape
        kcache, vcache = _f32(kcache), _f32(vcache)
        NKV, D = kcache.shape[1], kcache.shape[2]
        out = np.zeros((n, NH, D), np.float32)
        g = None if qg is None else _f32(qg)
        self.lib.orc_attention(_fp(q), QS, _fp(g), _fp(kcache), _fp(vcache), _fp(out), pos, n, NH, NKV, D)
        return out

    def attention_split(self, q, kcache, vcache, pos, chunk, qg=None):
        q = _f32(q)
        n, NH, QS = q.shape
        kcache, vcache = _f32(kcache), _f32(vcache)
        NKV, D = kcache.shape[1], kcache.shape[2]
        out = np.zeros((n, NH, D), np.float32)
        g = None if qg is None else _f32(qg)
        self.lib.orc_attention_split(_fp(q), QS, _fp(g), _fp(kcache), _fp(vcache), _fp(out), pos, n, NH, NKV, D,
                                     chunk)
        return out

    def attention_f64(self, q, kcache, vcache, pos, qg=None):
        q = np.ascontiguousarray(q, np.float64)
        n, NH, QS = q.shape
        kcache = np.ascontiguousarray(kcache, np.float64)
        vcache = np.ascontiguousarray(vcache, np.float64)
        NKV, D = kcache.shape[1], kcache.shape[2]
        out = np.zeros((n, NH, D), np.float64)
        g = None if qg is None else np.ascontiguousarray(qg, np.float64)
        self.lib.orc_attention_f64(_dp(q), QS, _dp(g), _dp(kcache), _dp(vcache), _dp(out), pos, n, NH, NKV, D)
        return out

    def qk_norm_rope_f64(self, x, gamma, row_pos, R, theta, eps, fp32_angle=True):
        x = np.ascontiguousarray(x, np.float64)
        rows, D = x.shape
        out = np.zeros_like(x)
        rp = np.ascontiguousarray(row_pos, np.int32)
        self.lib.orc_qk_norm_rope_f64(_dp(x), _dp(np.ascontiguousarray(gamma, np.float64)), _dp(out), rows, D, R,
                                      rp.ctypes.data_as(ctypes.POINTER(_I)), theta, eps, int(fp32_angle))
        return out


class RefPrimitives:
    """The reference's own compiled cpu_kernels.cpp + threadpool.h (oracle/_ref/libref.so)."""

    def __init__(self, path=REF_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        lib = ctypes.CDLL(path)
        lib.ref_set_threads.argtypes = [_I]
        lib.ref_set_threads.restype = _I
        lib.ref_dot_f32.argtypes = [_F, _F, _I]
        lib.ref_dot_f32.restype = ctypes.c_float
        lib.ref_axpy.argtypes = [_F, ctypes.c_float, _F, _I]
        lib.ref_axpy.restype = None
        lib.ref_sigmoid.argtypes = [ctypes.c_float]
        lib.ref_sigmoid.restype = ctypes.c_float
        lib.ref_half_to_f32.argtypes = [ctypes.c_uint16]
        lib.ref_half_to_f32.restype = ctypes.c_float
        lib.ref_rmsnorm_one_plus.argtypes = [_F, _F, _F, _I, ctypes.c_float]
        lib.ref_rmsnorm_one_plus.restype = None
        lib.ref_attention.argtypes = [_F, _I, _F, _F, _F, _F, _I, _I, _I, _I, _I]
        lib.ref_attention.restype = None
        self.lib = lib

    def set_threads(self, n):
        return self.lib.ref_set_threads(n)

    def dot(self, a, b):
        a, b = _f32(a), _f32(b)
        return float(self.lib.ref_dot_f32(_fp(a), _fp(b), a.size))

    def rmsnorm_one_plus(self, x, w, eps):
        x, w = _f32(x), _f32(w)
        out = np.zeros_like(x)
        self.lib.ref_rmsnorm_one_plus(_fp(x), _fp(w), _fp(out), x.size, eps)
        return out

    def attention(self, q, kcache, vcache, pos, qg=None):
        q = _f32(q)
        n, NH, QS = q.shape
        kcache, vcache = _f32(kcache), _f32(vcache)
        NKV, D = kcache.shape[1], kcache.shape[2]
        out = np.zeros((n, NH, D), np.float32)
        g = None if qg is None else _f32(qg)
        self.lib.ref_attention(_fp(q), QS, _fp(g), _fp(kcache), _fp(vcache), _fp(out), pos, n, NH, NKV, D)
        return out
