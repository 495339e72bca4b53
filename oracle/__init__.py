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
        _U = ctypes.POINTER(ctypes.c_uint32)
        lib.orc_qsa_pool.argtypes = [_F, _F, _F, _I, _I, _I, _I, _I, ctypes.c_double, ctypes.c_float]
        lib.orc_qsa_select.argtypes = [_F, _F, _F, _U, _I, _F, _I, _I, _I, _I, _I, _I, _I, _I, ctypes.c_double,
                                       ctypes.c_float]
        lib.orc_attention_qsa.argtypes = [_F, _I, _F, _F, _F, _F, _I, _I, _I, _I, _I, _U, _I, _I]
        lib.orc_mat.argtypes = [ctypes.c_void_p, _F, _F, _I, _I, _I, _F, _I, _F, _I, _I, _I, ctypes.c_float]
        for f in ("orc_mat", "orc_inv_freq", "orc_rope_table", "orc_rms_mul", "orc_rmsnorm_one_plus", "orc_rope",
                  "orc_qk_norm_rope", "orc_attention", "orc_attention_split", "orc_attention_f64",
                  "orc_qk_norm_rope_f64", "orc_qsa_pool", "orc_qsa_select", "orc_attention_qsa"):
            getattr(lib, f).restype = None
        self.lib = lib

    def set_threads(self, n):
        return self.lib.orc_set_threads(n)

    def mat(self, x, w8=None, s=None, wf=None, post=0, post_scale=0.0):
        """Y [n, rows] = X [n, cols] W^T (Qwen4Vulkan::mat): planar Q8 (w8 int8 [rows, cols], s [rows, cols/32])
        or f32 wf [rows, cols]; post 1 applies silu(y * post_scale)."""
        x = _f32(x)
        n, cols = x.shape
        q8 = w8 is not None
        if q8:
            w8 = np.ascontiguousarray(w8, dtype=np.int8)
            s = _f32(s)
            rows = w8.shape[0]
        else:
            wf = _f32(wf)
            rows = wf.shape[0]
        y = np.zeros((n, rows), np.float32)
        self.lib.orc_mat(w8.ctypes.data if q8 else None, _fp(s) if q8 else None, None if q8 else _fp(wf), int(q8),
                         rows, cols, _fp(x), cols, _fp(y), rows, n, post, post_scale)
        return y

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


    # ---- QSA indexer (src/qwen4_qsa.h) and block-sparse attention ----------------------------------

    def qsa_pool(self, raw, gamma, b0, b1, cr, R, theta, eps, pooled=None):
        """raw [rows, ID] raw indexer keys -> pooled [>= b1, ID] with blocks [b0, b1) (re)computed."""
        raw = _f32(raw)
        ID = raw.shape[1]
        if pooled is None:
            pooled = np.zeros((b1, ID), np.float32)
        assert pooled.dtype == np.float32 and pooled.flags.c_contiguous and pooled.shape[0] >= b1
        assert raw.shape[0] >= b1 * cr
        self.lib.orc_qsa_pool(_fp(raw), _fp(_f32(gamma)), _fp(pooled), b0, b1, ID, cr, R, theta, eps)
        return pooled

    def qsa_select(self, iq, gamma, pooled, pos, cr, top, R, theta, eps, mask_words, with_scores=False):
        """iq [n, IH, ID] raw indexer queries -> mask [n, mask_words] uint32 (and scores [n, nblk_max],
        NaN where a token does not select)."""
        iq = _f32(iq)
        n, IH, ID = iq.shape
        pooled = _f32(pooled)
        nmax = (pos + n) // cr
        assert pooled.shape[0] >= nmax and mask_words * 32 >= nmax
        mask = np.zeros((n, mask_words), np.uint32)
        scores = np.full((n, max(nmax, 1)), np.nan, np.float32) if with_scores else None
        self.lib.orc_qsa_select(_fp(iq), _fp(_f32(gamma)), _fp(pooled),
                                mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), mask_words, _fp(scores),
                                max(nmax, 1), pos, n, IH, ID, cr, top, R, theta, eps)
        return (mask, scores) if with_scores else mask

    def attention_qsa(self, q, kcache, vcache, pos, mask, cr, qg=None):
        """orc_attention with the QSA block mask [n, mask_words] (tail block always visible)."""
        q = _f32(q)
        n, NH, QS = q.shape
        kcache, vcache = _f32(kcache), _f32(vcache)
        NKV, D = kcache.shape[1], kcache.shape[2]
        mask = np.ascontiguousarray(mask, np.uint32)
        out = np.zeros((n, NH, D), np.float32)
        g = None if qg is None else _f32(qg)
        self.lib.orc_attention_qsa(_fp(q), QS, _fp(g), _fp(kcache), _fp(vcache), _fp(out), pos, n, NH, NKV, D,
                                   mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), mask.shape[1], cr)
        return out


TINY_GGUF = os.path.join(HERE, "_ref", "tiny_qwen4exp.gguf")
RQ4_KINDS = ("qg", "k", "v", "ik", "iq", "att")
_RQ4_CB = ctypes.CFUNCTYPE(None, ctypes.c_void_p, _I, _I, _I, _I, _F, ctypes.c_long)


class RefQwen4:
    """The reference's own qwen4exp CPU engine (Qwen4Cpu behind make_qwen4_cpu_backend, src/qwen4_cpu.cpp)
    compiled in place (oracle/_ref/libref_qwen4.so; see ref_qwen4_driver.cpp), on a GGUF model file.

    `hook(layer, kind, pos, n, arr)` (optional) sees, for every full-attention layer call, the engine's own
    arrays: kinds "qg" [n, NH, 2D], "k" / "v" [n, NKV, D], "ik" [n, ID], "iq" [n, IH, ID] (the indexer's raw
    projections; "iq" only on calls that select) and "att" [n, NH, D], the attention body's output just before
    o_proj reads it. `arr` is a numpy view of the engine's buffer: writing into the "att" array replaces the
    attention output the engine projects."""

    def __init__(self, gguf=TINY_GGUF, max_ctx=4096, threads=4,
                 path=os.path.join(HERE, "_ref", f"libref_qwen4{_SUFFIX}.so")):
        for f in (path, gguf):
            if not os.path.exists(f):
                raise FileNotFoundError(f)
        lib = ctypes.CDLL(path)
        P = ctypes.c_void_p
        lib.rq4_open.argtypes = [ctypes.c_char_p, _I, _I]
        lib.rq4_open.restype = P
        lib.rq4_error.argtypes = [P]
        lib.rq4_error.restype = ctypes.c_char_p
        lib.rq4_close.argtypes = [P]
        lib.rq4_info.argtypes = [P, ctypes.POINTER(_I), _F]
        lib.rq4_layer.argtypes = [P, _I, ctypes.POINTER(_I)]
        lib.rq4_norms.argtypes = [P, _I, _F, _F, _F, _F]
        lib.rq4_set_callback.argtypes = [P, _RQ4_CB, P]
        lib.rq4_forward.argtypes = [P, ctypes.POINTER(_I), _I, _F]
        for f in ("rq4_pos", "rq4_reset", "rq4_save_state", "rq4_restore_state"):
            getattr(lib, f).argtypes = [P]
        self.lib = lib
        self.h = lib.rq4_open(gguf.encode(), max_ctx, threads)
        if not self.h:
            raise RuntimeError(lib.rq4_error(None).decode())
        iv, fv = (_I * 10)(), (ctypes.c_float * 2)()
        lib.rq4_info(self.h, iv, fv)
        (self.hidden, self.n_layers, self.vocab, self.NH, self.NKV, self.D, self.R, self.IH, self.ID,
         self.budget) = list(iv)
        self.eps, self.theta = float(fv[0]), float(fv[1])
        self.layers = []
        for l in range(self.n_layers):
            lv = (_I * 2)()
            lib.rq4_layer(self.h, l, lv)
            self.layers.append((bool(lv[0]), int(lv[1])))
        self.hook = None
        self._cb = _RQ4_CB(self._on_array)  # kept alive with the engine
        lib.rq4_set_callback(self.h, self._cb, None)

    def _on_array(self, user, layer, kind, pos, n, data, count):
        if self.hook is None:
            return
        shapes = {0: (n, self.NH, 2 * self.D), 1: (n, self.NKV, self.D), 2: (n, self.NKV, self.D), 3: (n, self.ID),
                  4: (n, self.IH, self.ID), 5: (n, self.NH, self.D)}
        arr = np.ctypeslib.as_array(data, shape=(count,)).reshape(shapes[kind])
        self.hook(layer, RQ4_KINDS[kind], pos, n, arr)

    def full_layers(self):
        return [l for l, (full, _) in enumerate(self.layers) if full]

    def norms(self, layer):
        """(q_norm, k_norm, idx_q_norm, idx_k_norm) of a full-attention layer, as the engine holds them (the
        GGUF gammas, already 1 + w); the indexer's are zeros on a dense layer."""
        qn, kn = np.zeros(self.D, np.float32), np.zeros(self.D, np.float32)
        iqn, ikn = np.zeros(self.ID, np.float32), np.zeros(self.ID, np.float32)
        assert self.lib.rq4_norms(self.h, layer, _fp(qn), _fp(kn), _fp(iqn), _fp(ikn)) == 0
        return qn, kn, iqn, ikn

    def forward(self, tokens):
        """Backend::forward: the tokens at the current position; returns the last token's logits [vocab]."""
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.zeros(self.vocab, np.float32)
        rc = self.lib.rq4_forward(self.h, t.ctypes.data_as(ctypes.POINTER(_I)), len(t), _fp(logits))
        if rc:
            raise RuntimeError(self.lib.rq4_error(self.h).decode())
        return logits

    def pos(self):
        return self.lib.rq4_pos(self.h)

    def save_state(self):
        self.lib.rq4_save_state(self.h)

    def restore_state(self):
        self.lib.rq4_restore_state(self.h)

    def close(self):
        if self.h:
            self.lib.rq4_close(self.h)
            self.h = None


def qsa_key_bits(mask, pos, n, cr):
    """The per-key visibility the block-sparse kernels consume: bits [n, ceil((pos + n) / 32)] uint32, bit j
    of token t set when key j is in a complete block whose mask bit is set or in the tail block (keys from
    ((pos + t + 1) // cr) * cr on), as shaders/attention.comp:35-43 tests it. Keys past a token's own length
    follow the tail rule (visible); causality masks them separately."""
    maxlen = pos + n
    words = (maxlen + 31) // 32
    j = np.arange(words * 32)
    blk = j // cr
    mask = np.asarray(mask, np.uint32)
    out = np.zeros((n, words), np.uint32)
    for t in range(n):
        tail = (pos + t + 1) // cr * cr
        wi = np.minimum(blk >> 5, mask.shape[1] - 1)
        bit = (mask[t][wi] >> (blk & 31).astype(np.uint32)) & 1
        vis = (j >= tail) | ((bit == 1) & ((blk >> 5) < mask.shape[1]))
        out[t] = (vis.reshape(words, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1)
    return out


class RefQsa:
    """The reference's own QSA indexer (class QsaIndexer, src/qwen4_qsa.h) compiled in place with the sources
    it needs (oracle/_ref/libref_qsa.so; see ref_qsa_driver.cpp)."""

    def __init__(self, path=os.path.join(HERE, "_ref", f"libref_qsa{_SUFFIX}.so")):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        lib = ctypes.CDLL(path)
        _IP = ctypes.POINTER(_I)
        lib.ref_qsa_run.argtypes = [_I, _I, _I, _I, _I, ctypes.c_float, ctypes.c_float, _F, _F, _I, _I, _I, _IP, _IP,
                                    _F, _F, ctypes.POINTER(ctypes.c_uint32), _I]
        lib.ref_qsa_run.restype = _I
        lib.ref_mat_q8.argtypes = [ctypes.c_void_p, _I, _I, _F, _I, _F, _I]
        lib.ref_mat_q8.restype = _I
        self.lib = lib

    def mat_q8(self, blocks, rows, cols, x, threads=4):
        """Y [n, rows] = X [n, cols] W^T through the reference's CPU path (gq::run_jobs) for W in GGUF Q8_0
        blocks (uint8 [rows, cols/32*34])."""
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        x = _f32(x)
        y = np.zeros((x.shape[0], rows), np.float32)
        assert self.lib.ref_mat_q8(blocks.ctypes.data, rows, cols, _fp(x), x.shape[0], _fp(y), threads) == 0
        return y

    def run(self, calls, iq, ik, q_gamma, k_gamma, cr, budget, R, theta, eps, max_ctx, mask_words, threads=4):
        """calls: [(pos, n), ...] in order; iq [sum n, IH, ID], ik [sum n, ID] in call order ->
        mask [sum n, mask_words] uint32."""
        iq, ik = _f32(iq), _f32(ik)
        IH, ID = iq.shape[1], iq.shape[2]
        cp = np.array([c[0] for c in calls], np.int32)
        cn = np.array([c[1] for c in calls], np.int32)
        mask = np.zeros((int(cn.sum()), mask_words), np.uint32)
        rc = self.lib.ref_qsa_run(IH, ID, cr, budget, R, theta, eps, _fp(_f32(q_gamma)), _fp(_f32(k_gamma)), max_ctx,
                                  threads, len(calls), cp.ctypes.data_as(ctypes.POINTER(_I)),
                                  cn.ctypes.data_as(ctypes.POINTER(_I)), _fp(iq), _fp(ik),
                                  mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), mask_words)
        assert rc == 0, rc
        return mask


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
