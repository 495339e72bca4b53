"""qwattn: the MI355X full-attention hot path of the qwen4exp / Qwen3-Next engine.

Python mirror of the C ABI in include/qwattn.h, used by the tests and bench.py. Device memory and
streams come from PyTorch (plumbing only); every computation runs in libqwattn.so's HIP kernels.
There is no fallback: if the library is missing, or a call fails, an error is raised, the way the
reference backends throw std::runtime_error (src/vk_common.h:19-23, src/qwen4_vk.cpp:304).

The package directory name carries a hyphen, so it is loaded by path (see load_package in
tests/conftest.py, bench.py and __graft_entry__.py) under the module name `qwattn_amd`.
"""
import ctypes
import os

import torch  # loads the HIP runtime that libqwattn.so then shares

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libqwattn.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "qwattn.h")

OK, EINVAL, EHIP, ENOMEM, ERANGE, ESTATE, ETIMEOUT = 0, -1, -2, -3, -4, -5, -6
F32, BF16, F16 = 0, 1, 2
LOG2E = 1.4426950408889634


class QwattnError(RuntimeError):
    """A nonzero status from the C ABI, with qwattn_last_error's text."""

    def __init__(self, code, msg):
        super().__init__(f"{msg} (status {code})")
        self.code = code


class Config(ctypes.Structure):
    _fields_ = [("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("rope_dim", ctypes.c_int), ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("max_ctx", ctypes.c_int), ("max_tokens", ctypes.c_int), ("max_splits", ctypes.c_int)]


class MatOut(ctypes.Structure):
    """qwattn_mat_out: one matrix of qwattn_mat_multi and its output."""
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("rows", ctypes.c_int), ("y", ctypes.c_void_p),
                ("y_stride", ctypes.c_int), ("post", ctypes.c_int), ("post_scale", ctypes.c_float)]


_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int


def load_library():
    """Loads libqwattn.so (built by build.py); raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "qwattn_create": [ctypes.POINTER(_P), _I, ctypes.POINTER(Config)],
        "qwattn_destroy": [_P],
        "qwattn_get_config": [_P, ctypes.POINTER(Config)],
        "qwattn_rope_table": [_P, ctypes.POINTER(_P)],
        "qwattn_fill_rope": [_P, _P, _P, _I],
        "qwattn_kv_alloc": [_P, _I, _I],
        "qwattn_kv_grow": [_P, _P, _I],
        "qwattn_kv_slot": [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), ctypes.POINTER(_I)],
        "qwattn_qk_norm_rope_append": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I],
        "qwattn_attend_partial": [_P, _P, _P, _P, _P, _I, _I, _I, _I, ctypes.POINTER(_I)],
        "qwattn_decode_partial": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, ctypes.POINTER(_I)],
        "qwattn_decode": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, ctypes.POINTER(_I)],
        "qwattn_combine": [_P, _P, _P, _I, _P, _I, _I],
        "qwattn_attend_prefill": [_P, _P, _P, _I, _P, _P, _I, _P, _I, _P, _I, _I],
        "qwattn_attend_prefill_qg": [_P, _P, _P, _I, _P, _P, _P, _P, _I, _P, _I, _I],
        "qwattn_prefill": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I],
        "qwattn_layer_attention": [_P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I],
        "qwattn_sync_status": [_P, _P],
        "qwattn_qsa_pool": [_P, _P, _P, _I, _P, _I, _I, _P, _P, _I, _I, _I],
        "qwattn_qsa_select": [_P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _I, _I, _P, _I, _P, _I],
        "qwattn_qsa_index": [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _I, _P, _I],
        "qwattn_mat": [_P, _P, _P, _P, _I, _I, _I, _P, _I, _P, _I, _I, _I, ctypes.c_float],
        "qwattn_mat_multi": [_P, _P, _P, _I, _I, _I, _P, _I, _I],
        "qwattn_q8_unpack": [_P, _I, _I, _P, _P],
        "qwattn_qsa_key_bits": [_P, _P, _P, _I, _I, _I, _I, _P, _I],
        "qwattn_attend_partial_qsa": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P],
        "qwattn_decode_qsa": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P, _I, _P],
        "qwattn_attend_prefill_qsa": [_P, _P, _P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _P, _I],
        "qwattn_prefill_qsa": [_P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _P, _I],
        "qwattn_layer_attention_qsa": [_P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _P, _I],
        "qwattn_decode_noalloc": [_I, _P, ctypes.POINTER(Config), _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I,
                                  _I, _P, ctypes.POINTER(_I)],
        "qwattn_set_wait_limits": [_P, _I, _I],
        "qwattn_set_alloc_fault": [_P, _I],
    }
    for name, args in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = _I
    lib.qwattn_last_error.argtypes = [_P]
    lib.qwattn_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def q8_unpack(blocks, rows, cols):
    """GGUF Q8_0 rows (uint8 [rows, cols/32*34]) to the planar pair qwattn_mat takes: int8 [rows, cols] and
    float32 scales [rows, cols/32] (numpy, host memory), through the library's qwattn_q8_unpack."""
    import numpy as np
    lib = load_library()
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    w = np.zeros((rows, cols), np.int8)
    s = np.zeros((rows, cols // 32), np.float32)
    rc = lib.qwattn_q8_unpack(ctypes.c_void_p(b.ctypes.data), rows, cols, ctypes.c_void_p(w.ctypes.data),
                              ctypes.c_void_p(s.ctypes.data))
    if rc != OK:
        raise QwattnError(rc, "qwattn_q8_unpack: bad shape")
    return w, s


def header_functions():
    """Names of the functions include/qwattn.h declares."""
    import re
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(qwattn_\w+)\s*\(", text, re.M)))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}


def _check_weights(w, s):
    """(rows, cols) of a projection's weights: int8 [rows, cols] with float32 scales s [rows, cols/32] (planar
    Q8_0), or float32 [rows, cols] with s None; both contiguous, as the C ABI reads them."""
    if w.dim() != 2 or not w.is_contiguous():
        raise ValueError(f"weights must be a contiguous [rows, cols] matrix, got shape {tuple(w.shape)}")
    rows, cols = w.shape
    if s is None:
        if w.dtype != torch.float32:
            raise ValueError(f"float weights must be float32, got {w.dtype} (int8 weights need scales)")
    else:
        if w.dtype != torch.int8:
            raise ValueError(f"Q8 weights must be int8, got {w.dtype}")
        if s.dtype != torch.float32 or not s.is_contiguous() or tuple(s.shape) != (rows, cols // 32):
            raise ValueError(f"Q8 scales must be contiguous float32 [{rows}, {cols // 32}], got {s.dtype} "
                             f"{tuple(s.shape)}")
    return rows, cols


def _check_rows(t, name, width, n=None):
    """A float32 [n, >= width] operand with unit column stride (row stride free)."""
    if t.dtype != torch.float32 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be float32 [n, >= {width}] with unit column stride")
    if t.shape[1] < width:
        raise ValueError(f"{name} has {t.shape[1]} columns, needs >= {width}")
    if n is not None and t.shape[0] < n:
        raise ValueError(f"{name} has {t.shape[0]} rows, needs >= {n}")


BLK = 32  # positions per cache block


def k_block(rows):
    """[cap][NKV][D] K rows -> the blocked K cache layout of include/qwattn.h, flat (cap % 32 == 0):
    head h, block b, key kb, dim d at ((h*(cap/32) + b)*32*D) + ((((d/32)*2 + (kb/4)%2)*4 + (d/8)%4)*16
    + (kb/8)*4 + kb%4)*8 + d%8."""
    cap, nkv, d = rows.shape
    x = rows.reshape(cap // BLK, 4, 2, 4, nkv, d // 32, 4, 8)  # [b][kb/8][kb/4%2][kb%4][h][d/32][d/8%4][d%8]
    return x.permute(4, 0, 5, 2, 6, 1, 3, 7).contiguous().view(-1)


def k_rows(kcache, cap, nkv, d):
    """Inverse of k_block: the flat blocked K cache -> [cap][NKV][D] rows (a copy)."""
    x = kcache.view(nkv, cap // BLK, d // 32, 2, 4, 4, 4, 8)   # [h][b][d/32][s][g][kb/8][kb%4][e]
    return x.permute(1, 5, 3, 6, 0, 2, 4, 7).reshape(cap, nkv, d)


def v_block(rows):
    """[cap][NKV][D] V rows -> the blocked V cache layout, flat: head h, block b, key kb, dim d at
    ((h*(cap/32) + b)*32*D) + (((d/16)*4 + kb/8)*16 + d%16)*8 + kb%8."""
    cap, nkv, d = rows.shape
    x = rows.reshape(cap // BLK, 4, 8, nkv, d // 16, 16)        # [b][kb/8][kb%8][h][d/16][d%16]
    return x.permute(3, 0, 4, 1, 5, 2).contiguous().view(-1)


def v_rows(vcache, cap, nkv, d):
    """Inverse of v_block."""
    x = vcache.view(nkv, cap // BLK, d // 16, 4, 16, 8)         # [h][b][d/16][kb/8][d%16][kb%8]
    return x.permute(1, 3, 5, 0, 2, 4).reshape(cap, nkv, d)


class Attention:
    """One qwattn context: attention shape, rope table, split partials and (optionally) K/V caches."""

    def __init__(self, n_heads, n_kv_heads, head_dim, rope_dim, rope_theta=1e7, rms_eps=1e-6, max_ctx=262144,
                 max_tokens=2048, max_splits=1024, device=0):
        self.lib = load_library()
        self.cfg = Config(n_heads, n_kv_heads, head_dim, rope_dim, rope_theta, rms_eps, max_ctx, max_tokens,
                          max_splits)
        self.device = device
        h = ctypes.c_void_p()
        rc = self.lib.qwattn_create(ctypes.byref(h), device, ctypes.byref(self.cfg))
        if rc:
            raise QwattnError(rc, self.lib.qwattn_last_error(None).decode())
        self.h = h
        self.NH, self.NKV, self.D, self.R = n_heads, n_kv_heads, head_dim, rope_dim

    def close(self):
        if getattr(self, "h", None):
            self.lib.qwattn_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc:
            raise QwattnError(rc, self.lib.qwattn_last_error(self.h).decode())

    # ---- state ---------------------------------------------------------------------------------------
    def rope_table(self):
        """The context's rope table as a [max_ctx, R/2, 2] float32 tensor view (device memory)."""
        p = ctypes.c_void_p()
        self._check(self.lib.qwattn_rope_table(self.h, ctypes.byref(p)))
        n = self.cfg.max_ctx * (self.R // 2) * 2
        return _wrap_device_floats(p.value, n, self.device).view(self.cfg.max_ctx, self.R // 2, 2)

    def fill_rope(self, table, n_pos, stream=None):
        self._check(self.lib.qwattn_fill_rope(self.h, _stream(stream), _ptr(table), n_pos))

    def kv_alloc(self, n_slots, cap):
        self._check(self.lib.qwattn_kv_alloc(self.h, n_slots, cap))

    def kv_grow(self, tokens, stream=None):
        self._check(self.lib.qwattn_kv_grow(self.h, _stream(stream), tokens))

    def kv_slot(self, slot):
        """(K cache, V cache, cap): flat fp16 views of one slot's blocked caches (see k_rows / v_rows)."""
        k, v, cap = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int()
        self._check(self.lib.qwattn_kv_slot(self.h, slot, ctypes.byref(k), ctypes.byref(v), ctypes.byref(cap)))
        n = cap.value * self.NKV * self.D
        kc = _wrap_device_halfs(k.value, n, self.device)
        vc = _wrap_device_halfs(v.value, n, self.device)
        return kc, vc, cap.value

    # ---- kernels -------------------------------------------------------------------------------------
    def qk_norm_rope_append(self, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, q_out, pos, n, stream=None):
        """q_out None: the key and value rows only (for attend_prefill_qg)."""
        self._check(self.lib.qwattn_qk_norm_rope_append(
            self.h, _stream(stream), _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope),
            _ptr(kcache), _ptr(vcache), kv_cap, _ptr(q_out) if q_out is not None else None,
            _DT[q_out.dtype] if q_out is not None else 0, pos, n))

    def attend_partial(self, q, kcache, vcache, kv_cap, pos, n, n_split=0, stream=None):
        used = ctypes.c_int()
        self._check(self.lib.qwattn_attend_partial(self.h, _stream(stream), _ptr(q), _ptr(kcache), _ptr(vcache),
                                                   kv_cap, pos, n, n_split, ctypes.byref(used)))
        return used.value

    def decode_partial(self, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, pos, n, n_split=0, stream=None):
        """Fused norm + rope + append + split-KV partials (n <= 8, n * NH/NKV <= 32); returns splits."""
        used = ctypes.c_int()
        self._check(self.lib.qwattn_decode_partial(
            self.h, _stream(stream), _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope),
            _ptr(kcache), _ptr(vcache), kv_cap, pos, n, n_split, ctypes.byref(used)))
        return used.value

    def decode(self, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, out, pos, n, n_split=0, stream=None):
        """Norm + rope + append + split-KV attend + combine and gate in one launch (n <= 8, n * NH/NKV <= 32;
        the combine kernel follows only when a KV head or 16-row slice gets fewer splits than rows);
        returns the split count."""
        used = ctypes.c_int()
        self._check(self.lib.qwattn_decode(
            self.h, _stream(stream), _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope),
            _ptr(kcache), _ptr(vcache), kv_cap, _ptr(out), pos, n, n_split, ctypes.byref(used)))
        return used.value

    def combine(self, qg, out, n, n_split, stream=None):
        self._check(self.lib.qwattn_combine(self.h, _stream(stream), _ptr(qg), _DT[qg.dtype], _ptr(out), n, n_split))

    def attend_prefill(self, q, kcache, vcache, kv_cap, qg, out, pos, n, stream=None):
        self._check(self.lib.qwattn_attend_prefill(self.h, _stream(stream), _ptr(q), _DT[q.dtype], _ptr(kcache),
                                                   _ptr(vcache), kv_cap, _ptr(qg), _DT[qg.dtype], _ptr(out), pos, n))

    # ---- QSA indexer ------------------------------------------------------------------------------------

    def qsa_pool(self, ik, k_gamma, cr, raw, pooled, cap, pos, n, stream=None):
        """Caches raw indexer keys ik [n, ID] at positions pos.. into raw [cap, ID] and pools the blocks the
        call completes into pooled [cap // cr + 1, ID] (src/qwen4_qsa.h:38-54)."""
        self._check(self.lib.qwattn_qsa_pool(self.h, _stream(stream), _ptr(ik), _DT[ik.dtype], _ptr(k_gamma),
                                             ik.shape[-1], cr, _ptr(raw), _ptr(pooled), cap, pos, n))

    def qsa_select(self, iq, q_gamma, cr, budget, pooled, pos, n, mask=None, key_bits=None, stream=None):
        """Block selection of iq [n, IH, ID] (src/qwen4_qsa.h:58-91) into mask [n, mask_words] uint32 (as
        int32 storage) and/or key_bits [n, kb_words]."""
        self._check(self.lib.qwattn_qsa_select(
            self.h, _stream(stream), _ptr(iq), _DT[iq.dtype], _ptr(q_gamma), iq.shape[1], iq.shape[2], cr, budget,
            _ptr(pooled), pos, n, _ptr(mask), 0 if mask is None else mask.shape[-1], _ptr(key_bits),
            0 if key_bits is None else key_bits.shape[-1]))

    def qsa_index(self, ik, iq, k_gamma, q_gamma, cr, budget, raw, pooled, cap, pos, n, mask=None, key_bits=None,
                  stream=None):
        """qsa_pool then qsa_select in one call (one launch when no block completes); ik and iq in one dtype."""
        self._check(self.lib.qwattn_qsa_index(
            self.h, _stream(stream), _ptr(ik), _ptr(iq), _DT[iq.dtype], _ptr(k_gamma), _ptr(q_gamma), iq.shape[1],
            iq.shape[2], cr, budget, _ptr(raw), _ptr(pooled), cap, pos, n, _ptr(mask),
            0 if mask is None else mask.shape[-1], _ptr(key_bits), 0 if key_bits is None else key_bits.shape[-1]))

    def mat(self, x, y, w, s=None, post=0, post_scale=0.0, stream=None):
        """y [n, >= rows] = x [n, >= cols] W^T (Qwen4Vulkan::mat): W planar Q8 (w int8 [rows, cols] with s
        [rows, cols/32]) or float32 w [rows, cols]; post 1 applies silu(y * post_scale)."""
        rows, cols = _check_weights(w, s)
        _check_rows(x, "x", cols)
        _check_rows(y, "y", rows, n=x.shape[0])
        self._check(self.lib.qwattn_mat(self.h, _stream(stream), _ptr(w), _ptr(s), int(s is not None), rows, cols,
                                        _ptr(x), x.stride(0), _ptr(y), y.stride(0), x.shape[0], post, post_scale))

    def mat_multi(self, x, outs, stream=None):
        """Several projections of x in one call (qwattn_mat_multi): outs = [(y, w, s), ...] (s None for float32
        weights, all of one kind and one column count), each as in mat."""
        if not outs:
            raise ValueError("mat_multi: no matrices")
        q8 = outs[0][2] is not None
        cols = _check_weights(outs[0][1], outs[0][2])[1]
        _check_rows(x, "x", cols)
        arr = (MatOut * len(outs))()
        for i, (y, w, s) in enumerate(outs):
            if (s is not None) != q8:
                raise ValueError(f"mat_multi: matrix {i} mixes Q8 and float32 weights")
            rows, c = _check_weights(w, s)
            if c != cols:
                raise ValueError(f"mat_multi: matrix {i} has {c} columns, matrix 0 has {cols}")
            _check_rows(y, f"y[{i}]", rows, n=x.shape[0])
            arr[i] = MatOut(_ptr(w), _ptr(s), rows, _ptr(y), y.stride(0), 0, 0.0)
        self._check(self.lib.qwattn_mat_multi(self.h, _stream(stream), ctypes.cast(arr, ctypes.c_void_p), len(outs),
                                              int(q8), cols, _ptr(x), x.stride(0), x.shape[0]))

    def qsa_key_bits(self, mask, cr, pos, n, key_bits, stream=None):
        """Per-key visibility bits [n, kb_words] from a block mask [n, mask_words] (shaders/attention.comp:35-43)."""
        self._check(self.lib.qwattn_qsa_key_bits(self.h, _stream(stream), _ptr(mask), mask.shape[-1], cr, pos, n,
                                                 _ptr(key_bits), key_bits.shape[-1]))

    def attend_partial_qsa(self, q, kcache, vcache, kv_cap, pos, n, n_split, key_bits, stream=None):
        """attend_partial over the keys whose bit is set in key_bits [n, kb_words]; returns the split count."""
        used = ctypes.c_int()
        self._check(self.lib.qwattn_attend_partial_qsa(self.h, _stream(stream), _ptr(q), _ptr(kcache), _ptr(vcache),
                                                       kv_cap, pos, n, n_split, _ptr(key_bits), key_bits.shape[-1],
                                                       ctypes.byref(used)))
        return used.value

    def decode_qsa(self, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, out, pos, n, n_split, key_bits, stream=None):
        """decode over the keys whose bit is set in key_bits [n, kb_words]; returns the split count."""
        used = ctypes.c_int()
        self._check(self.lib.qwattn_decode_qsa(
            self.h, _stream(stream), _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope),
            _ptr(kcache), _ptr(vcache), kv_cap, _ptr(out), pos, n, n_split, _ptr(key_bits), key_bits.shape[-1],
            ctypes.byref(used)))
        return used.value

    def attend_prefill_qsa(self, q, kcache, vcache, kv_cap, qg, out, pos, n, key_bits, stream=None):
        """attend_prefill over the keys whose bit is set in key_bits [n, kb_words]."""
        self._check(self.lib.qwattn_attend_prefill_qsa(self.h, _stream(stream), _ptr(q), _DT[q.dtype], _ptr(kcache),
                                                       _ptr(vcache), kv_cap, _ptr(qg), _DT[qg.dtype], _ptr(out), pos,
                                                       n, _ptr(key_bits), key_bits.shape[-1]))

    def prefill_qsa(self, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, out, pos, n, key_bits, stream=None):
        """prefill (norm + rope + append, MFMA attention) over the keys whose bit is set in key_bits."""
        self._check(self.lib.qwattn_prefill_qsa(
            self.h, _stream(stream), _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope),
            _ptr(kcache), _ptr(vcache), kv_cap, _ptr(out), pos, n, _ptr(key_bits), key_bits.shape[-1]))

    def layer_attention_qsa(self, slot, qg, k, v, qn, kn, out, pos, n, key_bits, n_split=0, stream=None):
        self._check(self.lib.qwattn_layer_attention_qsa(
            self.h, _stream(stream), slot, _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(out),
            pos, n, n_split, _ptr(key_bits), key_bits.shape[-1]))

    def attend_prefill_qg(self, qg, qn, rope, kcache, vcache, kv_cap, out, pos, n, stream=None):
        """The MFMA prefill normalizing and rotating the query half of qg itself (the chunk's K/V rows
        already appended)."""
        self._check(self.lib.qwattn_attend_prefill_qg(self.h, _stream(stream), _ptr(qg), _DT[qg.dtype], _ptr(qn),
                                                      _ptr(rope), _ptr(kcache), _ptr(vcache), kv_cap, _ptr(out),
                                                      pos, n))

    def prefill(self, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, out, pos, n, stream=None):
        """Norm + rope + append of the chunk's K/V rows, then the MFMA prefill normalizing the query rows
        itself (rope_dim 0, 32, 64, 128 or 256; other widths go through the context's fp16 query buffer):
        two launches."""
        self._check(self.lib.qwattn_prefill(
            self.h, _stream(stream), _ptr(qg), _ptr(k), _ptr(v), _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope),
            _ptr(kcache), _ptr(vcache), kv_cap, _ptr(out), pos, n))

    def attend(self, q, kcache, vcache, kv_cap, qg, out, pos, n, n_split=0, stream=None):
        """Split-KV + combine when n * NH/NKV <= 32, else the prefill kernel (q fp32 unscaled)."""
        if n * (self.NH // self.NKV) <= 32:
            used = self.attend_partial(q, kcache, vcache, kv_cap, pos, n, n_split, stream)
            self.combine(qg, out, n, used, stream)
        else:
            self.attend_prefill(q, kcache, vcache, kv_cap, qg, out, pos, n, stream)

    def sync_status(self, stream=None):
        """Waits for the stream; raises QwattnError(ETIMEOUT) once if a bounded in-kernel wait gave up."""
        self._check(self.lib.qwattn_sync_status(self.h, _stream(stream)))

    def set_wait_limits(self, spin_max=0, epoch_skew=0):
        """Test hook of the decode kernels' bounded waits (0, 0 = production defaults)."""
        self._check(self.lib.qwattn_set_wait_limits(self.h, spin_max, epoch_skew))

    def set_alloc_fault(self, nth):
        """Test hook: the nth K/V buffer allocation of the next kv_alloc / kv_grow fails (0 = off)."""
        self._check(self.lib.qwattn_set_alloc_fault(self.h, nth))

    def layer_attention(self, slot, qg, k, v, qn, kn, out, pos, n, n_split=0, stream=None):
        self._check(self.lib.qwattn_layer_attention(self.h, _stream(stream), slot, _ptr(qg), _ptr(k), _ptr(v),
                                                    _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(out), pos, n, n_split))


def decode_noalloc(cfg, qg, k, v, qn, kn, rope, kcache, vcache, kv_cap, out, pos, n, n_split=0, wait_status=None,
                   device=0, stream=None):
    """qwattn_decode without a context or allocation (library-static scratch); returns the split count."""
    lib = load_library()
    used = ctypes.c_int()
    rc = lib.qwattn_decode_noalloc(device, _stream(stream), ctypes.byref(cfg), _ptr(qg), _ptr(k), _ptr(v),
                                   _DT[qg.dtype], _ptr(qn), _ptr(kn), _ptr(rope), _ptr(kcache), _ptr(vcache), kv_cap,
                                   _ptr(out), pos, n, n_split, _ptr(wait_status), ctypes.byref(used))
    if rc:
        raise QwattnError(rc, lib.qwattn_last_error(None).decode())
    return used.value


class _DeviceArray:
    """Minimal __cuda_array_interface__ exporter so torch can view library-owned device memory."""

    def __init__(self, ptr, n, typestr):
        self.__cuda_array_interface__ = {"shape": (n,), "typestr": typestr, "data": (ptr, False), "version": 3,
                                         "strides": None}


def _wrap_device_floats(ptr, n, device):
    return torch.as_tensor(_DeviceArray(ptr, n, "<f4"), device=f"cuda:{device}")


def _wrap_device_halfs(ptr, n, device):
    return torch.as_tensor(_DeviceArray(ptr, n, "<f2"), device=f"cuda:{device}")
