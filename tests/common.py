"""Shared helpers of the test suite: package loading, seeded inputs, the parity criterion."""
import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "qwen3-local-test_amd")

# Parity bar on the attention output: max-abs <= 2e-3 and relative <= 1e-2,
# the relative error measured as ||gpu - ref||_2 / ||ref||_2 (elementwise relative error is
# ill-conditioned where long-context outputs are close to 0).
ATOL = 2e-3
RTOL = 1e-2


def load_package():
    """Imports qwen3-local-test_amd/ (hyphenated, so by path) as the module `qwattn_amd`."""
    if "qwattn_amd" in sys.modules:
        return sys.modules["qwattn_amd"]
    spec = importlib.util.spec_from_file_location("qwattn_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qwattn_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def parity(out, ref, atol=ATOL, rtol=RTOL):
    """(max_abs, rel_l2, allclose) of out vs ref."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    d = out - ref
    max_abs = float(np.max(np.abs(d))) if d.size else 0.0
    rel = float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30))
    close = bool(np.allclose(out, ref, atol=atol, rtol=rtol))
    return max_abs, rel, close


def assert_parity(out, ref, what="", atol=ATOL, rtol=RTOL):
    max_abs, rel, close = parity(out, ref, atol, rtol)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    assert max_abs <= atol and rel <= rtol, f"{what}: max_abs {max_abs:.3e} rel_l2 {rel:.3e} (allclose {close})"
    return max_abs, rel


def assert_rows_parity(out, ref, what="", atol=ATOL, rtol=RTOL):
    """assert_parity for every token row of out/ref [n, ...] at once: each token's max-abs error <= atol and
    its relative L2 error <= rtol; the message names the worst token. Returns (max_abs, worst rel_l2)."""
    out = np.asarray(out, np.float64).reshape(len(out), -1)
    ref = np.asarray(ref, np.float64).reshape(len(ref), -1)
    assert out.shape == ref.shape, f"{what}: shapes {out.shape} vs {ref.shape}"
    assert np.all(np.isfinite(out)), f"{what}: non-finite output at tokens {np.nonzero(~np.isfinite(out).all(1))[0][:8]}"
    d = out - ref
    max_abs = np.abs(d).max(axis=1)
    rel = np.linalg.norm(d, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-30)
    bad = np.nonzero((max_abs > atol) | (rel > rtol))[0]
    t = int(bad[0]) if bad.size else int(np.argmax(max_abs))
    assert not bad.size, (f"{what}: {bad.size} of {len(out)} tokens off, first token {t}: max_abs {max_abs[t]:.3e} "
                          f"rel_l2 {rel[t]:.3e}")
    return float(max_abs.max()), float(rel.max())


class Shape:
    def __init__(self, NH, NKV, D, R, theta=1e7, eps=1e-6):
        self.NH, self.NKV, self.D, self.R, self.theta, self.eps = NH, NKV, D, R, theta, eps
        self.G = NH // NKV

    def __repr__(self):
        return f"{self.NH}q/{self.NKV}kv/d{self.D}/r{self.R}"


TINY = Shape(4, 1, 64, 16)
TINY_GGUF = Shape(2, 1, 256, 64)    # tests/make_tiny_gguf.py:10, 151 of the reference
QWEN3_NEXT = Shape(16, 2, 256, 64)  # src/model.h:15-20 of the reference
D128 = Shape(8, 2, 128, 32)        # a head_dim-128 layout: the 128-dim kernel variants


class QsaShape:
    """QSA indexer of a full-attention layer (src/qwen4.h:27, :61): IH indexer heads of ID dims, blocks of
    CR positions, a budget of `budget` keys (budget / CR blocks), rotated over the layer's rope_dim R."""

    def __init__(self, IH, ID, CR, budget, R, theta=1e7, eps=1e-6):
        self.IH, self.ID, self.CR, self.budget, self.R, self.theta, self.eps = IH, ID, CR, budget, R, theta, eps
        self.top = budget // CR

    def mask_words(self, max_ctx):
        """The mask row width of src/qwen4_vk.cpp:517-519."""
        return (max_ctx // self.CR + 1 + 31) // 32

    def __repr__(self):
        return f"qsa{self.IH}x{self.ID}/cr{self.CR}/b{self.budget}/r{self.R}"


QSA_TINY = QsaShape(2, 128, 4, 16, 64)     # tests/make_tiny_gguf.py:11 of the reference (rope_dim 64: :10)
QSA_WIDE = QsaShape(4, 128, 8, 512, 64)    # a production-like budget
QSA_BLOCK64 = QsaShape(2, 128, 64, 1024, 64)  # blocks longer than a 32-key tile
QSA_ODD = QsaShape(3, 64, 3, 48, 32)       # a ratio that divides no tile


def qsa_inputs(seed, n, qs):
    """Seeded raw indexer queries iq [n, IH, ID] and keys ik [n, ID] ~ N(0,1), and norm gammas ~ 1 + 0.1 N(0,1)
    (stored as is: the indexer multiplies by gamma, not 1 + gamma)."""
    r = np.random.default_rng(seed)
    iq = r.standard_normal((n, qs.IH, qs.ID)).astype(np.float32)
    ik = r.standard_normal((n, qs.ID)).astype(np.float32)
    qg = (1 + 0.1 * r.standard_normal(qs.ID)).astype(np.float32)
    kg = (1 + 0.1 * r.standard_normal(qs.ID)).astype(np.float32)
    return iq, ik, qg, kg


def qsa_oracle_run(oracle, calls, iq, ik, qg, kg, qs, max_ctx):
    """The oracle's indexer over a call sequence [(pos, n), ...] with inputs in call order (the reference's
    update-then-select per call, src/qwen4_cpu.cpp:326-329): masks [sum n, mask_words], and the raw and
    pooled key arrays after the last call."""
    mw = qs.mask_words(max_ctx)
    raw = np.zeros((max_ctx, qs.ID), np.float32)
    pooled = np.zeros((max_ctx // qs.CR + 1, qs.ID), np.float32)
    out, row = [], 0
    for pos, n in calls:
        raw[pos:pos + n] = ik[row:row + n]
        oracle.qsa_pool(raw, kg, pos // qs.CR, (pos + n) // qs.CR, qs.CR, qs.R, qs.theta, qs.eps, pooled)
        if (pos + n) // qs.CR > qs.top:
            out.append(oracle.qsa_select(iq[row:row + n], qg, pooled, pos, qs.CR, qs.top, qs.R, qs.theta, qs.eps, mw))
        else:
            out.append(np.full((n, mw), 0xFFFFFFFF, np.uint32))
        row += n
    return np.concatenate(out), raw, pooled


def rng(seed):
    return np.random.default_rng(seed)


def projections(seed, n, s, gamma_sd=0.1):
    """Seeded projection outputs: qg [n,NH,2D] (query | gate), k, v [n,NKV,D] ~ N(0,1), and QK-norm
    weights w with gamma = 1 + w, w ~ gamma_sd * N(0,1)."""
    r = rng(seed)
    qg = r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32)
    k = r.standard_normal((n, s.NKV, s.D)).astype(np.float32)
    v = r.standard_normal((n, s.NKV, s.D)).astype(np.float32)
    qn = (gamma_sd * r.standard_normal(s.D)).astype(np.float32)
    kn = (gamma_sd * r.standard_normal(s.D)).astype(np.float32)
    return qg, k, v, qn, kn


def cache_rows(seed, rows, s, heavy_frac=0.0, heavy_scale=8.0):
    """Seeded fp16 K/V cache rows [rows, NKV, D] ~ N(0,1); a fraction of key rows scaled (post-norm, so
    the scale survives)."""
    r = rng(seed)
    k = r.standard_normal((rows, s.NKV, s.D)).astype(np.float32)
    v = r.standard_normal((rows, s.NKV, s.D)).astype(np.float32)
    if heavy_frac > 0:
        idx = r.choice(rows, size=max(1, int(rows * heavy_frac)), replace=False)
        k[idx] *= heavy_scale
    return k.astype(np.float16), v.astype(np.float16)


def q8_blocks(seed, rows, cols, scale=0.02):
    """A seeded GGUF Q8_0 matrix: blocks uint8 [rows, cols/32*34] (per 32 weights an f16 scale then 32 int8),
    and its planar form as the GPU path takes it (src/qwen4_vk.cpp:98-106): w8 int8 [rows, cols] and
    s f32 [rows, cols/32] (the f16 scales widened)."""
    r = np.random.default_rng(seed)
    nb = cols // 32
    w8 = r.integers(-127, 128, size=(rows, cols), dtype=np.int16).astype(np.int8)
    sc16 = (scale * (0.5 + r.random((rows, nb)))).astype(np.float16)
    blocks = np.zeros((rows, nb, 34), np.uint8)
    blocks[:, :, 0:2] = sc16.view(np.uint8).reshape(rows, nb, 2)
    blocks[:, :, 2:] = w8.view(np.uint8).reshape(rows, nb, 32)
    return blocks.reshape(rows, nb * 34), w8, sc16.astype(np.float32)
