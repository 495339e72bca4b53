"""Pins of the CPU oracle (oracle/), the checker every GPU parity test uses.

Each function of the oracle is held to something other than its own formula: closed forms and
invariants, the fp64 golden fixtures (an independent float64 restatement with a portable seeded
generator), the reference's own compiled primitives (oracle/_ref, when /root/reference is present),
and a fixture from the installed Hugging Face Qwen3-Next attention. The planted-mistake tests show
that these pins catch the plausible errors (interleaved instead of rotate-half RoPE, gamma instead of
1 + gamma, wrong GQA grouping, non-causal mask).
"""
import os

import numpy as np
import pytest

from common import QWEN3_NEXT, TINY, cache_rows, projections

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---- primitives -----------------------------------------------------------------------------------------

def test_dot_matches_fp64(oracle):
    r = np.random.default_rng(0)
    for n in (1, 31, 32, 33, 64, 256, 1000):
        a, b = r.standard_normal(n).astype(np.float32), r.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert abs(oracle.dot(a, b) - exact) <= 1e-5 * (1 + np.abs(a * b).sum())


def test_inv_freq_closed_form(oracle):
    R, theta = 64, 1e7
    inv = oracle.inv_freq(R, theta)
    assert inv[0] == 1.0
    for i in range(R // 2):
        assert inv[i] == np.float32(1.0 / theta ** (2.0 * i / R))
    # geometric: consecutive ratios are theta^(-2/R)
    assert np.allclose(inv[1:] / inv[:-1], theta ** (-2.0 / R), rtol=1e-6)


def test_rms_mul_closed_form(oracle):
    D, eps = 256, 1e-6
    for c in (0.5, -3.0, 1e-3):
        x = np.full(D, c, np.float32)
        g = np.linspace(0.5, 1.5, D).astype(np.float32)
        out = oracle.rms_mul(x, g, eps)
        exp = np.sign(c) / np.sqrt(1 + eps / c ** 2) * g
        assert np.allclose(out, exp, rtol=1e-6, atol=1e-7)
    # unit gamma: RMS of the output is 1 (eps negligible)
    x = np.random.default_rng(1).standard_normal(D).astype(np.float32) * 7
    out = oracle.rms_mul(x, np.ones(D, np.float32), 0.0)
    assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1) < 1e-6


def test_rmsnorm_forms_agree(oracle):
    """rmsnorm(one_plus) with double accumulation (src/cpu_kernels.cpp:306-314) and rms_mul with the
    folded gamma (src/qwen4_cpu.cpp:19-23) are the same function."""
    r = np.random.default_rng(2)
    x = r.standard_normal(256).astype(np.float32)
    w = (0.1 * r.standard_normal(256)).astype(np.float32)
    assert np.allclose(oracle.rmsnorm_one_plus(x, w, 1e-6), oracle.rms_mul(x, 1 + w, 1e-6), rtol=2e-6, atol=1e-7)


def test_rope_identity_norm_passthrough(oracle):
    R, theta = 64, 1e7
    v = np.random.default_rng(3).standard_normal(256).astype(np.float32)
    assert np.array_equal(oracle.rope(v, 0, R, theta), v)  # p = 0: cos 1, sin 0
    for p in (1, 17, 4096, 262143):
        y = oracle.rope(v, p, R, theta)
        assert np.array_equal(y[R:], v[R:])  # dims >= R pass through
        pair = lambda a: a[:R // 2].astype(np.float64) ** 2 + a[R // 2:R].astype(np.float64) ** 2
        assert np.allclose(pair(y), pair(v), rtol=1e-5)  # each (i, i + R/2) pair is rotated


def test_rope_relative_position(oracle):
    """After rope, q.k depends on the position difference only (up to fp32 angle rounding)."""
    R, theta = 64, 1e7
    r = np.random.default_rng(4)
    q, k = r.standard_normal(256).astype(np.float32), r.standard_normal(256).astype(np.float32)
    base = float(np.dot(oracle.rope(q, 10, R, theta), oracle.rope(k, 3, R, theta)))
    for shift in (1, 50, 300):
        s = float(np.dot(oracle.rope(q, 10 + shift, R, theta), oracle.rope(k, 3 + shift, R, theta)))
        assert abs(s - base) <= 2e-4 * (1 + abs(base))


def test_rope_longpos_fixture(oracle):
    """Norm + rope at positions up to the 256K limit against fp64 with the engine's fp32 angle."""
    f = np.load(os.path.join(GOLDEN, "rope_longpos.npz"))
    D, R = (int(v) for v in f["dims"])
    for i, p in enumerate(f["pos"]):
        y = oracle.rope(oracle.rms_mul(f["x"][i], 1 + f["w"], float(f["eps"])), int(p), R, float(f["theta"]))
        assert np.abs(y - f["y"][i]).max() <= 2e-5, p
    # the fixture really pins the fp32 angle: the exact-angle rotation differs at large p
    x64 = f["x"][-1:].astype(np.float64)
    exact = oracle.qk_norm_rope_f64(x64, 1 + f["w"].astype(np.float64), f["pos"][-1:], R, float(f["theta"]),
                                    float(f["eps"]), fp32_angle=False)
    assert np.abs(exact[0] - f["y"][-1]).max() > 1e-3


# ---- attention special cases ------------------------------------------------------------------------------

def _rand_attn(seed, n, NH, NKV, D, rows):
    r = np.random.default_rng(seed)
    q = r.standard_normal((n, NH, D)).astype(np.float32)
    qg = r.standard_normal((n, NH, 2 * D)).astype(np.float32)
    kc = r.standard_normal((rows, NKV, D)).astype(np.float32)
    vc = r.standard_normal((rows, NKV, D)).astype(np.float32)
    return q, qg, kc, vc


def sig(x):
    return 1 / (1 + np.exp(-x.astype(np.float64)))


def test_single_key(oracle):
    q, qg, kc, vc = _rand_attn(5, 1, 4, 1, 64, 1)
    out = oracle.attention(q, kc, vc, 0, qg)
    assert np.allclose(out[0], vc[0, 0] * sig(qg[0, :, 64:]), rtol=1e-6, atol=1e-7)


def test_identical_keys_average_values(oracle):
    q, qg, kc, vc = _rand_attn(6, 1, 4, 1, 64, 50)
    kc[:] = kc[0]
    out = oracle.attention(q, kc, vc, 49, qg)
    assert np.allclose(out[0], vc[:, 0].mean(0) * sig(qg[0, :, 64:]), rtol=1e-5, atol=1e-6)


def test_dominant_key_selects_its_value(oracle):
    q, qg, kc, vc = _rand_attn(7, 1, 4, 1, 64, 40)
    kc[17, 0] = q[0, 0] * 50  # score ~ 50 * |q|^2 / 8 for head 0
    out = oracle.attention(q, kc, vc, 39, qg)
    assert np.allclose(out[0, 0], vc[17, 0] * sig(qg[0, 0, 64:]), rtol=1e-5, atol=1e-6)


def test_gqa_equals_repeated_kv_heads(oracle):
    q, qg, kc, vc = _rand_attn(8, 2, 8, 2, 64, 30)
    grouped = oracle.attention(q, kc, vc, 28, qg)
    rep = oracle.attention(q, np.repeat(kc, 4, axis=1), np.repeat(vc, 4, axis=1), 28, qg)
    assert np.array_equal(grouped, rep)


def test_causality(oracle):
    """Token t only sees keys < pos + t + 1: changing later rows leaves it unchanged."""
    q, qg, kc, vc = _rand_attn(9, 3, 4, 1, 64, 23)
    out = oracle.attention(q, kc, vc, 20, qg)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[21:], vc2[21:] = 9.0, -9.0
    out2 = oracle.attention(q, kc2, vc2, 20, qg)
    assert np.array_equal(out[0], out2[0])
    assert not np.allclose(out[2], out2[2])


def test_fp64_brute_force(oracle):
    for (NH, NKV, D, rows, n) in [(4, 1, 64, 129, 1), (16, 2, 256, 700, 4), (2, 1, 256, 40, 3)]:
        q, qg, kc, vc = _rand_attn(10 + rows, n, NH, NKV, D, rows)
        pos = rows - n
        out = oracle.attention(q, kc, vc, pos, qg)
        ref = oracle.attention_f64(q, kc, vc, pos, qg)
        assert np.abs(out - ref).max() <= 2e-6


@pytest.mark.parametrize("chunk", [1, 5, 32, 64, 100, 1000])
def test_split_merge_equals_two_pass(oracle, chunk):
    """The split-K online softmax + log-sum-exp merge (attention.comp + attn_combine.comp semantics),
    including splits that are empty for the earlier tokens, equals the two-pass softmax."""
    q, qg, kc, vc = _rand_attn(11, 4, 8, 2, 64, 260)
    out = oracle.attention_split(q, kc, vc, 256, chunk, qg)
    ref = oracle.attention(q, kc, vc, 256, qg)
    assert np.abs(out - ref).max() <= 2e-6


def test_peaked_softmax_range(oracle):
    """1% of keys x8 (BASELINE config 5's stress) stays finite and matches fp64."""
    s = QWEN3_NEXT
    k16, v16 = cache_rows(12, 3000, s, heavy_frac=0.01)
    r = np.random.default_rng(13)
    q = r.standard_normal((1, s.NH, s.D)).astype(np.float32)
    qg = r.standard_normal((1, s.NH, 2 * s.D)).astype(np.float32)
    out = oracle.attention(q, k16.astype(np.float32), v16.astype(np.float32), 2999, qg)
    ref = oracle.attention_f64(q, k16.astype(np.float32), v16.astype(np.float32), 2999, qg)
    # scores reach ~30 here, so the fp32 exponent carries ~1e-6 relative error
    assert np.isfinite(out).all() and np.abs(out - ref).max() <= 1e-5


# ---- golden fixtures ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["c1_tiny", "gguf_tiny", "qwen3next"])
def test_golden_fixture(oracle, name):
    f = np.load(os.path.join(GOLDEN, f"attn_{name}.npz"))
    NH, NKV, D, R, pos, n = (int(v) for v in f["dims"])
    theta, eps = float(f["theta"]), float(f["eps"])
    q_out, kc, vc = oracle.qk_norm_rope(f["qg"], f["k"], f["v"], 1 + f["wq"], 1 + f["wk"], pos, R, theta, eps)
    assert np.abs(q_out - f["q_out"]).max() <= 1e-5
    assert np.abs(kc[pos:] - f["k_new"]).max() <= 1e-5
    assert np.array_equal(vc[pos:], f["v"])
    kc[:pos], vc[:pos] = f["kc0"].astype(np.float32), f["vc0"].astype(np.float32)
    out = oracle.attention(q_out, kc, vc, pos, f["qg"])
    assert np.abs(out - f["out"]).max() <= 1e-5


def _hf():
    path = os.path.join(GOLDEN, "hf_qwen3next_attn.npz")
    return np.load(path)


def test_hf_qwen3next_fixture(oracle):
    f = _hf()
    NH, NKV, D, R, T = (int(v) for v in f["dims"])
    q_out, kc, vc = oracle.qk_norm_rope(f["qg"], f["k"], f["v"], 1 + f["wq"], 1 + f["wk"], 0, R, float(f["theta"]),
                                        float(f["eps"]))
    out = oracle.attention(q_out, kc, vc, 0, f["qg"])
    assert np.abs(out - f["out"]).max() <= 2e-5


def _np_attention(qg, k, v, wq, wk, R, theta, eps, rope="half", one_plus=True, group="block", causal=True):
    """A deliberately configurable numpy attention, for the planted-mistake checks."""
    T, NH, D2 = qg.shape
    D = D2 // 2
    NKV = k.shape[1]
    G = NH // NKV
    inv = np.array([1.0 / theta ** (2.0 * i / R) for i in range(R // 2)])

    def nr(x, w, p):
        y = x / np.sqrt(np.mean(x * x) + eps) * ((1 + w) if one_plus else w)
        a = p * inv
        if rope == "half":
            lo, hi = y[:R // 2].copy(), y[R // 2:R].copy()
            y[:R // 2], y[R // 2:R] = lo * np.cos(a) - hi * np.sin(a), hi * np.cos(a) + lo * np.sin(a)
        else:  # interleaved pairs (2i, 2i+1)
            ev, od = y[0:R:2].copy(), y[1:R:2].copy()
            y[0:R:2], y[1:R:2] = ev * np.cos(a) - od * np.sin(a), od * np.cos(a) + ev * np.sin(a)
        return y

    Q = np.stack([[nr(qg[t, h, :D], wq, t) for h in range(NH)] for t in range(T)])
    K = np.stack([[nr(k[t, h], wk, t) for h in range(NKV)] for t in range(T)])
    out = np.zeros((T, NH, D))
    for t in range(T):
        L = t + 1 if causal else T
        for h in range(NH):
            kh = h // G if group == "block" else h % NKV
            s = K[:L, kh] @ Q[t, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            out[t, h] = (p[:, None] * v[:L, kh]).sum(0) / p.sum() / (1 + np.exp(-qg[t, h, D:]))
    return out


def test_hf_fixture_catches_planted_mistakes():
    f = _hf()
    NH, NKV, D, R, T = (int(v) for v in f["dims"])
    args = (f["qg"], f["k"], f["v"], f["wq"], f["wk"], R, float(f["theta"]), float(f["eps"]))
    assert np.abs(_np_attention(*args) - f["out"]).max() <= 2e-5
    for wrong in ({"rope": "interleaved"}, {"one_plus": False}, {"group": "interleaved"}, {"causal": False}):
        assert np.abs(_np_attention(*args, **wrong) - f["out"]).max() > 1e-2, wrong


# ---- the reference's own compiled primitives ----------------------------------------------------------------

def _ref():
    import oracle as orc
    try:
        return orc.RefPrimitives()
    except (FileNotFoundError, OSError):
        pytest.skip("oracle/_ref/libref.so not built (needs /root/reference)")


def test_ref_primitives_agree():
    ref = _ref()
    import oracle as orc
    o = orc.Oracle()
    r = np.random.default_rng(14)
    for n in (32, 64, 256):
        a, b = r.standard_normal(n).astype(np.float32), r.standard_normal(n).astype(np.float32)
        assert abs(ref.dot(a, b) - o.dot(a, b)) <= 1e-5 * (1 + np.abs(a * b).sum())
    x = r.standard_normal(256).astype(np.float32)
    w = (0.1 * r.standard_normal(256)).astype(np.float32)
    assert np.allclose(ref.rmsnorm_one_plus(x, w, 1e-6), o.rmsnorm_one_plus(x, w, 1e-6), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("shape,rows,n", [(TINY, 129, 1), (QWEN3_NEXT, 2000, 4)])
def test_ref_attention_agrees(oracle, shape, rows, n):
    ref = _ref()
    q, qg, kc, vc = _rand_attn(15, n, shape.NH, shape.NKV, shape.D, rows)
    a = ref.attention(q, kc, vc, rows - n, qg)
    b = oracle.attention(q, kc, vc, rows - n, qg)
    assert np.abs(a - b).max() <= 1e-6


def test_qk_norm_rope_matches_projection_pipeline(oracle):
    """oracle.qk_norm_rope = rms_mul + rope per head, cache rows at pos.."""
    s = TINY
    qg, k, v, qn, kn = projections(16, 3, s)
    q_out, kc, vc = oracle.qk_norm_rope(qg, k, v, 1 + qn, 1 + kn, 10, s.R, s.theta, s.eps)
    for t in range(3):
        for h in range(s.NH):
            exp = oracle.rope(oracle.rms_mul(qg[t, h, :s.D], 1 + qn, s.eps), 10 + t, s.R, s.theta)
            assert np.array_equal(q_out[t, h], exp)
        assert np.array_equal(vc[10 + t], v[t])
    assert not kc[:10].any()
