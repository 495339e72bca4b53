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


# ---- QSA indexer and block-sparse attention (src/qwen4_qsa.h, shaders/attention.comp:35-43) ----------------

from common import QSA_BLOCK64, QSA_ODD, QSA_TINY, QSA_WIDE, qsa_inputs, qsa_oracle_run  # noqa: E402


def _ref_qsa():
    import oracle as orc
    try:
        return orc.RefQsa()
    except (FileNotFoundError, OSError):
        pytest.skip("oracle/_ref/libref_qsa.so not built (needs /root/reference)")


QSA_CALLS = {
    # a prefill chunk, decode steps, a 4-token verify pass, then a rollback: the pass is redone at the
    # smaller position (rows and blocks past it are rewritten, src/qwen4_vk.cpp:286-300)
    "tiny": (QSA_TINY, 256, [(0, 40), (40, 1), (41, 1), (42, 4), (44, 4), (48, 1), (49, 3)]),
    "wide": (QSA_WIDE, 8192, [(0, 3000), (3000, 1), (3001, 4), (3003, 4), (3007, 1), (3008, 64)]),
    "block64": (QSA_BLOCK64, 8192, [(0, 2000), (2000, 1), (2001, 100), (2101, 4), (2103, 1)]),
    "odd": (QSA_ODD, 1024, [(0, 100), (100, 1), (101, 4), (103, 2), (105, 50)]),
}


@pytest.mark.parametrize("name", list(QSA_CALLS))
def test_qsa_selection_matches_reference(oracle, name):
    """The oracle's indexer selects exactly the blocks the reference's own QsaIndexer selects (compiled in
    place: oracle/_ref/libref_qsa.so), over prefill chunks, decode steps, verify passes and a rollback."""
    ref = _ref_qsa()
    qs, max_ctx, calls = QSA_CALLS[name]
    tot = sum(c[1] for c in calls)
    iq, ik, qg, kg = qsa_inputs(31, tot, qs)
    mw = qs.mask_words(max_ctx)
    want = ref.run(calls, iq, ik, qg, kg, qs.CR, qs.budget, qs.R, qs.theta, qs.eps, max_ctx, mw)
    got, _, _ = qsa_oracle_run(oracle, calls, iq, ik, qg, kg, qs, max_ctx)
    assert np.array_equal(got, want)
    # the selecting tokens pick exactly budget / CR blocks
    row = 0
    for pos, n in calls:
        for t in range(n):
            if (pos + t + 1) // qs.CR > qs.top:
                assert sum(bin(int(w)).count("1") for w in got[row + t]) == qs.top
        row += n


def test_qsa_pool_closed_forms(oracle):
    """A block of identical raw keys pools to that key, normed (gamma as stored) and rotated to the block's
    first position; the first block is not rotated; pooling is the mean (order-free up to rounding)."""
    qs = QSA_WIDE
    r = np.random.default_rng(32)
    g = (1 + 0.1 * r.standard_normal(qs.ID)).astype(np.float32)
    x = r.standard_normal(qs.ID).astype(np.float32)
    raw = np.tile(x, (4 * qs.CR, 1))
    pooled = oracle.qsa_pool(raw, g, 0, 4, qs.CR, qs.R, qs.theta, qs.eps)
    normed = oracle.rms_mul(x, g, qs.eps)
    assert np.allclose(pooled[0], normed, rtol=1e-5, atol=1e-6)  # block 0: position 0, no rotation
    for b in range(1, 4):
        assert np.allclose(pooled[b], oracle.rope(normed, b * qs.CR, qs.R, qs.theta), rtol=1e-5, atol=1e-5)
    raw = r.standard_normal((qs.CR, qs.ID)).astype(np.float32)
    mean = raw.astype(np.float64).mean(axis=0)
    exp = mean / np.sqrt(np.mean(mean ** 2) + qs.eps) * g
    p0 = oracle.qsa_pool(raw, g, 0, 1, qs.CR, qs.R, qs.theta, qs.eps)[0]
    assert np.allclose(p0, exp, rtol=1e-5, atol=1e-6)
    p1 = oracle.qsa_pool(raw[::-1].copy(), g, 0, 1, qs.CR, qs.R, qs.theta, qs.eps)[0]
    assert np.allclose(p0, p1, rtol=1e-5, atol=1e-6)


def test_qsa_select_brute_force(oracle):
    """Selection = the budget/CR blocks with the largest fp64 score sum_h relu(q_h . k_b), where the k-th
    and (k+1)-th scores are apart; all-zero scores fall back to the lowest block ids; tokens that see at
    most budget/CR complete blocks select nothing (all-ones row)."""
    qs = QSA_TINY
    r = np.random.default_rng(33)
    nblk_max, pos, n = 60, 200, 3
    pooled = r.standard_normal((nblk_max, qs.ID)).astype(np.float32)
    iq = r.standard_normal((n, qs.IH, qs.ID)).astype(np.float32)
    g = np.ones(qs.ID, np.float32)
    mw = 2
    mask, scores = oracle.qsa_select(iq, g, pooled, pos, qs.CR, qs.top, qs.R, qs.theta, qs.eps, mw, with_scores=True)
    for t in range(n):
        p = pos + t
        nblk = (p + 1) // qs.CR
        q = np.stack([oracle.rope(oracle.rms_mul(iq[t, h], g, qs.eps), p, qs.R, qs.theta) for h in range(qs.IH)])
        s64 = np.maximum(0, q.astype(np.float64) @ pooled[:nblk].astype(np.float64).T).sum(axis=0)
        assert np.allclose(scores[t, :nblk], s64, rtol=1e-5, atol=1e-5)
        order = sorted(range(nblk), key=lambda b: (-s64[b], b))
        sel = {b for b in range(nblk) if (int(mask[t, b >> 5]) >> (b & 31)) & 1}
        assert len(sel) == qs.top
        gap = s64[order[qs.top - 1]] - s64[order[qs.top]]
        if gap > 1e-4:
            assert sel == set(order[:qs.top])
    # every score zero (queries opposite to every pooled key): the lowest ids win the ties
    neg = -np.abs(r.standard_normal((nblk_max, qs.ID))).astype(np.float32)
    pos_q = np.abs(r.standard_normal((1, qs.IH, qs.ID))).astype(np.float32)
    m0 = oracle.qsa_select(pos_q, g, neg, 100, qs.CR, qs.top, 0, qs.theta, qs.eps, mw)  # R = 0: no rotation
    sel = [b for b in range(64) if (int(m0[0, b >> 5]) >> (b & 31)) & 1]
    assert sel == list(range(qs.top))
    # not enough complete blocks yet: dense
    md = oracle.qsa_select(iq[:1], g, pooled, qs.top * qs.CR - 1, qs.CR, qs.top, qs.R, qs.theta, qs.eps, mw)
    assert np.all(md == 0xFFFFFFFF)


@pytest.mark.parametrize("cr", [3, 4, 64])
def test_attention_qsa_equals_attention_over_visible_keys(oracle, cr):
    """Masked attention equals plain causal attention over a cache that holds only the visible keys (the
    selected complete blocks, then the tail block), and with an all-ones mask it equals dense attention."""
    NH, NKV, D, pos, n = 4, 2, 64, 700, 4
    q, qg, kc, vc = _rand_attn(34, n, NH, NKV, D, pos + n)
    r = np.random.default_rng(35)
    mw = (pos + n) // cr // 32 + 1
    mask = r.integers(0, 2 ** 32, size=(n, mw), dtype=np.uint64).astype(np.uint32) & np.uint32(0x5A5A33CC)
    out = oracle.attention_qsa(q, kc, vc, pos, mask, cr, qg)
    for t in range(n):
        ln = pos + t + 1
        tail = ln // cr * cr
        keys = [j for j in range(ln) if j >= tail or (int(mask[t, (j // cr) >> 5]) >> ((j // cr) & 31)) & 1]
        exp = oracle.attention(q[t:t + 1], kc[keys], vc[keys], len(keys) - 1, qg[t:t + 1])
        assert np.abs(out[t] - exp[0]).max() <= 2e-6
    full = np.full((n, mw), 0xFFFFFFFF, np.uint32)
    assert np.abs(oracle.attention_qsa(q, kc, vc, pos, full, cr, qg) - oracle.attention(q, kc, vc, pos, qg)).max() <= 1e-6


def test_qsa_key_bits():
    """qsa_key_bits, checked key by key against the rule of shaders/attention.comp:35-43."""
    import oracle as orc
    r = np.random.default_rng(36)
    for cr, pos, n in [(4, 100, 3), (3, 61, 4), (64, 700, 2), (32, 95, 1)]:
        mw = (pos + n) // cr // 32 + 1
        mask = r.integers(0, 2 ** 32, size=(n, mw), dtype=np.uint64).astype(np.uint32)
        bits = orc.qsa_key_bits(mask, pos, n, cr)
        assert bits.shape == (n, (pos + n + 31) // 32)
        for t in range(n):
            tail = (pos + t + 1) // cr * cr
            for j in range(pos + n):
                b = j // cr
                vis = j >= tail or (int(mask[t, b >> 5]) >> (b & 31)) & 1 == 1
                assert ((int(bits[t, j >> 5]) >> (j & 31)) & 1) == int(vis), (cr, t, j)


# ---- projections (Qwen4Vulkan::mat, shaders/q4_matmul.comp C_Q8 / C_F32) ------------------------------------

from common import q8_blocks  # noqa: E402


@pytest.mark.parametrize("rows,cols,n", [(96, 256, 1), (64, 2048, 3), (40, 4096, 8)])
def test_mat_q8_matches_reference(oracle, rows, cols, n):
    """The oracle's planar-Q8 projection equals the reference's own CPU projection (gq::run_jobs over the same
    GGUF Q8_0 blocks, src/quant.cpp, compiled in place) to fp32 rounding: the planar form (int8 weights, f16
    scales widened) loses nothing, and each output is one dot product."""
    ref = _ref_qsa()
    blocks, w8, s = q8_blocks(51 + n, rows, cols)
    x = np.random.default_rng(52).standard_normal((n, cols)).astype(np.float32)
    got = oracle.mat(x, w8=w8, s=s)
    want = ref.mat_q8(blocks, rows, cols, x)
    mag = np.abs(w8.astype(np.float64) * np.repeat(s, 32, axis=1)) @ np.abs(x.astype(np.float64)).T  # [rows, n]
    assert np.all(np.abs(got - want) <= 1e-6 * mag.T + 1e-7), np.abs(got - want).max()


def test_mat_q8_exponent31_scales_match_reference(oracle, qw):
    """Q8_0 blocks whose binary16 scale has exponent 31 (0x7C00, 0x7FFF, 0xFE01, 0x7C01: inf / NaN in IEEE,
    finite 65536, 131008, -98368, 65600 in the reference's ck::half_to_f32), repacked by qwattn_q8_unpack and
    multiplied by the oracle, give what the reference's GPU path computes from its upload (unpack_q8_row,
    src/qwen4_vk.cpp:98-106, which widens with half_to_f32): an fp64 product over the reference's own compiled
    half_to_f32 of each pattern. Rows without such a scale also equal the reference's CPU projection
    (gq::run_jobs). That CPU path widens scales with F16C on AVX-512 hosts (src/quant.cpp:17-25), i.e. IEEE
    inf / NaN, so the reference's CPU and GPU paths disagree on exactly these rows; this build follows the GPU
    upload it replaces."""
    ref = _ref_qsa()
    prim = _ref()
    rows, cols, n = 24, 256, 2
    blocks, w8, _ = q8_blocks(57, rows, cols)
    b = blocks.reshape(rows, cols // 32, 34).copy()
    hot = np.array([0x7C00, 0x7FFF, 0xFE01, 0x7C01], np.uint16)
    hot_rows = np.arange(rows) % 3 == 0
    for r in np.nonzero(hot_rows)[0]:
        b[r, r % (cols // 32), 0:2] = hot[r % 4:r % 4 + 1].view(np.uint8)
    bits = b[:, :, 0:2].copy().view(np.uint16)[:, :, 0]
    b = b.reshape(rows, -1)
    w, s = qw.q8_unpack(b, rows, cols)
    want_s = np.array([[prim.lib.ref_half_to_f32(int(h)) for h in row] for row in bits], np.float32)
    assert np.array_equal(w, w8) and np.array_equal(s.view(np.uint32), want_s.view(np.uint32))
    assert s.max() == 131008.0 and s.min() == -98368.0
    x = np.random.default_rng(58).standard_normal((n, cols)).astype(np.float32)
    got = oracle.mat(x, w8=w, s=s)
    wf = w8.astype(np.float64) * np.repeat(want_s.astype(np.float64), 32, axis=1)
    exact = x.astype(np.float64) @ wf.T
    mag = np.abs(wf) @ np.abs(x.astype(np.float64)).T
    assert np.all(np.abs(got - exact) <= 1e-6 * mag.T + 1e-7), np.abs(got - exact).max()
    cpu = ref.mat_q8(b, rows, cols, x)
    assert np.all(np.abs(got - cpu)[:, ~hot_rows] <= 1e-6 * mag.T[:, ~hot_rows] + 1e-7)


def test_mat_closed_forms(oracle):
    """f32 identity and permutation matrices return x (permuted); zero weights return 0; a Q8 row of k with
    scale 1/k sums x; post 1 is silu(y * scale) of the plain result; the product is linear in x."""
    r = np.random.default_rng(53)
    n, cols = 3, 64
    x = r.standard_normal((n, cols)).astype(np.float32)
    assert np.array_equal(oracle.mat(x, wf=np.eye(cols, dtype=np.float32)), x)
    perm = r.permutation(cols)
    assert np.array_equal(oracle.mat(x, wf=np.eye(cols, dtype=np.float32)[perm]), x[:, perm])
    assert not np.any(oracle.mat(x, wf=np.zeros((5, cols), np.float32)))
    w8 = np.full((2, cols), 8, np.int8)
    s = np.full((2, cols // 32), 0.125, np.float32)
    assert np.allclose(oracle.mat(x, w8=w8, s=s), np.repeat(x.sum(axis=1, keepdims=True), 2, axis=1), atol=1e-5)
    wf = r.standard_normal((7, cols)).astype(np.float32)
    y = oracle.mat(x, wf=wf)
    u = y * 0.7
    assert np.allclose(oracle.mat(x, wf=wf, post=1, post_scale=0.7), u / (1 + np.exp(-u)), rtol=1e-6, atol=1e-7)
    x2 = r.standard_normal((n, cols)).astype(np.float32)
    assert np.allclose(oracle.mat(2 * x - x2, wf=wf), 2 * y - oracle.mat(x2, wf=wf), rtol=1e-5, atol=1e-5)


def test_fp16_cache_cost_against_fp32_cache(oracle):
    """The FP8 model's Vulkan path keeps fp32 K/V caches (src/vk_backend.cpp:297-299, 584-610; the CPU paths
    too, src/qwen4_cpu.cpp:318-319); this build serves every model with fp16 caches. The cost, on the oracle
    at the Qwen3-Next shape over 4,097 keys: with N(0,1) cache rows the outputs from fp16-rounded rows differ
    from fp32 rows by a relative 3e-4 (max-abs ~2e-5); with 1% of the keys x8 (the long-context config's
    stress) by a relative 4e-4, max-abs ~3e-3 on outputs of magnitude up to ~3.4, i.e. ~1e-3 of the output
    scale. The check also sees that the difference is more than fp32 rounding."""
    from common import QWEN3_NEXT as s
    for heavy, rel_max, scaled_max in ((0, 1e-3, 1e-3), (8, 1e-3, 2e-3)):
        r = np.random.default_rng(77)
        pos, n = 4096, 4
        qg = r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32)
        k = r.standard_normal((pos + n, s.NKV, s.D)).astype(np.float32)
        v = r.standard_normal((pos + n, s.NKV, s.D)).astype(np.float32)
        if heavy:
            k[r.choice(pos, pos // 100, replace=False)] *= heavy
        qn = (1 + 0.1 * r.standard_normal(s.D)).astype(np.float32)
        kn = (1 + 0.1 * r.standard_normal(s.D)).astype(np.float32)
        rq, rk, rv = oracle.qk_norm_rope(qg, k[pos:], v[pos:], qn, kn, pos, s.R, s.theta, s.eps)
        kc, vc = k.copy(), v.copy()
        kc[pos:], vc[pos:] = rk[pos:], rv[pos:]
        full = oracle.attention(rq, kc, vc, pos, qg)
        half = oracle.attention(rq, kc.astype(np.float16).astype(np.float32), vc.astype(np.float16).astype(np.float32),
                                pos, qg)
        d = np.abs(full - half)
        rel = float(np.linalg.norm(full - half) / np.linalg.norm(full))
        print(f"fp16 vs fp32 cache (keys x{heavy or 1}): max-abs {d.max():.2e}, rel-l2 {rel:.2e}, "
              f"max |out| {np.abs(full).max():.2f}")
        assert rel < rel_max and d.max() < scaled_max * np.abs(full).max()
        assert d.max() > 1e-6
