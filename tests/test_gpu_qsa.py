"""QSA block-sparse attention on the GPU against the CPU oracle (oracle/, pinned to the reference's own
QsaIndexer in tests/test_oracle.py).

Indexer: the pooled block keys agree with the oracle's to fp32 rounding (rtol 1e-5); the selection is the
oracle's exactly, except where the oracle's own scores put the budget boundary within float rounding of a
tie (|score - threshold| <= 1e-5 * (1 + threshold)): there a block may swap with its near-equal neighbour,
and the test checks that only such blocks differ. Zero scores (all heads' dots negative) tie exactly on
both sides and fall back to the lower block ids: the cases whose threshold is 0 allow no swap (zero
queries) or at most two (a near-zero dot whose sign rounding flips), where a wrong tie order would swap
thousands.
"""
import numpy as np
import pytest
import torch

from common import QSA_BLOCK64, QSA_ODD, QSA_TINY, QSA_WIDE, QWEN3_NEXT, QsaShape, assert_rows_parity, qsa_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def host(t):
    t = t.detach()
    return (t.float() if t.dtype in (torch.bfloat16, torch.float16) else t).cpu().numpy()


def _ctx(qw, max_ctx, max_tokens=4096, R=64):
    s = QWEN3_NEXT
    return qw.Attention(s.NH, s.NKV, s.D, R, s.theta, s.eps, max_ctx=max_ctx, max_tokens=max_tokens, max_splits=256)


def _bits(m, b):
    return (int(m[b >> 5]) >> (b & 31)) & 1


def assert_selection(got, want, scores, qs, pos, n, what):
    """got/want [n, mask_words] uint32; scores [n, nblk] from the oracle (NaN for dense tokens). Returns the
    number of near-tie swaps the comparison allowed (blocks selected on one side only)."""
    swaps = 0
    for t in range(n):
        nblk = (pos + t + 1) // qs.CR
        if nblk <= qs.top:
            assert np.all(got[t] == 0xFFFFFFFF), f"{what}: token {t} should be dense"
            continue
        if np.array_equal(got[t], want[t]):
            continue
        s = scores[t, :nblk].astype(np.float64)
        thr = np.sort(s)[::-1][qs.top - 1]
        tol = 1e-5 * (1 + thr)
        g = {b for b in range(nblk) if _bits(got[t], b)}
        w = {b for b in range(nblk) if _bits(want[t], b)}
        assert len(g) == qs.top, f"{what}: token {t} selected {len(g)} blocks"
        for b in g ^ w:
            assert abs(s[b] - thr) <= tol, f"{what}: token {t} block {b} score {s[b]} vs threshold {thr}"
        swaps += len(g ^ w) // 2
        assert not np.any(got[t, (nblk + 31) // 32:]), f"{what}: token {t} bits past its complete blocks"
    return swaps


# (pos, n, select): indexer calls in order (select False: keys cached and pooled only, as for a long prompt
# whose selection is not under test)
CASES = {
    "tiny": (QSA_TINY, 256, [(0, 40, 1), (40, 1, 1), (41, 1, 1), (42, 4, 1), (44, 4, 1), (48, 1, 1), (49, 3, 1)], "f32"),
    "wide": (QSA_WIDE, 8192, [(0, 3000, 1), (3000, 1, 1), (3001, 4, 1), (3003, 4, 1), (3007, 1, 1), (3008, 64, 1)],
             "f32"),
    "block64": (QSA_BLOCK64, 8192, [(0, 2000, 1), (2000, 1, 1), (2001, 100, 1), (2101, 4, 1), (2103, 1, 1)], "bf16"),
    "odd": (QSA_ODD, 1024, [(0, 100, 1), (100, 1, 1), (101, 4, 1), (103, 2, 1), (105, 50, 1)], "f32"),
    # 131,000+ blocks: the select reads the scores from memory at each use, and 40 tokens take two select launches
    "long_cr2": (QsaShape(1, 64, 2, 64, 64), 262144, [(0, 262000, 0), (262000, 40, 1)], "f32"),
    # 8,192 blocks at 32K: 8 keys a select thread
    "cr4_32k": (QsaShape(4, 128, 4, 2048, 64), 32776, [(0, 32768, 0), (32768, 1, 1), (32769, 4, 1)], "f32"),
    # 16,384 / 32,768 / 65,536 blocks: 16, 32 and 64 keys a select thread
    "cr4_64k": (QsaShape(4, 128, 4, 2048, 64), 65544, [(0, 65536, 0), (65536, 1, 1), (65537, 2, 1)], "f32"),
    "cr2_64k": (QsaShape(2, 64, 2, 512, 64), 65544, [(0, 65536, 0), (65536, 1, 1), (65537, 3, 1)], "f32"),
    "cr4_256k": (QsaShape(1, 64, 4, 1024, 64), 262152, [(0, 262144, 0), (262144, 1, 1), (262145, 2, 1)], "f32"),
    # zero indexer queries: every score is 0, the lowest block ids win (no histogram pass at all)
    "zeros": (QsaShape(2, 128, 4, 256, 64), 8200, [(0, 8000, 0), (8000, 2, 1), (8002, 1, 1)], "f32"),
    # the same at 1,000 blocks (scoring and selection in one launch) and past 32,768 (a scoring launch, then
    # the spread selection launch)
    "zeros_cr8": (QsaShape(2, 128, 8, 8 * 64, 64), 8200, [(0, 8000, 0), (8000, 2, 1)], "f32"),
    "zeros_cr2_64k": (QsaShape(2, 64, 2, 512, 64), 65560, [(0, 65544, 0), (65544, 2, 1)], "f32"),
    # one indexer head: about half the blocks score exactly 0 (a negative dot), and the budget reaches into
    # them, so the threshold is 0 and only part of its ties are taken, lowest block ids first; in the
    # one-workgroup select, the one-launch select, the two-launch select and the one that reads the scores
    # from memory
    "halfzero_cr8": (QsaShape(1, 64, 8, 8 * 600, 64), 8200, [(0, 8000, 0), (8000, 2, 1)], "f32"),
    "halfzero_cr4_8k": (QsaShape(1, 64, 4, 4 * 1500, 64), 8200, [(0, 8000, 0), (8000, 2, 1)], "f32"),
    "halfzero_cr2_64k": (QsaShape(1, 64, 2, 2 * 24000, 64), 65560, [(0, 65544, 0), (65544, 2, 1)], "f32"),
    "halfzero_long_cr2": (QsaShape(1, 64, 2, 2 * 70000, 64), 262144, [(0, 262000, 0), (262000, 2, 1)], "f32"),
    # raw keys repeating every `period` blocks and queries zero on the rotated dims: every score value recurs
    # on many blocks, exactly, so the threshold's ties are cut by block id among the compacted candidates
    "ties_cr8": (QsaShape(2, 128, 8, 8 * 100, 64), 8200, [(0, 8000, 0), (8000, 2, 1)], "f32"),
    "ties_cr4_8k": (QsaShape(2, 128, 4, 4 * 300, 64), 8200, [(0, 8000, 0), (8000, 2, 1), (8002, 1, 1)], "f32"),
    "ties_cr2_64k": (QsaShape(1, 128, 2, 2 * 5000, 64), 65560, [(0, 65544, 0), (65544, 2, 1)], "f32"),
    "ties_long_cr2": (QsaShape(1, 128, 2, 2 * 9000, 64), 262144, [(0, 262000, 0), (262000, 2, 1)], "f32"),
}
TIE_PERIOD = {"ties_cr8": 37, "ties_cr4_8k": 37, "ties_cr2_64k": 101, "ties_long_cr2": 1009}  # blocks


@pytest.mark.parametrize("name", list(CASES))
def test_qsa_indexer_matches_oracle(qw, oracle, name):
    _indexer_case(qw, oracle, name, *CASES[name])


def test_qsa_select_widest_indexer_after_narrow(qw, oracle):
    """The select's dynamic LDS grows with heads x dims; a call at the widest indexer the host accepts
    (32 heads x 256 dims = 8,192) right after a narrow one in the same process launches and selects the
    oracle's blocks."""
    _indexer_case(qw, oracle, "tiny", *CASES["tiny"])
    _indexer_case(qw, oracle, "heads32_dims256", QsaShape(32, 256, 4, 256, 64), 2056,
                  [(0, 2000, 0), (2000, 1, 1), (2001, 3, 1)], "f32")


def _indexer_case(qw, oracle, name, qs, max_ctx, calls, dt):
    import oracle as orc
    tot = sum(c[1] for c in calls)
    iq, ik, qg, kg = qsa_inputs(41, tot, qs)
    if name.startswith("zeros"):
        iq[:] = 0.0
    if name in TIE_PERIOD:
        rows = TIE_PERIOD[name] * qs.CR
        ik = np.ascontiguousarray(np.tile(ik[:rows], (-(-len(ik) // rows), 1))[:len(ik)])
        iq[..., :qs.R] = 0.0
    if dt == "bf16":  # the oracle reads the same bf16-rounded values
        iq = torch.from_numpy(iq).bfloat16().float().numpy()
        ik = torch.from_numpy(ik).bfloat16().float().numpy()
    tdt = torch.float32 if dt == "f32" else torch.bfloat16
    ctx = _ctx(qw, max_ctx, R=qs.R)
    mw = qs.mask_words(max_ctx)
    raw = torch.zeros((max_ctx, qs.ID), device=DEV)
    pooled = torch.full((max_ctx // qs.CR + 1, qs.ID), float("nan"), device=DEV)
    raw_ref = np.zeros((max_ctx, qs.ID), np.float32)
    pooled_ref = np.zeros((max_ctx // qs.CR + 1, qs.ID), np.float32)
    qg_d, kg_d = dev(qg), dev(kg)
    row = 0
    for pos, n, sel in calls:
        print(f"qsa {name}: pos={pos} n={n} select={sel}", flush=True)
        ik_d = dev(ik[row:row + n]).to(tdt)
        ctx.qsa_pool(ik_d, kg_d, qs.CR, raw, pooled, max_ctx, pos, n)
        raw_ref[pos:pos + n] = ik[row:row + n]
        oracle.qsa_pool(raw_ref, kg, pos // qs.CR, (pos + n) // qs.CR, qs.CR, qs.R, qs.theta, qs.eps, pooled_ref)
        nb = (pos + n) // qs.CR
        torch.cuda.synchronize()
        assert np.allclose(host(pooled[:nb]), pooled_ref[:nb], rtol=1e-5, atol=1e-5)
        if sel:
            iq_d = dev(iq[row:row + n]).to(tdt)
            mask = torch.full((n, mw), -1, dtype=torch.int32, device=DEV)
            kw = (pos + n + 31) // 32
            kbits = torch.full((n, kw), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
            ctx.qsa_select(iq_d, qg_d, qs.CR, qs.budget, pooled, pos, n, mask, kbits)
            ctx.sync_status()
            got = host(mask).view(np.uint32)
            want, scores = oracle.qsa_select(iq[row:row + n], qg, pooled_ref, pos, qs.CR, qs.top, qs.R, qs.theta,
                                             qs.eps, mw, with_scores=True)
            swaps = assert_selection(got, want, scores, qs, pos, n, f"{name} pos={pos}")
            print(f"qsa {name} pos={pos} n={n}: {swaps} near-tie swap(s) of {n * qs.top} selected blocks",
                  flush=True)
            if name.startswith(("zeros", "ties")):  # exact ties on both sides: block order alone decides
                assert swaps == 0
            # thousands of exact zeros at the threshold (halfzero): at most a sign flip or two; random scores: a
            # near-tie at the budget boundary is rare (a few blocks lie within 1e-5 of it at 65,536 blocks), so
            # more than two swaps in a call would be a wrong selection, not rounding
            assert swaps <= 2, f"{name} pos={pos}: {swaps} near-tie swaps"
            # the key bits follow the GPU's own selection by the reference's visibility rule
            assert np.array_equal(host(kbits).view(np.uint32), orc.qsa_key_bits(got, pos, n, qs.CR))
        row += n
    # the raw cache holds each position's last written key (passes redone at a smaller pos rewrite it)
    exp = raw_ref
    assert np.array_equal(host(raw), exp)
    ctx.close()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_qsa_index_equals_pool_then_select(qw, dt):
    """qsa_index (one launch when no block completes, the select appending the raw keys) leaves the raw and
    pooled arrays, the mask and the key bits bit for bit as qsa_pool then qsa_select do, over a call sequence
    with and without completed blocks (blocks of 4, 8,192+ of them)."""
    qs = QsaShape(4, 128, 4, 2048, 64)
    max_ctx = 32800
    calls = [(0, 32768, 0), (32768, 1, 1), (32769, 1, 1), (32770, 1, 1), (32771, 1, 1), (32772, 3, 1), (32775, 8, 1)]
    tot = sum(c[1] for c in calls)
    iq, ik, qg, kg = qsa_inputs(57, tot, qs)
    tdt = torch.float32 if dt == "f32" else torch.bfloat16
    ctx = _ctx(qw, max_ctx, R=qs.R)
    mw = qs.mask_words(max_ctx)
    arrs = [(torch.zeros((max_ctx, qs.ID), device=DEV), torch.zeros((max_ctx // qs.CR + 1, qs.ID), device=DEV))
            for _ in range(2)]
    qg_d, kg_d = dev(qg), dev(kg)
    row = 0
    for pos, n, sel in calls:
        print(f"qsa_index {dt}: pos={pos} n={n} completes={(pos + n) // qs.CR != pos // qs.CR}", flush=True)
        ik_d, iq_d = dev(ik[row:row + n]).to(tdt), dev(iq[row:row + n]).to(tdt)
        kw = (pos + n + 31) // 32
        outs = []
        for k, (raw, pooled) in enumerate(arrs):
            mask = torch.full((n, mw), -1, dtype=torch.int32, device=DEV)
            kbits = torch.full((n, kw), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
            if not sel:
                ctx.qsa_pool(ik_d, kg_d, qs.CR, raw, pooled, max_ctx, pos, n)
            elif k == 0:
                ctx.qsa_pool(ik_d, kg_d, qs.CR, raw, pooled, max_ctx, pos, n)
                ctx.qsa_select(iq_d, qg_d, qs.CR, qs.budget, pooled, pos, n, mask, kbits)
            else:
                ctx.qsa_index(ik_d, iq_d, kg_d, qg_d, qs.CR, qs.budget, raw, pooled, max_ctx, pos, n, mask, kbits)
            outs.append((host(mask), host(kbits)))
        ctx.sync_status()
        if sel:
            assert np.array_equal(outs[0][0], outs[1][0]), f"mask at pos {pos}"
            assert np.array_equal(outs[0][1], outs[1][1]), f"key bits at pos {pos}"
        assert np.array_equal(host(arrs[0][0]), host(arrs[1][0])), f"raw keys at pos {pos}"
        assert np.array_equal(host(arrs[0][1]), host(arrs[1][1])), f"pooled keys at pos {pos}"
        row += n
    ctx.close()


def test_qsa_key_bits_from_mask(qw):
    import oracle as orc
    r = np.random.default_rng(42)
    ctx = _ctx(qw, 4096)
    for cr, pos, n in [(4, 1000, 3), (3, 611, 4), (64, 3000, 2), (32, 95, 1), (2, 4000, 8)]:
        mw = (pos + n) // cr // 32 + 1
        mask = r.integers(0, 2 ** 32, size=(n, mw), dtype=np.uint64).astype(np.uint32)
        kw = (pos + n + 31) // 32
        out = torch.zeros((n, kw), dtype=torch.int32, device=DEV)
        ctx.qsa_key_bits(dev(mask.view(np.int32)), cr, pos, n, out)
        ctx.sync_status()
        assert np.array_equal(host(out).view(np.uint32), orc.qsa_key_bits(mask, pos, n, cr)), (cr, pos, n)
    ctx.close()


def test_qsa_select_rejects_bad_shapes(qw):
    ctx = _ctx(qw, 4096)
    qs = QSA_TINY
    iq = torch.zeros((1, qs.IH, qs.ID), device=DEV)
    g = torch.ones(qs.ID, device=DEV)
    pooled = torch.zeros((4096 // qs.CR + 1, qs.ID), device=DEV)
    mask = torch.zeros((1, 1), dtype=torch.int32, device=DEV)  # 32 blocks: too few for 1,000 / 4
    with pytest.raises(qw.QwattnError, match="mask_words"):
        ctx.qsa_select(iq, g, qs.CR, qs.budget, pooled, 999, 1, mask, None)
    with pytest.raises(qw.QwattnError, match="budget"):
        ctx.qsa_select(iq, g, qs.CR, 18, pooled, 10, 1, torch.zeros((1, 8), dtype=torch.int32, device=DEV), None)
    with pytest.raises(qw.QwattnError, match="idx_dim"):
        ctx.qsa_pool(torch.zeros((1, 96), device=DEV), g, qs.CR, torch.zeros((4096, 96), device=DEV), pooled, 4096, 0, 1)
    ctx.close()


# ---- block-sparse attention -------------------------------------------------------------------------------

from common import D128, TINY, TINY_GGUF, assert_parity  # noqa: E402
from test_gpu_kernels import _fused_setup, make_ctx  # noqa: E402


def _rand_mask(seed, pos, n, cr, density, mw=None):
    """A block mask [n, mask_words] with about `density` of each token's complete blocks set."""
    r = np.random.default_rng(seed)
    nmax = (pos + n) // cr
    mw = mw or nmax // 32 + 1
    bits = r.random((n, mw * 32)) < density
    bits[:, nmax:] = False
    return (bits.reshape(n, mw, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)


# (shape, pos, n, n_split, dtype, cr, density)
QSA_DEC = [
    (QWEN3_NEXT, 3000, 1, 0, "f32", 4, 0.1),     # decode: one launch, a few keys per tile
    (QWEN3_NEXT, 32768, 1, 0, "bf16", 64, 0.05),  # the headline shape, blocks of two tiles: most tiles skipped
    (QWEN3_NEXT, 20000, 1, 1, "f32", 8, 0.1),    # one split requested: raised until a workgroup lists <= 256 tiles
    (QWEN3_NEXT, 5000, 4, 0, "f32", 3, 0.2),     # verify: 16-row slices and the combine kernel, blocks across tiles
    (QWEN3_NEXT, 5000, 4, 1, "bf16", 4, 0.1),    # verify, one split requested: raised to <= 64 tiles a chunk
    (TINY, 500, 2, 0, "f32", 4, 0.3),            # two tokens on the loader kernel (G = 4): per-token key words
    (TINY_GGUF, 100, 5, 0, "bf16", 4, 0.25),     # 10 rows at G = 2: 5 tokens in one slice
    (D128, 2000, 8, 0, "bf16", 8, 0.1),          # 32 rows, 8 tokens in two slices
    (QWEN3_NEXT, 700, 1, 0, "f32", 4, 0.0),      # nothing selected: only the tail block is visible
]


@pytest.mark.parametrize("s,pos,n,n_split,dtype,cr,density", QSA_DEC, ids=lambda v: repr(v))
def test_decode_qsa_parity(qw, oracle, s, pos, n, n_split, dtype, cr, density):
    """qwattn_decode_qsa and qwattn_attend_partial_qsa + qwattn_combine against the oracle's masked attention
    (src/qwen4_cpu.cpp:325-372 semantics) on the same fp16 rows; the new rows are appended as in the dense
    path whether or not a token sees them."""
    import oracle as orc
    print(f"qsa decode {s} pos={pos} n={n} split={n_split} {dtype} cr={cr} d={density}", flush=True)
    rows = pos + n
    cap, k16, v16, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, dtype, 700 + pos + n)
    mask = _rand_mask(pos + cr, pos, n, cr, density)
    kbits = dev(orc.qsa_key_bits(mask, pos, n, cr).view(np.int32))
    ctx = make_ctx(qw, s, max_ctx=cap)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    used = ctx.decode_qsa(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, n_split, kbits)
    torch.cuda.synchronize()
    qg_h, k_h, v_h = host(qg_d), host(k_d), host(v_d)
    rq, rk, _ = oracle.qk_norm_rope(qg_h, k_h, v_h, 1 + host(qn_d), 1 + host(kn_d), pos, s.R, s.theta, s.eps)
    krows, vrows = qw.k_rows(kc, cap, s.NKV, s.D), qw.v_rows(vc, cap, s.NKV, s.D)
    assert np.all(np.abs(host(krows[pos:rows]) - rk[pos:rows]) <= np.abs(rk[pos:rows]) * 2.0 ** -10 + 1e-6)
    assert np.array_equal(host(vrows[pos:rows]), v_h.astype(np.float16).astype(np.float32))
    kr, vr = host(krows[:rows]), host(vrows[:rows])
    ref = oracle.attention_qsa(rq, kr, vr, pos, mask, cr, qg_h)
    assert_parity(host(out), ref, f"qsa decode {s} pos={pos} n={n} splits={used}")
    # the per-dispatch form on the same caches (the rows are in place now): normalized query, partials, combine
    q = dev(rq)
    out2 = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    used2 = ctx.attend_partial_qsa(q, kc, vc, cap, pos, n, n_split, kbits)
    ctx.combine(qg_d, out2, n, used2)
    ctx.sync_status()
    assert_parity(host(out2), ref, f"qsa attend_partial {s} pos={pos} n={n} splits={used2}")


@pytest.mark.parametrize("s,pos,n", [(QWEN3_NEXT, 3000, 1), (QWEN3_NEXT, 3001, 4), (TINY, 301, 2)], ids=repr)
def test_decode_qsa_all_visible_equals_dense(qw, s, pos, n):
    """Key bits all set: the masked kernels compute exactly what the dense ones do (same splits, same order)."""
    cap, _, _, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, "f32", 800 + pos)
    kc2, vc2 = kc.clone(), vc.clone()
    ctx = make_ctx(qw, s, max_ctx=cap)
    kbits = torch.full((n, (pos + n + 31) // 32), -1, dtype=torch.int32, device=DEV)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    out2 = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    used = ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, 0)
    used2 = ctx.decode_qsa(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc2, vc2, cap, out2, pos, n, 0, kbits)
    ctx.sync_status()
    assert used == used2
    # bit patterns: the caches hold NaN past their end on purpose
    assert torch.equal(kc.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vc2.view(torch.int16))
    assert torch.equal(out, out2)


def test_qsa_indexer_then_decode(qw, oracle):
    """The whole QSA layer step on the GPU: pool the keys of a 3,000-token history and of one new token,
    select its blocks (budget 512 keys of 3,001), and decode over them; against the oracle's masked attention
    with the GPU's selection (the selection itself is checked against the oracle above)."""
    import oracle as orc
    s, qs = QWEN3_NEXT, QSA_WIDE
    pos, n = 3000, 1
    rows = pos + n
    cap, k16, v16, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, "f32", 901)
    iq, ik, qg_i, kg_i = qsa_inputs(902, rows, qs)
    ctx = make_ctx(qw, s, max_ctx=cap)
    raw = torch.zeros((cap, qs.ID), device=DEV)
    pooled = torch.zeros((cap // qs.CR + 1, qs.ID), device=DEV)
    ctx.qsa_pool(dev(ik[:pos]), dev(kg_i), qs.CR, raw, pooled, cap, 0, pos)
    ctx.qsa_pool(dev(ik[pos:]), dev(kg_i), qs.CR, raw, pooled, cap, pos, n)
    mw = qs.mask_words(cap)
    mask = torch.zeros((n, mw), dtype=torch.int32, device=DEV)
    kbits = torch.zeros((n, (rows + 31) // 32), dtype=torch.int32, device=DEV)
    ctx.qsa_select(dev(iq[pos:]), dev(qg_i), qs.CR, qs.budget, pooled, pos, n, mask, kbits)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    ctx.decode_qsa(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, 0, kbits)
    ctx.sync_status()
    m = host(mask).view(np.uint32)
    assert sum(bin(int(w)).count("1") for w in m[0]) == qs.top
    assert np.array_equal(host(kbits).view(np.uint32), orc.qsa_key_bits(m, pos, n, qs.CR))
    qg_h = host(qg_d)
    rq, _, _ = oracle.qk_norm_rope(qg_h, host(k_d), host(v_d), 1 + host(qn_d), 1 + host(kn_d), pos, s.R, s.theta, s.eps)
    kr = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    vr = host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows])
    ref = oracle.attention_qsa(rq, kr, vr, pos, m, qs.CR, qg_h)
    assert_parity(host(out), ref, "qsa layer step")
    # and it is not the dense result: the selection matters
    dense = oracle.attention(rq, kr, vr, pos, qg_h)
    assert np.abs(ref - dense).max() > 1e-2


# ---- block-sparse prefill ----------------------------------------------------------------------------------

from test_gpu_kernels import capacity, empty_caches, gpu_caches  # noqa: E402
from common import cache_rows, projections  # noqa: E402

# (shape, pos, n, dtype, cr, density, path): "prefill" = qwattn_prefill_qsa (the in-kernel query norm where
# the rope width allows, else the fp16 query buffer), "attend_f32" = norm/rope/append to fp32 queries, then
# qwattn_attend_prefill_qsa
QSA_PF = [
    (QWEN3_NEXT, 1000, 600, "bf16", 4, 0.2, "prefill"),     # paired schedule, keys of 4 over 64-key tiles
    (QWEN3_NEXT, 2048, 2048, "bf16", 64, 0.1, "prefill"),   # the prefill benchmark's shape, whole-tile blocks
    (QWEN3_NEXT, 300, 257, "f32", 3, 0.3, "attend_f32"),    # split schedule, a ratio dividing no tile
    (TINY, 500, 100, "f32", 4, 0.25, "prefill"),            # rope_dim 16: the fp16 query-buffer path
    (D128, 700, 333, "bf16", 8, 0.15, "prefill"),           # D = 128
    (QWEN3_NEXT, 100, 64, "f32", 4, 0.0, "prefill"),        # nothing selected: tails only
]


@pytest.mark.parametrize("s,pos,n,dt,cr,density,path", QSA_PF, ids=lambda v: repr(v))
def test_prefill_qsa_parity(qw, oracle, s, pos, n, dt, cr, density, path):
    import oracle as orc
    print(f"qsa prefill {s} pos={pos} n={n} {dt} cr={cr} d={density} {path}", flush=True)
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(70 + pos, pos, s) if pos else (np.zeros((0, s.NKV, s.D), np.float16),) * 2
    qg, k, v, qn, kn = projections(71 + n, n, s)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    qg_d, k_d, v_d = dev(qg).to(tdt), dev(k).to(tdt), dev(v).to(tdt)
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=max(n, 1))
    kc, vc = gpu_caches(qw, k16, v16, cap) if pos else empty_caches(s, cap)
    mask = _rand_mask(pos + n + cr, pos, n, cr, density)
    kbits = dev(orc.qsa_key_bits(mask, pos, n, cr).view(np.int32))
    rope = ctx.rope_table() if s.R else None
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    if path == "prefill":
        ctx.prefill_qsa(qg_d, k_d, v_d, dev(qn), dev(kn), rope, kc, vc, cap, out, pos, n, kbits)
    else:
        q = torch.zeros((n, s.NH, s.D), device=DEV)
        ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), rope, kc, vc, cap, q, pos, n)
        ctx.attend_prefill_qsa(q, kc, vc, cap, qg_d, out, pos, n, kbits)
    ctx.sync_status()
    rq, _, _ = oracle.qk_norm_rope(host(qg_d), host(k_d), host(v_d), 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
    kcache = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    vcache = host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows])
    qg_h, out = host(qg_d), host(out)
    # every token row, one batched oracle call
    ref = oracle.attention_qsa(rq, kcache, vcache, pos, mask, cr, qg_h)
    assert_rows_parity(out, ref, f"qsa prefill {s} pos={pos} n={n}")


def test_prefill_qsa_all_visible_equals_dense(qw):
    s, pos, n = QWEN3_NEXT, 1500, 700
    cap = capacity(pos + n)
    k16, v16 = cache_rows(81, pos, s)
    qg, k, v, qn, kn = projections(82, n, s)
    qg_d, k_d, v_d = dev(qg).bfloat16(), dev(k).bfloat16(), dev(v).bfloat16()
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=n)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    kc2, vc2 = kc.clone(), vc.clone()
    kbits = torch.full((n, (pos + n + 31) // 32), -1, dtype=torch.int32, device=DEV)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    out2 = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    ctx.prefill(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc, vc, cap, out, pos, n)
    ctx.prefill_qsa(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc2, vc2, cap, out2, pos, n, kbits)
    ctx.sync_status()
    assert torch.equal(out, out2)


def test_layer_attention_qsa(qw, oracle):
    """qwattn_layer_attention_qsa over a prefill chunk, a 4-token verify pass and a decode step of one layer
    slot, each with its own key bits, against the oracle's masked attention on the cache it built."""
    import oracle as orc
    s, cr = QWEN3_NEXT, 8
    ctx = make_ctx(qw, s, max_ctx=4096, max_tokens=1024)
    ctx.kv_alloc(1, 4096)
    kc, vc, cap = ctx.kv_slot(0)
    pos = 0
    for step, n in enumerate([700, 4, 1]):
        qg, k, v, qn, kn = projections(90 + step, n, s)
        mask = _rand_mask(91 + step, pos, n, cr, 0.3)
        kbits = dev(orc.qsa_key_bits(mask, pos, n, cr).view(np.int32))
        out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
        ctx.layer_attention_qsa(0, dev(qg), dev(k), dev(v), dev(qn), dev(kn), out, pos, n, kbits)
        ctx.sync_status()
        rq, _, _ = oracle.qk_norm_rope(qg, k, v, 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
        kcache = host(qw.k_rows(kc, cap, s.NKV, s.D)[:pos + n])
        vcache = host(qw.v_rows(vc, cap, s.NKV, s.D)[:pos + n])
        o = host(out)
        for t in ([0, 1, 350, n - 1] if n > 4 else range(n)):
            ref = oracle.attention_qsa(rq[t:t + 1], kcache, vcache, pos + t, mask[t:t + 1], cr, qg[t:t + 1])
            assert_parity(o[t:t + 1], ref, f"layer qsa step {step} token {t}")
        pos += n


@pytest.mark.parametrize("s,pos,n,cr,kind", [(TINY, 500, 2, 4, "decode"), (QWEN3_NEXT, 3000, 4, 4, "decode"),
                                              (QWEN3_NEXT, 1000, 300, 8, "prefill")], ids=repr)
def test_qsa_token_hidden_from_leading_tiles(qw, oracle, s, pos, n, cr, kind):
    """Token 0 selects only blocks near its end while every other token selects all: in the leading tiles
    token 0's rows see no key while the others' maxima grow (their rescale must leave token 0's empty
    accumulator finite). Loader-wave decode (G = 4, two tokens), 16-row-slice verify, and the prefill."""
    import oracle as orc
    rows = pos + n
    nmax = rows // cr
    mw = nmax // 32 + 1
    mask = np.full((n, mw), 0xFFFFFFFF, np.uint32)
    bits = np.zeros(mw * 32, bool)
    bits[max(0, nmax - 3):nmax] = True
    mask[0] = (bits.reshape(mw, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)).sum(axis=1).astype(np.uint32)
    kbits = dev(orc.qsa_key_bits(mask, pos, n, cr).view(np.int32))
    cap, k16, v16, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, "f32", 950 + n)
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=max(n, 64))
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    if kind == "decode":
        ctx.decode_qsa(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, 0, kbits)
    else:
        ctx.prefill_qsa(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, kbits)
    ctx.sync_status()
    qg_h = host(qg_d)
    rq, _, _ = oracle.qk_norm_rope(qg_h, host(k_d), host(v_d), 1 + host(qn_d), 1 + host(kn_d), pos, s.R, s.theta, s.eps)
    kr = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    vr = host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows])
    o = host(out)
    for t in sorted({0, 1, n - 1}):
        ref = oracle.attention_qsa(rq[t:t + 1], kr, vr, pos + t, mask[t:t + 1], cr, qg_h[t:t + 1])
        assert_parity(o[t:t + 1], ref, f"{kind} token {t}")
