"""GPU parity of every kernel against the CPU oracle, through the C ABI (libqwattn.so).

Inputs are seeded; the oracle reads the same fp16-rounded K/V the GPU reads (the reference CPU path
keeps fp32 caches, src/qwen4_cpu.cpp:30-32, the GPU path fp16, src/qwen4_vk.cpp:565-574).
"""
import numpy as np
import pytest
import torch

from common import D128, QWEN3_NEXT, TINY, TINY_GGUF, Shape, assert_parity, assert_rows_parity, cache_rows, projections

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    return t.detach().float().cpu().numpy()


def make_ctx(qw, s, max_ctx=8192, max_tokens=2048, max_splits=1024):
    return qw.Attention(s.NH, s.NKV, s.D, s.R, s.theta, s.eps, max_ctx=max_ctx, max_tokens=max_tokens,
                        max_splits=max_splits)


def capacity(rows):
    return (rows + 31) // 32 * 32


def gpu_caches(qw, k16, v16, cap):
    """Caller-owned device caches (blocked layout) of capacity cap holding rows [0, len(k16))."""
    rows, nkv, d = k16.shape
    krows = torch.zeros((cap, nkv, d), dtype=torch.float16, device=DEV)
    krows[:rows] = dev(k16)
    vrows = torch.zeros((cap, nkv, d), dtype=torch.float16, device=DEV)
    vrows[:rows] = dev(v16)
    return qw.k_block(krows), qw.v_block(vrows)


def empty_caches(s, cap):
    n = cap * s.NKV * s.D
    return (torch.zeros(n, dtype=torch.float16, device=DEV), torch.zeros(n, dtype=torch.float16, device=DEV))


# ---- rope table --------------------------------------------------------------------------------------

@pytest.mark.parametrize("s", [TINY, QWEN3_NEXT], ids=repr)
def test_rope_table(qw, oracle, s):
    ctx = make_ctx(qw, s, max_ctx=262144)
    tab = host(ctx.rope_table())
    for lo, hi in [(0, 4096), (262144 - 4096, 262144)]:
        ref = oracle.rope_table(hi, s.R, s.theta)[lo:hi]
        err = np.abs(tab[lo:hi] - ref).max()
        assert err <= 1e-6, (lo, hi, err)
    own = torch.zeros((1000, s.R // 2, 2), device=DEV)
    ctx.fill_rope(own, 1000)
    torch.cuda.synchronize()
    assert np.array_equal(host(own), tab[:1000])


# ---- fused QK-norm + rope + append --------------------------------------------------------------------

CASES_NR = [(TINY, 1, 128), (TINY, 37, 5), (TINY_GGUF, 4, 300), (QWEN3_NEXT, 1, 16384), (QWEN3_NEXT, 4, 32768),
            (QWEN3_NEXT, 64, 1000), (QWEN3_NEXT, 1, 262143)]


@pytest.mark.parametrize("s,n,pos", CASES_NR, ids=lambda v: repr(v))
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_qk_norm_rope_append(qw, oracle, s, n, pos, dtype):
    print(f"norm_rope {s} n={n} pos={pos} {dtype}", flush=True)
    qg, k, v, qn, kn = projections(11 + n, n, s)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    qg_d, k_d, v_d = dev(qg).to(tdt), dev(k).to(tdt), dev(v).to(tdt)
    # the oracle sees exactly the values the GPU reads
    qg_h, k_h, v_h = host(qg_d), host(k_d), host(v_d)
    ctx = make_ctx(qw, s, max_ctx=262144)
    cap = capacity(pos + n)
    kc, vc = empty_caches(s, cap)
    q_out = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc, vc, cap, q_out, pos, n)
    q16 = torch.zeros((n, s.NH, s.D), dtype=torch.float16, device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc, vc, cap, q16, pos, n)
    torch.cuda.synchronize()
    rq, rk, rv = oracle.qk_norm_rope(qg_h, k_h, v_h, 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
    assert np.abs(host(q_out) - rq).max() <= 2e-5 * max(1.0, np.abs(rq).max())
    # fp16 K rows: within one fp16 rounding step of the oracle's fp32 row
    krows = qw.k_rows(kc, cap, s.NKV, s.D)
    gk = host(krows[pos:pos + n])
    assert np.all(np.abs(gk - rk[pos:pos + n]) <= np.abs(rk[pos:pos + n]) * 2.0 ** -10 + 1e-6)
    # V is copied: bit-exact fp16 of the input
    gv = host(qw.v_rows(vc, cap, s.NKV, s.D)[pos:pos + n])
    assert np.array_equal(gv, v_h.astype(np.float16).astype(np.float32))
    # rows outside [pos, pos+n) untouched
    assert float(krows[:pos].abs().max() if pos else 0) == 0.0
    assert float(krows[pos + n:].abs().max() if pos + n < cap else 0) == 0.0
    # fp16 prefill operand = fp16(q * log2(e)/sqrt(D))
    ref16 = rq * (qw.LOG2E / np.sqrt(s.D))
    assert np.all(np.abs(host(q16) - ref16) <= np.abs(ref16) * 2.0 ** -10 + 1e-6)


# ---- split-KV decode / verify -------------------------------------------------------------------------

def run_split(qw, ctx, q, kc, vc, cap, qg, pos, n, n_split=0):
    out = torch.zeros((n, ctx.NH, ctx.D), device=DEV)
    used = ctx.attend_partial(q, kc, vc, cap, pos, n, n_split)
    ctx.combine(qg, out, n, used)
    torch.cuda.synchronize()
    return host(out), used


CASES_DEC = [
    (TINY, 128, 1, 0),
    (TINY, 0, 1, 0),              # a single key: out = V0 * sigmoid(gate)
    (TINY, 33, 4, 0),
    (TINY_GGUF, 300, 1, 3),       # the reference's own tiny shape, 3 splits
    (TINY_GGUF, 17, 4, 0),
    (QWEN3_NEXT, 16384, 1, 64),   # BASELINE config 2 with the reference's 64 splits
    (QWEN3_NEXT, 16384, 1, 0),
    (QWEN3_NEXT, 31, 1, 0),
    (QWEN3_NEXT, 32768, 4, 0),    # BASELINE config 3 (MTP verify)
    (QWEN3_NEXT, 1000, 3, 7),
    (QWEN3_NEXT, 32768, 1, 0),    # the headline metric's shape
]


@pytest.mark.parametrize("s,pos,n,n_split", CASES_DEC, ids=lambda v: repr(v))
def test_split_decode_parity(qw, oracle, s, pos, n, n_split):
    print(f"decode {s} pos={pos} n={n} split={n_split}", flush=True)
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(100 + pos, rows, s)
    r = np.random.default_rng(pos + 7)
    q = r.standard_normal((n, s.NH, s.D)).astype(np.float32)
    qg = r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32)
    ctx = make_ctx(qw, s, max_ctx=cap)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    out, used = run_split(qw, ctx, dev(q), kc, vc, cap, dev(qg), pos, n, n_split)
    if n_split:  # a requested split count runs as given, capped at the 32-key blocks that hold keys
        assert used == min(n_split, (rows + 31) // 32), used
    ref = oracle.attention(q, k16.astype(np.float32), v16.astype(np.float32), pos, qg)
    assert_parity(out, ref, f"{s} pos={pos} n={n} splits={used}")
    if pos == 0:
        sig = 1 / (1 + np.exp(-qg[0, :, s.D:].astype(np.float64)))
        exp0 = v16[0].astype(np.float64)[np.arange(s.NH) // s.G] * sig
        assert np.abs(out[0] - exp0).max() <= 1e-6


def test_split_peaked_keys(qw, oracle):
    """1% of the key rows scaled x8 (BASELINE config 5's softmax-range stress) at 16K."""
    s = QWEN3_NEXT
    pos, n = 16384, 1
    rows = pos + n
    k16, v16 = cache_rows(5, rows, s, heavy_frac=0.01)
    r = np.random.default_rng(9)
    q = r.standard_normal((n, s.NH, s.D)).astype(np.float32)
    qg = r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32)
    ctx = make_ctx(qw, s, max_ctx=rows + 7)
    cap = capacity(rows)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    out, _ = run_split(qw, ctx, dev(q), kc, vc, cap, dev(qg), pos, n, 256)
    ref = oracle.attention(q, k16.astype(np.float32), v16.astype(np.float32), pos, qg)
    assert_parity(out, ref, "peaked")


@pytest.mark.parametrize("n", [1, 4])
def test_split_invariance(qw, n):
    """Any split count, including splits that end up empty for some rows, gives the same output.

    Tolerance: both the single-token and the 4-token kernels carry the query and P as an fp16 hi part
    plus an fp16 lo remainder (about 22 mantissa bits together) against the exact fp16 cache, so split
    counts, which change only the order of fp32 sums and the running maxima P is taken against, agree
    to fp32 rounding."""
    s = QWEN3_NEXT
    pos = 5000
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(3, rows, s)
    r = np.random.default_rng(4)
    q = dev(r.standard_normal((n, s.NH, s.D)).astype(np.float32))
    qg = dev(r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32))
    ctx = make_ctx(qw, s, max_ctx=cap)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    outs = {sp: run_split(qw, ctx, q, kc, vc, cap, qg, pos, n, sp)[0] for sp in (1, 2, 7, 64, 0, 157, 1024)}
    base = outs[1]
    for sp, o in outs.items():
        err = np.abs(o - base).max()
        print(f"n={n} splits={sp}: max |diff| vs 1 split {err:.2e} (output scale {np.abs(base).max():.2e})")
        assert err <= 2e-7, sp


def test_verify_equals_sequential_decodes(qw):
    """A 4-token verify pass equals 4 single-token decodes at pos..pos+3 (src/main.cpp:457-460)."""
    s = QWEN3_NEXT
    pos, n = 3000, 4
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(21, rows, s)
    r = np.random.default_rng(22)
    q = r.standard_normal((n, s.NH, s.D)).astype(np.float32)
    qg = r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32)
    ctx = make_ctx(qw, s, max_ctx=cap)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    together, _ = run_split(qw, ctx, dev(q), kc, vc, cap, dev(qg), pos, n)
    for t in range(n):
        one, _ = run_split(qw, ctx, dev(q[t:t + 1]), kc, vc, cap, dev(qg[t:t + 1]), pos + t, 1)
        # both kernels carry Q and P as fp16 hi + lo parts: they agree to fp32 rounding
        err = np.abs(one[0] - together[t]).max()
        print(f"token {t}: max |verify - decode| {err:.2e}")
        assert err <= 2e-7, t


# ---- fused decode: norm + rope + append + split attend in one launch ----------------------------------

CASES_FUSED = [
    (TINY, 128, 1, 0, "f32"),           # BASELINE config 1 through the fused path
    (TINY, 0, 1, 0, "f32"),             # first token: the only key is the new one
    (TINY, 45, 4, 0, "bf16"),
    (TINY_GGUF, 300, 1, 3, "f32"),      # the reference's tiny shape, 3 splits
    (TINY_GGUF, 30, 4, 2, "bf16"),      # new keys straddle a block and a split boundary
    (QWEN3_NEXT, 16384, 1, 0, "f32"),
    (QWEN3_NEXT, 16384, 1, 64, "bf16"),  # BASELINE config 2 with the reference's 64 splits
    (QWEN3_NEXT, 32768, 4, 0, "f32"),
    (D128, 4000, 1, 0, "bf16"),
    (D128, 777, 4, 0, "f32"),
    (QWEN3_NEXT, 32766, 4, 0, "f32"),   # the 4 new keys straddle a 32-key block
    (QWEN3_NEXT, 1000, 3, 7, "bf16"),
    (QWEN3_NEXT, 32768, 1, 0, "f32"),   # the headline shape
]


def _fused_setup(qw, s, pos, n, dtype, seed):
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(seed, pos, s) if pos else (np.zeros((0, s.NKV, s.D), np.float16),) * 2
    qg, k, v, qn, kn = projections(seed + 1, n, s)
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    qg_d, k_d, v_d = dev(qg).to(tdt), dev(k).to(tdt), dev(v).to(tdt)
    # stale rows at the new positions and NaN past the cache end must not reach the result
    krows = torch.full((cap, s.NKV, s.D), float("nan"), dtype=torch.float16, device=DEV)
    vrows = torch.full((cap, s.NKV, s.D), float("nan"), dtype=torch.float16, device=DEV)
    krows[pos:rows] = 100.0
    vrows[pos:rows] = -100.0
    if pos:
        krows[:pos] = dev(k16)
        vrows[:pos] = dev(v16)
    return cap, k16, v16, qg_d, k_d, v_d, dev(qn), dev(kn), qw.k_block(krows), qw.v_block(vrows)


@pytest.mark.parametrize("s,pos,n,n_split,dtype", CASES_FUSED, ids=lambda v: repr(v))
def test_fused_decode_parity(qw, oracle, s, pos, n, n_split, dtype):
    """qwattn_decode_partial + qwattn_combine against the oracle's norm/rope/append and attention on the
    same inputs; the appended rows land in the cache (K within one fp16 step, V bit-exact), earlier rows
    are untouched, stale rows at the new positions and NaN past the end do not leak in."""
    print(f"fused decode {s} pos={pos} n={n} split={n_split} {dtype}", flush=True)
    rows = pos + n
    cap, k16, v16, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, dtype, 400 + pos + n)
    ctx = make_ctx(qw, s, max_ctx=cap)
    out = torch.zeros((n, s.NH, s.D), device=DEV)
    used = ctx.decode_partial(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, pos, n, n_split)
    ctx.combine(qg_d, out, n, used)
    torch.cuda.synchronize()
    qg_h, k_h, v_h = host(qg_d), host(k_d), host(v_d)
    rq, rk, _ = oracle.qk_norm_rope(qg_h, k_h, v_h, 1 + host(qn_d), 1 + host(kn_d), pos, s.R, s.theta, s.eps)
    krows, vrows = qw.k_rows(kc, cap, s.NKV, s.D), qw.v_rows(vc, cap, s.NKV, s.D)
    gk = host(krows[pos:rows])
    assert np.all(np.abs(gk - rk[pos:rows]) <= np.abs(rk[pos:rows]) * 2.0 ** -10 + 1e-6)
    assert np.array_equal(host(vrows[pos:rows]), v_h.astype(np.float16).astype(np.float32))
    if pos:
        assert np.array_equal(host(krows[:pos]), k16.astype(np.float32))
        assert np.array_equal(host(vrows[:pos]), v16.astype(np.float32))
    ref = oracle.attention(rq, host(krows[:rows]), host(vrows[:rows]), pos, qg_h)
    assert_parity(host(out), ref, f"{s} pos={pos} n={n} splits={used}")


@pytest.mark.parametrize("s,pos,n", [(QWEN3_NEXT, 5000, 1), (QWEN3_NEXT, 4093, 4), (TINY, 77, 2)], ids=repr)
def test_fused_equals_unfused(qw, s, pos, n):
    """The fused launch computes what the per-dispatch entry points compute in sequence
    (qk_norm_rope_append -> attend_partial -> combine). The fused kernel sums the RMSNorm over 32 lanes
    per row, the standalone kernel over 64, so K rows may differ by one fp16 rounding step and the
    outputs by fp32 rounding; V rows and the split are identical."""
    cap, _, _, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, "f32", 500 + pos)
    kc2, vc2 = kc.clone(), vc.clone()
    ctx = make_ctx(qw, s, max_ctx=cap)
    out = torch.zeros((n, s.NH, s.D), device=DEV)
    used = ctx.decode_partial(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, pos, n, 0)
    ctx.combine(qg_d, out, n, used)
    q = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc2, vc2, cap, q, pos, n)
    out2 = torch.zeros((n, s.NH, s.D), device=DEV)
    used2 = ctx.attend_partial(q, kc2, vc2, cap, pos, n, 0)
    ctx.combine(qg_d, out2, n, used2)
    torch.cuda.synchronize()
    assert used == used2
    k1 = host(qw.k_rows(kc, cap, s.NKV, s.D)[:pos + n])
    k2 = host(qw.k_rows(kc2, cap, s.NKV, s.D)[:pos + n])
    assert np.array_equal(k1[:pos], k2[:pos])
    assert np.all(np.abs(k1[pos:] - k2[pos:]) <= np.abs(k2[pos:]) * 2.0 ** -10)
    assert torch.equal(qw.v_rows(vc, cap, s.NKV, s.D)[:pos + n], qw.v_rows(vc2, cap, s.NKV, s.D)[:pos + n])
    assert np.abs(host(out) - host(out2)).max() <= 2e-6


ONE_LAUNCH = CASES_FUSED + [
    (TINY_GGUF, 61, 4, 0, "f32"),       # automatic splits of one block each: the new rows straddle two chunks
    (TINY, 63, 2, 0, "bf16"),           # the same with one new row in each chunk
    (QWEN3_NEXT, 16383, 1, 64, "f32"),  # 64 splits of 8 blocks, the new row opening the last block
    # 9 to 32 rows (qwattn_decode's 16-row-slice kernel; the combine on the slices' last chunks when a
    # slice has at least as many chunks as rows, else the combine kernel): partly filled slices, 8 new
    # rows, one split holding every tile, splits of a single tile that holds new rows
    (TINY, 500, 3, 0, "f32"),           # 12 rows: the second group half full, two idle waves
    (QWEN3_NEXT, 32768, 4, 0, "bf16"),  # 32 rows in two slices, 64 chunks each
    (QWEN3_NEXT, 3000, 3, 16, "f32"),   # 24 rows: a full and a half slice, 16 chunks (every chunk of the
                                        # first slice combines a row)
    (TINY_GGUF, 100, 5, 0, "bf16"),     # 10 rows at D = 256, G = 2
    (D128, 2000, 8, 0, "bf16"),         # 32 rows, 8 new rows across a block boundary
    (QWEN3_NEXT, 5000, 4, 1, "f32"),    # one split: 157 tiles through one ring
    (QWEN3_NEXT, 40, 2, 0, "bf16"),     # 16 rows, two splits of one tile each
    # the in-launch combine's dim slices: 4 per row of 16 dims (D = 64), 2 of 128 (D = 256, 32 splits)
    (TINY, 4000, 1, 0, "f32"),
    (QWEN3_NEXT, 9000, 1, 32, "bf16"),
]


@pytest.mark.parametrize("s,pos,n,n_split,dtype", ONE_LAUNCH, ids=lambda v: repr(v))
def test_decode_one_launch_parity(qw, oracle, s, pos, n, n_split, dtype):
    """qwattn_decode (norm, rope, append, split attend and the combine with its gate in one launch)
    against the oracle, with the cache checks of the two-launch test."""
    print(f"one-launch decode {s} pos={pos} n={n} split={n_split} {dtype}", flush=True)
    rows = pos + n
    cap, k16, v16, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, dtype, 400 + pos + n)
    ctx = make_ctx(qw, s, max_ctx=cap)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    used = ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, n_split)
    torch.cuda.synchronize()
    qg_h, k_h, v_h = host(qg_d), host(k_d), host(v_d)
    rq, rk, _ = oracle.qk_norm_rope(qg_h, k_h, v_h, 1 + host(qn_d), 1 + host(kn_d), pos, s.R, s.theta, s.eps)
    krows, vrows = qw.k_rows(kc, cap, s.NKV, s.D), qw.v_rows(vc, cap, s.NKV, s.D)
    assert np.all(np.abs(host(krows[pos:rows]) - rk[pos:rows]) <= np.abs(rk[pos:rows]) * 2.0 ** -10 + 1e-6)
    assert np.array_equal(host(vrows[pos:rows]), v_h.astype(np.float16).astype(np.float32))
    ref = oracle.attention(rq, host(krows[:rows]), host(vrows[:rows]), pos, qg_h)
    assert_parity(host(out), ref, f"{s} pos={pos} n={n} splits={used}")


def test_decode_one_launch_equals_two_launches(qw):
    """The in-launch combine merges what qwattn_combine merges: over a run of calls on one context with
    changing token counts (decode n=1 on the loader-wave kernel, verify n=4 on two 16-row slices, combined
    by the slices' last chunks with 16 chunks or more, else by the combine kernel) and split counts (fewer
    splits than combine units, one split, many; the two-launch call is given the first call's count), each
    output matches decode_partial + combine to fp32 rounding (the two merges visit the splits in different
    orders).
    The one-launch calls use the context's ready flags with changing split counts: a flag left by one
    call that passed for a later call's epoch would let its combiners merge stale partials."""
    s, pos = QWEN3_NEXT, 3000
    cap, _, _, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, 4, "f32", 77)
    ctx = make_ctx(qw, s, max_ctx=cap)
    for n, n_split in [(1, 3), (4, 0), (1, 0), (4, 1), (1, 1), (4, 7), (1, 93), (4, 93), (1, 0), (2, 2), (4, 16),
                       (3, 16), (4, 0)]:
        print(f"one-launch vs two-launch n={n} splits={n_split}", flush=True)
        out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
        used = ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n, n_split)
        out2 = torch.zeros((n, s.NH, s.D), device=DEV)
        used2 = ctx.decode_partial(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, pos, n, used)
        ctx.combine(qg_d, out2, n, used2)
        torch.cuda.synchronize()
        assert used == used2
        assert np.abs(host(out) - host(out2)).max() <= 2e-6, f"splits={used}"


@pytest.mark.parametrize("n", [1, 4])
def test_decode_one_launch_graph_replays(qw, n):
    """Captured into a HIP graph, the one-launch decode (n = 1: the KV heads' last chunks combine; n = 4:
    the 16-row slices' last chunks) gives the eager result on every replay, with eager work and
    synchronizations in between (each launch advances its own epoch inside the kernel; nothing is cleared
    by a memset node)."""
    s, pos = QWEN3_NEXT, 8190
    cap, _, _, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, "f32", 91)
    ctx = make_ctx(qw, s, max_ctx=cap)
    rope = ctx.rope_table()
    eager = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, eager, pos, n, 0)
    torch.cuda.synchronize()
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, out, pos, n, 0, stream=stream)
    for rep in range(4):
        print(f"graph replay {rep}", flush=True)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, eager, pos, n, 0)  # eager work in between
        torch.cuda.synchronize()


def test_decode_256k_peaked_keys(qw, oracle):
    """262,144 cached tokens + 1, with 1% of the cached key rows scaled x8
    (softmax-range stress), against the oracle on the same fp16 rows: through the one-launch decode (norm,
    rope, append, split attend, in-launch combine) at the automatic split count and with the
    configuration's 1,024 splits requested (capped at the automatic count: one streaming workgroup per
    CU, the same launch bit for bit), and with exactly 1,024 split partials (8,193 blocks of keys: part z
    the blocks z, z + 1,024, ...) through the fused partial entry point and the combine kernel."""
    s = QWEN3_NEXT
    pos, n = 262144, 1
    rows = pos + n
    cap = capacity(rows)
    print(f"decode 256K: building {cap} cache rows on the GPU", flush=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(2561)
    krows = torch.randn((cap, s.NKV, s.D), generator=g, device=DEV).half()
    vrows = torch.randn((cap, s.NKV, s.D), generator=g, device=DEV).half()
    heavy = torch.randperm(pos, generator=g, device=DEV)[:pos // 100]
    krows[heavy] *= 8.0
    krows[pos:] = float("nan")  # the new row is appended by the kernel; past it nothing may leak in
    vrows[pos:] = float("nan")
    kc, vc = qw.k_block(krows), qw.v_block(vrows)
    del krows, vrows
    qg, k, v, qn, kn = projections(2562, n, s)
    qg_d, k_d, v_d, qn_d, kn_d = dev(qg), dev(k), dev(v), dev(qn), dev(kn)
    ctx = make_ctx(qw, s, max_ctx=cap)
    outs, used_by_req = {}, {}
    for n_split in (0, 1024):
        print(f"decode 256K: one launch, splits requested {n_split or 'auto'}", flush=True)
        out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
        used_by_req[n_split] = ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, out, pos, n,
                                          n_split)
        ctx.sync_status()
        outs[f"one launch, {n_split or 'auto'} requested"] = host(out)
    assert used_by_req[1024] == used_by_req[0] < 1024, used_by_req
    assert np.array_equal(outs["one launch, 1024 requested"], outs["one launch, auto requested"])
    print("decode 256K: 1,024 split partials + combine", flush=True)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    used = ctx.decode_partial(qg_d, k_d, v_d, qn_d, kn_d, ctx.rope_table(), kc, vc, cap, pos, n, 1024)
    assert used == 1024
    ctx.combine(qg_d, out, n, used)
    ctx.sync_status()
    outs["1024 partials"] = host(out)
    rq, rk, _ = oracle.qk_norm_rope(qg, k, v, 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
    kr = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    assert np.all(np.abs(kr[pos] - rk[pos]) <= np.abs(rk[pos]) * 2.0 ** -10 + 1e-6)
    ref = oracle.attention(rq, kr, host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows]), pos, qg)
    for name, o in outs.items():
        print(f"decode 256K {name}: max_abs {np.abs(o - ref).max():.2e}", flush=True)
        assert_parity(o, ref, f"256K {name}")


@pytest.mark.parametrize("n", [1, 4])
def test_decode_wait_timeout_is_reported(qw, n):
    """A bounded in-kernel wait that gives up is an error, not silently wrong output: with the test hook
    skewing the epoch the in-launch combine waits for (n = 1: the KV heads' last chunks; n = 4: the 16-row
    slices' last chunks), no split's ready flag ever matches, the poller gives up after 64 polls, every kernel
    still ends, and the context reports QWATTN_ETIMEOUT once (through qwattn_sync_status, or the next
    call). With the hook off, the context computes correctly again."""
    s, pos = QWEN3_NEXT, 3000
    cap, _, _, qg_d, k_d, v_d, qn_d, kn_d, kc, vc = _fused_setup(qw, s, pos, n, "f32", 123)
    ctx = make_ctx(qw, s, max_ctx=cap)
    rope = ctx.rope_table()
    good = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, good, pos, n, 16)
    ctx.sync_status()
    ctx.set_wait_limits(spin_max=64, epoch_skew=5)
    out = torch.zeros((n, s.NH, s.D), device=DEV)
    print("forced give-up: decode with skewed epoch", flush=True)
    ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, out, pos, n, 16)
    with pytest.raises(qw.QwattnError, match="bounded wait") as e:
        ctx.sync_status()
    assert e.value.code == qw.ETIMEOUT
    ctx.sync_status()  # reported once
    print("forced give-up: the next call reports it", flush=True)
    ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, out, pos, n, 16)
    torch.cuda.synchronize()  # that launch has ended; its give-up waits in the context
    with pytest.raises(qw.QwattnError) as e:
        ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, out, pos, n, 16)  # refused, launches nothing
    assert e.value.code == qw.ETIMEOUT
    ctx.sync_status()
    ctx.set_wait_limits(0, 0)
    out.fill_(float("nan"))
    ctx.decode(qg_d, k_d, v_d, qn_d, kn_d, rope, kc, vc, cap, out, pos, n, 16)
    ctx.sync_status()
    assert torch.equal(out, good)


# ---- prefill -------------------------------------------------------------------------------------------

CASES_PF = [
    (TINY, 0, 64),
    (TINY, 100, 37),
    (TINY_GGUF, 5, 50),
    (QWEN3_NEXT, 0, 5),
    (QWEN3_NEXT, 0, 300),
    (QWEN3_NEXT, 777, 129),
    (QWEN3_NEXT, 2048, 2048),
    (QWEN3_NEXT, 1500, 1100),   # paired schedule (69 tiles x 2 KV heads > 256 CUs / 2), odd tile count
    (QWEN3_NEXT, 1024, 1024),   # split schedule at its limit on 256 CUs (64 tiles x 2 KV heads x 2)
    (TINY, 1000, 200),          # odd tile count, a split tile with D = 64 (two dim tiles)
    (D128, 1000, 200),          # the same with D = 128
]


@pytest.mark.parametrize("s,pos,n", CASES_PF, ids=lambda v: repr(v))
def test_prefill_parity(qw, oracle, s, pos, n):
    """bf16 projections -> fused norm/rope/append (fp16 pre-scaled q) -> MFMA prefill, against the
    oracle's norm/rope/append and attention on the same values."""
    print(f"prefill {s} pos={pos} n={n}", flush=True)
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(40 + pos, pos, s) if pos else (np.zeros((0, s.NKV, s.D), np.float16),) * 2
    qg, k, v, qn, kn = projections(41 + n, n, s)
    qg_d, k_d, v_d = dev(qg).to(torch.bfloat16), dev(k).to(torch.bfloat16), dev(v).to(torch.bfloat16)
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=max(n, 1))
    kc, vc = gpu_caches(qw, k16, v16, cap) if pos else empty_caches(s, cap)
    q16 = torch.zeros((n, s.NH, s.D), dtype=torch.float16, device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc, vc, cap, q16, pos, n)
    out_d = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.attend_prefill(q16, kc, vc, cap, qg_d, out_d, pos, n)
    # again on the same context: the split query tiles' arrival counters are back at zero and their
    # merge order is fixed, so the bits repeat
    out_d2 = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    ctx.attend_prefill(q16, kc, vc, cap, qg_d, out_d2, pos, n)
    torch.cuda.synchronize()
    out = host(out_d)
    assert np.array_equal(out, host(out_d2)), f"{s} pos={pos} n={n}: second launch differs"
    # oracle on the same inputs; K/V cache rows as the GPU holds them (fp16)
    rq, _, _ = oracle.qk_norm_rope(host(qg_d), host(k_d), host(v_d), 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
    kcache = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    vcache = host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows])
    qg_h = host(qg_d)
    # every token row (both halves of each split or paired query tile included), one batched oracle call
    ref = oracle.attention(rq, kcache, vcache, pos, qg_h)
    assert_rows_parity(out, ref, f"{s} pos={pos} n={n}")


@pytest.mark.parametrize("s,pos,n", CASES_PF, ids=lambda v: repr(v))
def test_prefill_entry_parity(qw, oracle, s, pos, n):
    """qwattn_prefill against the oracle and against the two entry points called in sequence (norm/rope/
    append into a query buffer, then the MFMA prefill on it). With a rope width the prefill kernel takes
    (here every shape but TINY's r16), qwattn_prefill appends only K/V and the kernel normalizes the
    queries itself: same K/V bits, and outputs that differ only where a query element's fp16 rounding
    does (its mean of squares is summed in another order); otherwise it is that same sequence, bit for
    bit."""
    print(f"fused prefill {s} pos={pos} n={n}", flush=True)
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(40 + pos, pos, s) if pos else (np.zeros((0, s.NKV, s.D), np.float16),) * 2
    qg, k, v, qn, kn = projections(41 + n, n, s)
    qg_d, k_d, v_d = dev(qg).to(torch.bfloat16), dev(k).to(torch.bfloat16), dev(v).to(torch.bfloat16)
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=max(n, 1))
    kc, vc = gpu_caches(qw, k16, v16, cap) if pos else empty_caches(s, cap)
    kc2, vc2 = kc.clone(), vc.clone()
    out = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.prefill(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc, vc, cap, out, pos, n)
    q16 = torch.zeros((n, s.NH, s.D), dtype=torch.float16, device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc2, vc2, cap, q16, pos, n)
    out2 = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.attend_prefill(q16, kc2, vc2, cap, qg_d, out2, pos, n)
    torch.cuda.synchronize()
    # the same K/V rows appended by both paths
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    out, out2 = host(out), host(out2)
    if s.R in (0, 32, 64, 128, 256):
        assert_parity(out, out2, f"{s} in-kernel vs buffered query", atol=5e-4, rtol=1e-3)
    else:
        assert np.array_equal(out, out2)
    rq, _, _ = oracle.qk_norm_rope(host(qg_d), host(k_d), host(v_d), 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
    kcache = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    vcache = host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows])
    qg_h = host(qg_d)
    # every token row (both halves of each split or paired query tile included), one batched oracle call
    ref = oracle.attention(rq, kcache, vcache, pos, qg_h)
    assert_rows_parity(out, ref, f"{s} pos={pos} n={n}")


CASES_PF_QG = [
    (Shape(4, 1, 64, 32), 300, 200, "bf16"),     # rotate-half partner one k-step away
    (Shape(4, 1, 64, 64), 0, 130, "f32"),        # R = D = 64: two k-steps away, fp32 projections
    (Shape(8, 2, 128, 128), 500, 300, "bf16"),   # four k-steps away
    (Shape(16, 2, 256, 128), 1000, 257, "f32"),  # four, at D = 256
    (Shape(16, 2, 256, 256), 64, 700, "bf16"),   # R = D = 256: eight k-steps away
    (Shape(16, 2, 256, 0), 100, 100, "bf16"),    # no rope
    (QWEN3_NEXT, 2048, 2048, "f32"),             # the bench shape with fp32 projections
    # paired schedules with bf16 rows: the two-segment workgroups take their second segment's query rows
    # and first K tiles from the first segment
    (Shape(8, 2, 128, 64), 300, 2200, "bf16"),   # D = 128, (cos, sin) loaded with the rows; a middle tile
    (Shape(4, 1, 64, 32), 100, 4200, "bf16"),    # D = 64, the R = 32 cross-lane partner
]


@pytest.mark.parametrize("s,pos,n,dt", CASES_PF_QG, ids=lambda v: repr(v))
def test_prefill_qg_parity(qw, oracle, s, pos, n, dt):
    """The K/V-only append (q_out NULL) then qwattn_attend_prefill_qg, which normalizes, rotates and
    scales the query rows in the attention kernel, against the oracle for every rope width the kernel
    takes (the partner dim d + R/2 one, two, four and eight k-steps away in a lane) and both input
    dtypes; the K/V-only append writes the same cache bits as the full one and no query rows."""
    print(f"prefill qg {s} pos={pos} n={n} {dt}", flush=True)
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(60 + pos, pos, s) if pos else (np.zeros((0, s.NKV, s.D), np.float16),) * 2
    qg, k, v, qn, kn = projections(61 + n, n, s)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    qg_d, k_d, v_d = dev(qg).to(tdt), dev(k).to(tdt), dev(v).to(tdt)
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=max(n, 1))
    kc, vc = gpu_caches(qw, k16, v16, cap) if pos else empty_caches(s, cap)
    kc2, vc2 = kc.clone(), vc.clone()
    rope = ctx.rope_table() if s.R else None
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), rope, kc, vc, cap, None, pos, n)
    q16 = torch.zeros((n, s.NH, s.D), dtype=torch.float16, device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), rope, kc2, vc2, cap, q16, pos, n)
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    ctx.attend_prefill_qg(qg_d, dev(qn), rope, kc, vc, cap, out, pos, n)
    out2 = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.attend_prefill(q16, kc2, vc2, cap, qg_d, out2, pos, n)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    out = host(out)
    assert_parity(out, host(out2), f"{s} in-kernel vs buffered query", atol=5e-4, rtol=1e-3)
    rq, _, _ = oracle.qk_norm_rope(host(qg_d), host(k_d), host(v_d), 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
    kcache = host(qw.k_rows(kc, cap, s.NKV, s.D)[:rows])
    vcache = host(qw.v_rows(vc, cap, s.NKV, s.D)[:rows])
    qg_h = host(qg_d)
    # every token row (both halves of each split or paired query tile included), one batched oracle call
    ref = oracle.attention(rq, kcache, vcache, pos, qg_h)
    assert_rows_parity(out, ref, f"{s} pos={pos} n={n}")


def test_prefill_qg_rejects_rope_width(qw):
    """A rope width the in-kernel query normalization does not take is refused (and qwattn_prefill
    takes the query-buffer path for it, covered by the TINY cases above)."""
    s = TINY  # r16
    ctx = make_ctx(qw, s, max_ctx=256, max_tokens=64)
    kc, vc = empty_caches(s, 256)
    qg = torch.zeros((16, s.NH, 2 * s.D), device=DEV)
    out = torch.zeros((16, s.NH, s.D), device=DEV)
    with pytest.raises(qw.QwattnError, match="rope_dim 16") as e:
        ctx.attend_prefill_qg(qg, torch.zeros(s.D, device=DEV), ctx.rope_table(), kc, vc, 256, out, 0, 16)
    assert e.value.code == qw.EINVAL


def test_prefill_graph_replays(qw):
    """Captured into a HIP graph, the prefill (with split query tiles: 9 tiles, pairs merged through
    the context's arrival counters, which each launch leaves at zero) gives the eager bits on every
    replay, with eager launches and synchronizations in between."""
    s, pos, n = QWEN3_NEXT, 777, 129
    cap = capacity(pos + n)
    k16, v16 = cache_rows(95, pos, s)
    qg, k, v, qn, kn = projections(96, n, s)
    qg_d, k_d, v_d = dev(qg).to(torch.bfloat16), dev(k).to(torch.bfloat16), dev(v).to(torch.bfloat16)
    ctx = make_ctx(qw, s, max_ctx=cap, max_tokens=n)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    q16 = torch.zeros((n, s.NH, s.D), dtype=torch.float16, device=DEV)
    ctx.qk_norm_rope_append(qg_d, k_d, v_d, dev(qn), dev(kn), ctx.rope_table(), kc, vc, cap, q16, pos, n)
    eager = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.attend_prefill(q16, kc, vc, cap, qg_d, eager, pos, n)
    torch.cuda.synchronize()
    out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            ctx.attend_prefill(q16, kc, vc, cap, qg_d, out, pos, n, stream=stream)
    for rep in range(4):
        print(f"prefill graph replay {rep}", flush=True)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        ctx.attend_prefill(q16, kc, vc, cap, qg_d, eager, pos, n)  # eager work in between
        torch.cuda.synchronize()


def test_prefill_equals_decodes(qw):
    """A prefill chunk gives the same rows as decoding its tokens one at a time (block-causal vs
    token-causal masks agree)."""
    s = QWEN3_NEXT
    pos, n = 200, 70
    rows = pos + n
    cap = capacity(rows)
    k16, v16 = cache_rows(51, rows, s)
    r = np.random.default_rng(52)
    q = r.standard_normal((n, s.NH, s.D)).astype(np.float32)
    qg = dev(r.standard_normal((n, s.NH, 2 * s.D)).astype(np.float32))
    ctx = make_ctx(qw, s, max_ctx=cap)
    kc, vc = gpu_caches(qw, k16, v16, cap)
    out = torch.zeros((n, s.NH, s.D), device=DEV)
    ctx.attend_prefill(dev(q), kc, vc, cap, qg, out, pos, n)
    torch.cuda.synchronize()
    pf = host(out)
    for t in range(0, n, 7):
        one, _ = run_split(qw, ctx, dev(q[t:t + 1]), kc, vc, cap, qg[t:t + 1], pos + t, 1)
        # prefill rounds q and p to fp16, decode keeps them at ~fp32: compare at the parity bar
        assert_parity(pf[t:t + 1], one, f"token {t}")


# ---- the whole layer body through context-owned caches -------------------------------------------------

def test_layer_attention_prefill_then_decode(qw, oracle):
    """qwattn_layer_attention over a prefill chunk then decode steps, with cache growth in between,
    against the oracle's norm/rope/cache/attention sequence (fp32 inputs)."""
    s = QWEN3_NEXT
    ctx = make_ctx(qw, s, max_ctx=4096, max_tokens=512)
    ctx.kv_alloc(2, 64)  # forces growth: 64 -> 512 -> ...
    n0 = 300
    ref_k = np.zeros((4096, s.NKV, s.D), np.float32)
    ref_v = np.zeros((4096, s.NKV, s.D), np.float32)
    pos = 0
    for step, n in enumerate([n0, 1, 1, 4, 1]):
        qg, k, v, qn, kn = projections(70 + step, n, s)
        ctx.kv_grow(pos + n)
        out = torch.zeros((n, s.NH, s.D), device=DEV)
        ctx.layer_attention(1, dev(qg), dev(k), dev(v), dev(qn), dev(kn), out, pos, n)
        torch.cuda.synchronize()
        rq, rk, rv = oracle.qk_norm_rope(qg, k, v, 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
        ref_k[pos:pos + n] = rk[pos:pos + n].astype(np.float16)
        ref_v[pos:pos + n] = rv[pos:pos + n].astype(np.float16)
        ref = oracle.attention(rq, ref_k[:pos + n], ref_v[:pos + n], pos, qg)
        assert_parity(host(out), ref, f"step {step} pos={pos} n={n}")
        pos += n
    kc, vc, cap = ctx.kv_slot(1)
    assert cap >= pos
    assert np.array_equal(host(qw.v_rows(vc, cap, s.NKV, s.D)[:pos]), ref_v[:pos])


def test_kv_grow_failure_leaves_caches_whole(qw, oracle):
    """A qwattn_kv_grow whose fourth buffer allocation fails (slot 1's V, after slot 0's pair and slot 1's K
    were allocated) returns QWATTN_ENOMEM and leaves every slot's buffers, contents and the capacity as they
    were, so the next layer call still matches the oracle; the grow then succeeds when retried. A failing
    qwattn_kv_alloc leaves no cache. Reference: src/qwen4_vk.cpp:657-685 throws before touching the caches."""
    s = QWEN3_NEXT
    print("kv_grow failure path", flush=True)
    ctx = make_ctx(qw, s, max_ctx=1024, max_tokens=128)
    ctx.set_alloc_fault(3)
    with pytest.raises(qw.QwattnError, match="out of device memory") as e:
        ctx.kv_alloc(3, 64)
    assert e.value.code == qw.ENOMEM
    with pytest.raises(qw.QwattnError, match="no K/V cache"):
        ctx.kv_grow(100)
    ctx.kv_alloc(3, 64)
    ref_k = np.zeros((1024, s.NKV, s.D), np.float32)
    ref_v = np.zeros((1024, s.NKV, s.D), np.float32)
    pos = 0

    def step(seed, n):
        nonlocal pos
        qg, k, v, qn, kn = projections(seed, n, s)
        out = torch.zeros((n, s.NH, s.D), device=DEV)
        ctx.layer_attention(2, dev(qg), dev(k), dev(v), dev(qn), dev(kn), out, pos, n)
        torch.cuda.synchronize()
        rq, rk, rv = oracle.qk_norm_rope(qg, k, v, 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
        ref_k[pos:pos + n] = rk[pos:pos + n].astype(np.float16)
        ref_v[pos:pos + n] = rv[pos:pos + n].astype(np.float16)
        ref = oracle.attention(rq, ref_k[:pos + n], ref_v[:pos + n], pos, qg)
        assert_parity(host(out), ref, f"pos={pos} n={n}")
        pos += n

    step(80, 60)
    before = [ctx.kv_slot(i) for i in range(3)]
    snap = [(kc.clone(), vc.clone()) for kc, vc, _ in before]
    ctx.set_alloc_fault(4)
    with pytest.raises(qw.QwattnError, match="out of VRAM growing the K/V caches") as e:
        ctx.kv_grow(100)
    assert e.value.code == qw.ENOMEM
    after = [ctx.kv_slot(i) for i in range(3)]
    for (kc0, vc0, cap0), (kc1, vc1, cap1), (ks, vs) in zip(before, after, snap):
        assert cap1 == cap0 == 64 and kc1.data_ptr() == kc0.data_ptr() and vc1.data_ptr() == vc0.data_ptr()
        assert torch.equal(kc1, ks) and torch.equal(vc1, vs)
    step(81, 1)
    step(82, 3)
    ctx.kv_grow(100)
    assert ctx.kv_slot(2)[2] == 128
    step(83, 36)
    step(84, 1)


def test_rollback_is_position_reset(qw, oracle):
    """accept(2) after a 4-token verify: the next step equals a run that never saw drafts 3-4 (the
    reference rolls attention back by resetting pos_, src/qwen4_vk.cpp:286-300)."""
    s = QWEN3_NEXT
    ctx = make_ctx(qw, s, max_ctx=2048, max_tokens=512)
    ctx.kv_alloc(1, 2048)
    base = 500
    qg0, k0, v0, qn, kn = projections(90, base, s)
    out = torch.zeros((base, s.NH, s.D), device=DEV)
    ctx.layer_attention(0, dev(qg0), dev(k0), dev(v0), dev(qn), dev(kn), out, 0, base)
    # verify pass of 1 + 3 drafts, keep 2
    qg1, k1, v1, _, _ = projections(91, 4, s)
    out4 = torch.zeros((4, s.NH, s.D), device=DEV)
    ctx.layer_attention(0, dev(qg1), dev(k1), dev(v1), dev(qn), dev(kn), out4, base, 4)
    pos = base + 2
    qg2, k2, v2, _, _ = projections(92, 1, s)
    out1 = torch.zeros((1, s.NH, s.D), device=DEV)
    ctx.layer_attention(0, dev(qg2), dev(k2), dev(v2), dev(qn), dev(kn), out1, pos, 1)
    torch.cuda.synchronize()
    # a context that only ever saw the 2 kept tokens
    ctx2 = make_ctx(qw, s, max_ctx=2048, max_tokens=512)
    ctx2.kv_alloc(1, 2048)
    o = torch.zeros((base, s.NH, s.D), device=DEV)
    ctx2.layer_attention(0, dev(qg0), dev(k0), dev(v0), dev(qn), dev(kn), o, 0, base)
    o2 = torch.zeros((2, s.NH, s.D), device=DEV)
    ctx2.layer_attention(0, dev(qg1[:2]), dev(k1[:2]), dev(v1[:2]), dev(qn), dev(kn), o2, base, 2)
    o1 = torch.zeros((1, s.NH, s.D), device=DEV)
    ctx2.layer_attention(0, dev(qg2), dev(k2), dev(v2), dev(qn), dev(kn), o1, pos, 1)
    torch.cuda.synchronize()
    assert np.array_equal(host(out1), host(o1))
    # the same kernel (16-row slices) over 4 and 2 tokens: fp32 rounding apart
    assert np.abs(host(out4)[:2] - host(o2)).max() <= 2e-6


def test_errors_are_status_codes(qw):
    s = QWEN3_NEXT
    ctx = make_ctx(qw, s, max_ctx=1024, max_tokens=64)
    kc, vc = empty_caches(s, 1024)
    q = torch.zeros((8, s.NH, s.D), device=DEV)
    with pytest.raises(qw.QwattnError, match="context overflow") as e:
        ctx.attend_partial(q, kc, vc, 1024, 1024, 1)
    assert e.value.code == qw.ERANGE
    with pytest.raises(qw.QwattnError, match="> 32 rows"):
        ctx.attend_partial(q, kc, vc, 1024, 10, 8)
    with pytest.raises(qw.QwattnError, match="slot"):
        ctx.layer_attention(0, q, q, q, q, q, q, 0, 1)
    with pytest.raises(qw.QwattnError, match="not a multiple of 32"):
        ctx.attend_partial(q, kc, vc, 1000, 0, 1)
    with pytest.raises(qw.QwattnError, match="fused decode"):
        ctx.decode_partial(q, q, q, q, q, ctx.rope_table(), kc, vc, 1024, 10, 9)
    with pytest.raises(qw.QwattnError):
        qw.Attention(16, 3, 256, 64)
