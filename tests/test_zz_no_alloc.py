"""qwattn_decode_noalloc (no context, library-static scratch) computes exactly what qwattn_decode
computes: the same kernels, split counts and merge order, so the outputs and the appended cache rows are
bit-identical. Two calls in a row, the second with a smaller input; the one-launch path (n = 1) and the
verify path (n = 4: the 16-row-slice kernel, its slices' last chunks combining) both run."""
import numpy as np
import pytest
import torch

from common import QWEN3_NEXT, projections, cache_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _setup(qw, s, pos, n, seed):
    rows = pos + n
    cap = (rows + 31) // 32 * 32
    k16, v16 = cache_rows(seed, pos, s)
    qg, k, v, qn, kn = projections(seed + 1, n, s)
    krows = torch.zeros((cap, s.NKV, s.D), dtype=torch.float16, device=DEV)
    vrows = torch.zeros((cap, s.NKV, s.D), dtype=torch.float16, device=DEV)
    krows[:pos] = torch.from_numpy(k16).to(DEV)
    vrows[:pos] = torch.from_numpy(v16).to(DEV)
    d = lambda x: torch.from_numpy(x).to(DEV)
    return cap, d(qg), d(k), d(v), d(qn), d(kn), qw.k_block(krows), qw.v_block(vrows)


@pytest.mark.parametrize("calls", [[(9000, 4, 0), (3000, 1, 0)], [(20000, 1, 64), (700, 1, 0)]], ids=["verify_then_decode", "decode_then_decode"])
def test_decode_noalloc_matches_decode(qw, calls):
    s = QWEN3_NEXT
    ctx = qw.Attention(s.NH, s.NKV, s.D, s.R, s.theta, s.eps, max_ctx=32768, max_tokens=64, max_splits=1024)
    rope = ctx.rope_table()
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    for pos, n, n_split in calls:
        print(f"noalloc vs decode: pos={pos} n={n} splits={n_split or 'auto'}", flush=True)
        cap, qg, k, v, qn, kn, kc, vc = _setup(qw, s, pos, n, 300 + pos)
        kc2, vc2 = kc.clone(), vc.clone()
        ref = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
        used = ctx.decode(qg, k, v, qn, kn, rope, kc, vc, cap, ref, pos, n, n_split)
        out = torch.full((n, s.NH, s.D), float("nan"), device=DEV)
        used2 = qw.decode_noalloc(ctx.cfg, qg, k, v, qn, kn, rope, kc2, vc2, cap, out, pos, n, n_split, status)
        torch.cuda.synchronize()
        ctx.sync_status()
        assert used2 == used
        assert int(status.item()) == 0
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
        assert torch.equal(out, ref), float((out - ref).abs().max())
    ctx.close()


def test_decode_noalloc_rejects_beyond_scratch(qw):
    """A split count whose partials exceed the 32 MiB scratch is rejected before any launch: the 4-token
    verify path, which runs a requested count exactly (4,096 splits x 64 rows). Every buffer is sized for
    the call, so nothing could be touched out of bounds even if a launch did happen."""
    s = QWEN3_NEXT
    cfg = qw.Config(s.NH, s.NKV, s.D, s.R, s.theta, s.eps, 262144, 64, 4096)
    pos, n, cap = 262100, 4, 262144
    qg = torch.zeros((n, s.NH, 2 * s.D), device=DEV)
    k = torch.zeros((n, s.NKV, s.D), device=DEV)
    v = torch.zeros((n, s.NKV, s.D), device=DEV)
    w = torch.zeros(s.D, device=DEV)
    rope = torch.zeros((cap, s.R // 2, 2), device=DEV)
    kc = torch.zeros(cap * s.NKV * s.D, dtype=torch.float16, device=DEV)
    vc = torch.zeros(cap * s.NKV * s.D, dtype=torch.float16, device=DEV)
    out = torch.zeros((n, s.NH, s.D), device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    with pytest.raises(qw.QwattnError, match="scratch") as e:
        qw.decode_noalloc(cfg, qg, k, v, w, w, rope, kc, vc, cap, out, pos, n, 4096, status)
    assert e.value.code == qw.EINVAL
    torch.cuda.synchronize()
    assert int(status.item()) == 0
