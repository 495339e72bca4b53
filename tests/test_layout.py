"""The blocked K/V cache layout of include/qwattn.h, checked element by element on the CPU.

The Python mirror's k_block/v_block (used by every GPU test to build and read caches) must place row
element (position p, KV head h, dim d) where the kernels address it:
  part  = (h * cap/32 + p/32) * 32*D                      (head-major, blocks in position order)
  K     = part + ((((d/32)*2 + (kb/4)%2)*4 + (d/8)%4)*16 + (kb/8)*4 + kb%4)*8 + d%8,   kb = p % 32
  V     = part + (((d/16)*4 + kb/8)*16 + d%16)*8 + kb%8
k_rows/v_rows must invert them.
"""
import numpy as np
import pytest

from common import load_package


def k_index(p, h, d, cap, D):
    kb = p % 32
    part = (h * (cap // 32) + p // 32) * 32 * D
    return part + ((((d // 32) * 2 + (kb // 4) % 2) * 4 + (d // 8) % 4) * 16 + (kb // 8) * 4 + kb % 4) * 8 + d % 8


def v_index(p, h, d, cap, D):
    kb = p % 32
    part = (h * (cap // 32) + p // 32) * 32 * D
    return part + (((d // 16) * 4 + kb // 8) * 16 + d % 16) * 8 + kb % 8


@pytest.mark.parametrize("cap,nkv,D", [(32, 1, 64), (64, 2, 64), (96, 2, 256), (64, 3, 128)])
def test_block_layout_matches_formulas(cap, nkv, D):
    import torch
    qw = load_package()
    # every element distinct (exact in fp32 up to 2^24)
    rows = torch.arange(cap * nkv * D, dtype=torch.float32).reshape(cap, nkv, D)
    kb, vb = qw.k_block(rows).numpy(), qw.v_block(rows).numpy()
    p, h, d = np.meshgrid(np.arange(cap), np.arange(nkv), np.arange(D), indexing="ij")
    r = rows.numpy()
    assert np.array_equal(kb[k_index(p, h, d, cap, D)], r)
    assert np.array_equal(vb[v_index(p, h, d, cap, D)], r)
    # both maps are permutations of the whole cache
    assert np.unique(k_index(p, h, d, cap, D)).size == cap * nkv * D
    assert np.unique(v_index(p, h, d, cap, D)).size == cap * nkv * D
    assert torch.equal(qw.k_rows(qw.k_block(rows), cap, nkv, D), rows)
    assert torch.equal(qw.v_rows(qw.v_block(rows), cap, nkv, D), rows)


def test_head_region_is_contiguous_and_grows_by_prefix():
    """A head's positions [0, cap) occupy one contiguous range, and growing the capacity keeps each head's
    old range as the prefix of its new one (what qwattn_kv_grow copies)."""
    import torch
    qw = load_package()
    D, nkv, cap, cap2 = 64, 2, 64, 128
    rows = torch.randn(cap2, nkv, D)
    small = qw.k_block(rows[:cap].contiguous()).view(nkv, cap * D)
    big = qw.k_block(rows).view(nkv, cap2 * D)
    for h in range(nkv):
        assert torch.equal(big[h, :cap * D], small[h])
    small_v = qw.v_block(rows[:cap].contiguous()).view(nkv, cap * D)
    big_v = qw.v_block(rows).view(nkv, cap2 * D)
    for h in range(nkv):
        assert torch.equal(big_v[h, :cap * D], small_v[h])
