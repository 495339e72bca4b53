"""GPU parity of the projection kernel (qwattn_mat: Qwen4Vulkan::mat, src/qwen4_vk.cpp:848-856, on the
q4_matmul_q8 / q4_matmul_f32 pipelines of shaders/q4_matmul.comp) against the CPU oracle's projection, itself
pinned against the reference's own CPU path (tests/test_oracle.py: test_mat_q8_matches_reference).

Tolerance: every output is one fp32 dot product in both, summed in different orders, so the bound is relative
to the magnitude sum |W| |x| of that output: 1e-5 of it (a few fp32 roundings of a 4,096-term sum) plus 1e-6."""
import numpy as np
import pytest
import torch

from common import q8_blocks

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _ctx(qw):
    return qw.Attention(16, 2, 256, 64, max_ctx=1024, max_tokens=64, max_splits=16)


def _check(got, want, w_abs, x):
    mag = w_abs.astype(np.float64) @ np.abs(x.astype(np.float64)).T  # [rows, n]
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= 1e-5 * mag.T + 1e-6), float((err / (mag.T + 1e-30)).max())


# (rows, cols): the attention layer's projections at hidden 2,048 (query + gate, key, value, output), then odd
# shapes: a partial last workgroup of rows (one row a wave below 4,096 rows, four from there), a column count
# that leaves lanes idle
SHAPES = [(8192, 2048), (512, 2048), (2048, 4096), (100, 96), (37, 1056), (4100, 96)]


@pytest.mark.parametrize("rows,cols", SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize("n", [1, 4, 5, 13])
def test_mat_q8_parity(qw, oracle, rows, cols, n):
    print(f"mat q8 {rows}x{cols} n={n}", flush=True)
    blocks, _, _ = q8_blocks(71 + rows + n, rows, cols)
    w8, s = qw.q8_unpack(blocks, rows, cols)
    x = np.random.default_rng(72 + n).standard_normal((n, cols)).astype(np.float32)
    ctx = _ctx(qw)
    y = torch.full((n, rows), float("nan"), device=DEV)
    ctx.mat(dev(x), y, dev(w8), dev(s))
    torch.cuda.synchronize()
    want = oracle.mat(x, w8=w8, s=s)
    _check(y.cpu().numpy(), want, np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)), x)
    ctx.close()


@pytest.mark.parametrize("rows,cols,n", [(512, 2048, 1), (300, 48, 6), (2048, 4096, 4)])
def test_mat_f32_parity(qw, oracle, rows, cols, n):
    print(f"mat f32 {rows}x{cols} n={n}", flush=True)
    r = np.random.default_rng(73)
    w = (0.05 * r.standard_normal((rows, cols))).astype(np.float32)
    x = r.standard_normal((n, cols)).astype(np.float32)
    ctx = _ctx(qw)
    y = torch.full((n, rows), float("nan"), device=DEV)
    ctx.mat(dev(x), y, dev(w))
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), oracle.mat(x, wf=w), np.abs(w), x)
    ctx.close()


def test_mat_strides_and_post(qw, oracle):
    """Row strides wider than the rows (the reference's x_stride / y_stride), outputs beyond `rows` of each y
    row untouched, and post 1 = silu(y * post_scale)."""
    rows, cols, n = 200, 512, 3
    blocks, _, _ = q8_blocks(74, rows, cols)
    w8, s = qw.q8_unpack(blocks, rows, cols)
    x = np.random.default_rng(75).standard_normal((n, cols + 64)).astype(np.float32)
    ctx = _ctx(qw)
    xd = dev(x)[:, :cols]
    y = torch.full((n, rows + 24), 7.0, device=DEV)
    ctx.mat(xd, y, dev(w8), dev(s), post=1, post_scale=0.37)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = oracle.mat(x[:, :cols], w8=w8, s=s, post=1, post_scale=0.37)
    _check(got[:, :rows], want, np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)), x[:, :cols])
    assert np.all(got[:, rows:] == 7.0)
    ctx.close()


def test_mat_rejects_bad_shapes(qw):
    ctx = _ctx(qw)
    w = torch.zeros((64, 48), dtype=torch.int8, device=DEV)  # 48 columns: not whole Q8 blocks
    s = torch.zeros((64, 1), device=DEV)
    x = torch.zeros((1, 48), device=DEV)
    y = torch.zeros((1, 64), device=DEV)
    with pytest.raises(qw.QwattnError):
        ctx.mat(x, y, w, s)
    ctx.close()


# The MFMA kernels from 16 tokens (columns a multiple of 32). Q8 up to 64 tokens, Q8 matrices of up to 1,024
# rows at any token count, and Q8 launches the GEMM would cut into fewer than 256 tiles: the skinny kernel with 16, 32 or 64 tokens a workgroup (partial row and
# token groups, waves with no column blocks at 96 columns); otherwise, and fp32 weights: the tiled GEMM with
# each token tile width (128 when that still gives 512 workgroups, else 64 when that does, else 32). The
# attention layer's shapes among them.
GEMM_CASES = [(512, 2048, 16), (512, 2048, 200), (100, 96, 33), (37, 1056, 130), (2048, 4096, 64),
              (8192, 2048, 20), (300, 64, 257), (160, 256, 1100), (64, 64, 1500),
              (8192, 64, 512), (8000, 96, 530), (8192, 64, 1100), (8000, 96, 1030),
              (70, 64, 24), (45, 160, 17), (8192, 2048, 64), (33, 2048, 61), (2000, 96, 100), (1100, 64, 300), (4096, 64, 300), (2048, 64, 100)]


@pytest.mark.parametrize("rows,cols,n", GEMM_CASES, ids=lambda v: str(v))
def test_gemm_q8_parity(qw, oracle, rows, cols, n):
    print(f"gemm q8 {rows}x{cols} n={n}", flush=True)
    blocks, _, _ = q8_blocks(81 + rows + n, rows, cols)
    w8, s = qw.q8_unpack(blocks, rows, cols)
    x = np.random.default_rng(82 + n).standard_normal((n, cols)).astype(np.float32)
    ctx = _ctx(qw)
    y = torch.full((n, rows), float("nan"), device=DEV)
    ctx.mat(dev(x), y, dev(w8), dev(s))
    torch.cuda.synchronize()
    want = oracle.mat(x, w8=w8, s=s)
    _check(y.cpu().numpy(), want, np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)), x)
    ctx.close()


@pytest.mark.parametrize("rows,cols,n", [(300, 64, 40), (512, 2048, 130), (130, 96, 17), (200, 128, 1030),
                                          (8000, 64, 530), (8192, 64, 1030)],
                         ids=lambda v: str(v))
def test_gemm_f32_parity(qw, oracle, rows, cols, n):
    print(f"gemm f32 {rows}x{cols} n={n}", flush=True)
    r = np.random.default_rng(83)
    w = (0.05 * r.standard_normal((rows, cols))).astype(np.float32)
    x = r.standard_normal((n, cols)).astype(np.float32)
    ctx = _ctx(qw)
    y = torch.full((n, rows), float("nan"), device=DEV)
    ctx.mat(dev(x), y, dev(w))
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), oracle.mat(x, wf=w), np.abs(w), x)
    ctx.close()


@pytest.mark.parametrize("n", [40, 200])
def test_gemm_strides_post_and_scale_range(qw, oracle, n):
    """The MFMA kernels (skinny at 40 tokens, tiled at 200) with x_stride / y_stride wider than the rows,
    post 1, outputs beyond `rows` untouched, and inputs whose magnitudes span 2^-20 .. 2^20 (the hi / lo
    split keeps fp32 range and relative accuracy)."""
    rows, cols = 200, 512
    blocks, _, _ = q8_blocks(84, rows, cols)
    w8, s = qw.q8_unpack(blocks, rows, cols)
    r = np.random.default_rng(85)
    x = (r.standard_normal((n, cols + 32)) * np.exp2(r.integers(-20, 21, (n, cols + 32)))).astype(np.float32)
    ctx = _ctx(qw)
    y = torch.full((n, rows + 8), 7.0, device=DEV)
    ctx.mat(dev(x)[:, :cols], y, dev(w8), dev(s), post=1, post_scale=1e-3)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = oracle.mat(x[:, :cols], w8=w8, s=s, post=1, post_scale=1e-3)
    _check(got[:, :rows], want, np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)), x[:, :cols])
    assert np.all(got[:, rows:] == 7.0)
    ctx.close()


def test_gemm_full_prefill_matches_matvec(qw):
    """At the full prefill size (2,048 tokens through the 8,192 x 2,048 query + gate projection, too large for
    the CPU oracle in a test) each token's outputs do not depend on the batch: the GEMM's rows for a spread of
    tokens equal the matrix-vector kernel's outputs for those tokens alone (both kernels are pinned to the
    oracle above), to the same tolerance."""
    rows, cols, n = 8192, 2048, 2048
    blocks, _, _ = q8_blocks(86, rows, cols)
    w8, s = qw.q8_unpack(blocks, rows, cols)
    x = np.random.default_rng(87).standard_normal((n, cols)).astype(np.float32)
    ctx = _ctx(qw)
    wd, sd, xd = dev(w8), dev(s), dev(x)
    y = torch.empty((n, rows), device=DEV)
    ctx.mat(xd, y, wd, sd)
    pick = [0, 1, 63, 64, 127, 128, 1000, 2047]
    ys = torch.empty((len(pick), rows), device=DEV)
    ctx.mat(xd[pick].contiguous(), ys, wd, sd)  # 8 tokens: the matrix-vector kernel
    torch.cuda.synchronize()
    mag = np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)).astype(np.float64) @ np.abs(x[pick]).T.astype(np.float64)
    err = np.abs(y.cpu().numpy()[pick].astype(np.float64) - ys.cpu().numpy())
    assert np.all(err <= 2e-5 * mag.T + 2e-6), float((err / mag.T).max())
    assert np.isfinite(y.cpu().numpy()).all()
    ctx.close()


@pytest.mark.parametrize("n", [1, 4, 5, 40])
def test_mat_multi_equals_separate_calls(qw, oracle, n):
    """qwattn_mat_multi (one matrix-vector launch over several matrices below 16 tokens, one GEMM a matrix
    from 16) gives each matrix the bits of its own qwattn_mat call, and the oracle's values: the attention
    layer's query + gate, key and value projections of one input (8,192 + 512 + 512 rows, one row a wave
    below 4,096 rows in total, four from there), then three small ones."""
    print(f"mat_multi n={n}", flush=True)
    ctx = _ctx(qw)
    for shapes, cols in (([8192, 512, 512], 2048), ([100, 36, 64], 96)):
        x = np.random.default_rng(91 + n).standard_normal((n, cols)).astype(np.float32)
        xd = dev(x)
        mats, outs, sep = [], [], []
        for i, rows in enumerate(shapes):
            blocks, _, _ = q8_blocks(92 + i + rows, rows, cols)
            w8, s = qw.q8_unpack(blocks, rows, cols)
            mats.append((w8, s))
            wd, sd = dev(w8), dev(s)
            y = torch.full((n, rows + 3), 7.0, device=DEV)[:, :rows]
            outs.append((y, wd, sd))
            ys = torch.empty((n, rows), device=DEV)
            ctx.mat(xd, ys, wd, sd)
            sep.append(ys)
        ctx.mat_multi(xd, outs)
        torch.cuda.synchronize()
        for (y, _, _), ys, (w8, s) in zip(outs, sep, mats):
            assert torch.equal(y, ys)
            want = oracle.mat(x, w8=w8, s=s)
            _check(y.cpu().numpy(), want, np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)), x)
    ctx.close()


def test_mat_multi_rejects_bad_input(qw):
    ctx = _ctx(qw)
    x = torch.zeros((1, 64), device=DEV)
    w = torch.zeros((32, 64), dtype=torch.int8, device=DEV)
    s = torch.zeros((32, 2), device=DEV)
    y = torch.zeros((1, 32), device=DEV)
    with pytest.raises(qw.QwattnError):
        ctx.mat_multi(x, [(y, w, s)] * 5)  # more than 4 matrices
    w48 = torch.zeros((32, 48), dtype=torch.int8, device=DEV)
    with pytest.raises(qw.QwattnError):
        ctx.mat_multi(x[:, :48], [(y, w48, s[:, :1].contiguous())])  # 48 columns: not whole Q8 blocks
    with pytest.raises(ValueError):
        ctx.mat_multi(x, [(y, w, s), (y, torch.zeros((32, 96), dtype=torch.int8, device=DEV), s)])  # column counts
    with pytest.raises(ValueError):
        ctx.mat_multi(x[:, :32], [(y, w, s)])  # x narrower than the weights
    ctx.close()


@pytest.mark.parametrize("n", [1, 4, 20])
def test_mat_multi_padded_x(qw, oracle, n):
    """A padded input (x wider than the weights' columns, row stride beyond them) gives each matrix of
    qwattn_mat_multi the bits of qwattn_mat on the same operands: the column count is the weights', not x's."""
    print(f"mat_multi padded x n={n}", flush=True)
    ctx = _ctx(qw)
    rows_list, cols, pad = (96, 40, 64), 128, 64
    x = np.random.default_rng(97 + n).standard_normal((n, cols + pad)).astype(np.float32)
    xd = dev(x)
    outs, sep, mats = [], [], []
    for i, rows in enumerate(rows_list):
        blocks, _, _ = q8_blocks(98 + i, rows, cols)
        w8, s = qw.q8_unpack(blocks, rows, cols)
        mats.append((w8, s))
        wd, sd = dev(w8), dev(s)
        y = torch.empty((n, rows), device=DEV)
        outs.append((y, wd, sd))
        ys = torch.empty((n, rows), device=DEV)
        ctx.mat(xd, ys, wd, sd)
        sep.append(ys)
    ctx.mat_multi(xd, outs)
    torch.cuda.synchronize()
    for (y, _, _), ys, (w8, s) in zip(outs, sep, mats):
        assert torch.equal(y, ys)
        _check(y.cpu().numpy(), oracle.mat(x[:, :cols], w8=w8, s=s),
               np.abs(w8.astype(np.float32) * np.repeat(s, 32, axis=1)), x[:, :cols])
    ctx.close()


@pytest.mark.parametrize("n", [1, 4, 20])
def test_mat_multi_f32_equals_separate_calls(qw, oracle, n):
    """qwattn_mat_multi on fp32 weights (the matrix-vector kernel below 16 tokens, the GEMM from 16): each
    matrix gets the bits of its own qwattn_mat call and the oracle's values."""
    print(f"mat_multi f32 n={n}", flush=True)
    ctx = _ctx(qw)
    r = np.random.default_rng(95 + n)
    cols = 128
    x = r.standard_normal((n, cols)).astype(np.float32)
    xd = dev(x)
    outs, sep, ws = [], [], []
    for rows in (96, 40, 200):
        w = (0.05 * r.standard_normal((rows, cols))).astype(np.float32)
        ws.append(w)
        wd = dev(w)
        y = torch.empty((n, rows), device=DEV)
        outs.append((y, wd, None))
        ys = torch.empty((n, rows), device=DEV)
        ctx.mat(xd, ys, wd)
        sep.append(ys)
    ctx.mat_multi(xd, outs)
    torch.cuda.synchronize()
    for (y, _, _), ys, w in zip(outs, sep, ws):
        assert torch.equal(y, ys)
        _check(y.cpu().numpy(), oracle.mat(x, wf=w), np.abs(w), x)
    ctx.close()
