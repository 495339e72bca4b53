"""End-to-end parity on the reference's own tiny qwen4exp model (tests/make_tiny_gguf.py of the reference, checked
there by tests/check_gguf.py:35-48), through the reference's own CPU engine compiled in place.

- CPU: the oracle replays every full-attention layer call of the recorded run (fp32 caches, the oracle's QSA
  indexer) and gives the engine's attention outputs; the compiled engine, run again, reproduces the
  fixture's logits (so the fixture is the engine's, not stale).
- GPU: libqwattn replays the same calls (fp16 caches, its GPU indexer: qwattn_qsa_index /
  qwattn_layer_attention_qsa on the budget-16 QSA layer) within the parity bar; and, run inside the
  reference's engine as its attention body (every full-attention layer's output replaced by libqwattn's),
  the engine's logits keep the argmax and the top-10 ids of the reference run at every call.
"""
import numpy as np
import pytest

from common import assert_rows_parity
from tiny_gguf import GpuLayers, TinyGguf, oracle_layer_replay


@pytest.fixture(scope="module")
def tg():
    return TinyGguf()


def _engine():
    import oracle
    try:
        return oracle.RefQwen4(oracle.TINY_GGUF, max_ctx=4096, threads=4)
    except FileNotFoundError as e:
        pytest.skip(f"reference engine or tiny GGUF not built here ({e}); tests/golden/make_tiny_qwen4exp.py builds both")


def test_fixture_shape(tg):
    """The tiny model's attention layout (make_tiny_gguf.py:10-11): 2 query heads, 1 KV head, head_dim 256,
    rope 64, theta 1e7, and one full-attention layer (the fourth) with QSA blocks of 4 and a budget of 16; the
    indexer selected on most calls."""
    assert (tg.NH, tg.NKV, tg.D, tg.R, tg.IH, tg.ID, tg.budget) == (2, 1, 256, 64, 2, 128, 16)
    assert tg.full == [3] and tg.compress == {3: 4}
    selected = sum(tg.arr(ci, 3, "iq") is not None for ci, _, _ in tg.calls())
    assert selected >= tg.n_calls - 1, selected


def test_oracle_equals_reference_engine_attention(oracle, tg):
    """The oracle's norm/RoPE/cache/QSA-indexer/attention over the recorded projections gives the engine's own
    attention outputs, call after call (prompt, decode steps, a 4-token pass rolled back to 2 kept tokens,
    a 16-token chunk), to fp32 rounding."""
    for layer in tg.full:
        for ci, pos, n, out, ref in oracle_layer_replay(oracle, tg, layer):
            assert np.abs(out - ref).max() <= 2e-6 * (1 + np.abs(ref).max()), (ci, pos, n, np.abs(out - ref).max())


def test_reference_engine_reproduces_fixture(tg):
    """The reference engine compiled here, run on the same tokens and schedule, gives the fixture's logits and
    attention outputs bit for bit."""
    eng = _engine()
    got = {}
    eng.hook = lambda layer, kind, pos, n, arr: got.__setitem__((layer, kind), arr.copy())
    ci = 0
    for op, n, pos in tg.ops:
        if op == 1:
            eng.save_state()
        elif op == 2:
            eng.restore_state()
        else:
            assert eng.pos() == pos
            got.clear()
            logits = eng.forward(tg.tokens(ci))
            assert np.array_equal(logits, tg.logits(ci)), ci
            for layer in tg.full:
                assert np.array_equal(got[(layer, "att")], tg.arr(ci, layer, "att")), ci
            ci += 1
    eng.close()


@pytest.mark.gpu
def test_gpu_replay_equals_reference_engine(qw, tg):
    """libqwattn as the tiny model's attention body, fed the engine's recorded projections call by call (fp16 K/V
    caches, the GPU indexer selecting on the QSA layer), gives the engine's attention outputs within the
    parity bar."""
    gpu = GpuLayers(qw, tg)
    worst = 0.0
    for ci, pos, n in tg.calls():
        for layer in tg.full:
            print(f"tiny gguf replay: call {ci} layer {layer} pos={pos} n={n}", flush=True)
            out = gpu.call(layer, pos, n, *(tg.arr(ci, layer, k) for k in ("qg", "k", "v", "ik", "iq")))
            mx, _ = assert_rows_parity(out, tg.arr(ci, layer, "att"), f"call {ci} pos={pos} n={n}")
            worst = max(worst, mx)
    print(f"tiny gguf replay: worst max-abs {worst:.2e}", flush=True)
    gpu.close()


@pytest.mark.gpu
def test_gpu_attention_inside_reference_engine_same_tokens(qw, tg):
    """The reference's own engine with libqwattn as its attention body (each full-attention layer's output
    replaced, before o_proj, by libqwattn's for the same projections): at every call of the schedule the
    logits' argmax and top-10 ids are the reference run's, and the logits are within 2e-3 of it (the
    reference's own tiny-model tolerance, tests/check_gguf.py:35-48)."""
    eng = _engine()
    gpu = GpuLayers(qw, tg)
    pending = {}

    def hook(layer, kind, pos, n, arr):
        if kind != "att":
            pending[kind] = arr.copy()
            return
        arr[...] = gpu.call(layer, pos, n, pending["qg"], pending["k"], pending["v"], pending.get("ik"),
                            pending.get("iq"))
        pending.clear()

    eng.hook = hook
    ci, worst = 0, 0.0
    for op, n, pos in tg.ops:
        if op == 1:
            eng.save_state()
        elif op == 2:
            eng.restore_state()
        else:
            print(f"tiny gguf engine call {ci} pos={pos} n={n}", flush=True)
            logits = eng.forward(tg.tokens(ci))
            ref = tg.logits(ci)
            assert int(np.argmax(logits)) == int(np.argmax(ref)), ci
            assert set(np.argsort(-logits)[:10]) == set(np.argsort(-ref)[:10]), ci
            worst = max(worst, float(np.abs(logits - ref).max()))
            ci += 1
    print(f"tiny gguf engine: worst logit difference {worst:.2e}", flush=True)
    assert worst <= 2e-3, worst
    gpu.close()
    eng.close()
