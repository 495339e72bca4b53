"""HipBackend : Backend (tests/cxx/hip_backend.cpp), the reference-side binding of libqwattn, linked into a program
(tests/cxx/backend_driver.cpp, built against the reference's own src/backend.h and src/qwen4.h) and driven through
every Backend entry point on the GPU: forward (a prompt longer than one pass chunk is not needed here; a
24-plus-token prompt), decode steps, forward_all over 1 + 3 drafts then accept(2), save_state / restore_state
around a rejected continuation, and reset.

The model is attention-only with one residual stream (the backend refuses anything else): embedding -> per
layer [RMSNorm -> q|gate, k, v projections -> the attention layer body -> o_proj, residual] -> final RMSNorm ->
lm_head, with one dense layer and one QSA layer (blocks of 4, a budget of 16 keys: the indexer selects from the
20th position on), weights in fp32 or GGUF Q8_0. The CPU oracle computes the same model (numpy for the dense
parts, the oracle's attention and QSA indexer for the layer bodies, fp16-rounded cache rows as on the GPU); the
argmax of every returned logit row must agree and the logits stay within 1e-3.
"""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

from common import QWEN3_NEXT, TINY_GGUF
from tiny_model import rmsnorm, top2_margin

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "tests", "cxx"))
import build as cxx_build  # noqa: E402

IH, ID, CR, BUDGET = 2, 128, 4, 16


def q8_quantize(w):
    """fp32 [rows, cols] -> (GGUF Q8_0 blocks uint8 [rows, cols/32*34], the fp32 values they hold)."""
    rows, cols = w.shape
    b = w.reshape(rows, cols // 32, 32)
    d = (np.abs(b).max(axis=2) / 127.0).astype(np.float16)
    q = np.clip(np.rint(b / np.maximum(d.astype(np.float32), 1e-30)[..., None]), -127, 127).astype(np.int8)
    blocks = np.zeros((rows, cols // 32, 34), np.uint8)
    blocks[:, :, 0:2] = d.view(np.uint8).reshape(rows, cols // 32, 2)
    blocks[:, :, 2:] = q.view(np.uint8)
    return blocks.reshape(rows, -1), (q.astype(np.float32) * d.astype(np.float32)[..., None]).reshape(rows, cols)


class Model:
    """Seeded weights of the attention-only stack. Matrices are [rows, cols] as the engine's GMat views hold
    them (y = x W^T); norm gammas are the engine's (1 + w)."""

    def __init__(self, s, hidden, vocab, compress, seed, q8):
        r = np.random.default_rng(seed)
        f = np.float32
        self.s, self.hidden, self.vocab, self.compress, self.q8 = s, hidden, vocab, compress, q8
        self.emb = r.standard_normal((vocab, hidden)).astype(f)

        def m(rows, cols):
            w = (r.standard_normal((rows, cols)) / np.sqrt(cols)).astype(f)
            return q8_quantize(w) if q8 else (w, w)

        self.layers = []
        for cr in compress:
            L = dict(cr=cr, norm=(1 + 0.1 * r.standard_normal(hidden)).astype(f),
                     qn=(1 + 0.1 * r.standard_normal(s.D)).astype(f), kn=(1 + 0.1 * r.standard_normal(s.D)).astype(f),
                     q=m(s.NH * 2 * s.D, hidden), k=m(s.NKV * s.D, hidden), v=m(s.NKV * s.D, hidden),
                     o=m(hidden, s.NH * s.D))
            if cr:
                L.update(iq=m(IH * ID, hidden), ik=m(ID, hidden), iqn=(1 + 0.1 * r.standard_normal(ID)).astype(f),
                         ikn=(1 + 0.1 * r.standard_normal(ID)).astype(f))
            self.layers.append(L)
        self.fnorm = (1 + 0.1 * r.standard_normal(hidden)).astype(f)
        self.out = m(vocab, hidden)

    def write(self, f, max_ctx, ops):
        s = self.s
        f.write(b"QWHB")
        f.write(struct.pack("<12i", self.hidden, len(self.layers), self.vocab, s.NH, s.NKV, s.D, s.R, IH, ID, BUDGET,
                            max_ctx, int(self.q8)))
        f.write(struct.pack("<2f", s.eps, s.theta))
        mat = lambda pair: f.write(np.ascontiguousarray(pair[0]).tobytes())
        for L in self.layers:
            f.write(struct.pack("<i", L["cr"]))
            for k in ("norm", "qn", "kn"):
                f.write(L[k].astype("<f4").tobytes())
            for k in ("q", "k", "v", "o"):
                mat(L[k])
            if L["cr"]:
                mat(L["iq"]), mat(L["ik"])
                f.write(L["iqn"].astype("<f4").tobytes())
                f.write(L["ikn"].astype("<f4").tobytes())
        f.write(self.fnorm.astype("<f4").tobytes())
        f.write(self.emb.astype("<f4").tobytes())
        mat(self.out)
        f.write(struct.pack("<i", len(ops)))
        for code, n, toks in ops:
            f.write(struct.pack("<2i", code, n))
            if toks is not None:
                f.write(np.asarray(toks, "<i4").tobytes())


class OracleRun:
    """The model on the CPU oracle, position by position as the backend runs it."""

    def __init__(self, oracle, model, max_ctx):
        self.o, self.m = oracle, model
        s = model.s
        self.kc = [np.zeros((max_ctx, s.NKV, s.D), np.float32) for _ in model.layers]
        self.vc = [np.zeros((max_ctx, s.NKV, s.D), np.float32) for _ in model.layers]
        self.raw = [np.zeros((max_ctx, ID), np.float32) for _ in model.layers]
        self.pooled = [np.zeros((max_ctx // CR + 1, ID), np.float32) for _ in model.layers]
        self.mw = (max_ctx // CR + 1 + 31) // 32

    def forward(self, ids, pos):
        m, s, o = self.m, self.m.s, self.o
        n = len(ids)
        x = m.emb[np.asarray(ids)]
        for li, L in enumerate(m.layers):
            h = rmsnorm(x, L["norm"])
            qg = (h @ L["q"][1].T).reshape(n, s.NH, 2 * s.D)
            k = (h @ L["k"][1].T).reshape(n, s.NKV, s.D)
            v = (h @ L["v"][1].T).reshape(n, s.NKV, s.D)
            rq, rk, rv = o.qk_norm_rope(qg, k, v, L["qn"], L["kn"], pos, s.R, s.theta, s.eps)
            self.kc[li][pos:pos + n] = rk[pos:pos + n].astype(np.float16)
            self.vc[li][pos:pos + n] = rv[pos:pos + n].astype(np.float16)
            kc, vc = self.kc[li][:pos + n], self.vc[li][:pos + n]
            if L["cr"]:
                self.raw[li][pos:pos + n] = h @ L["ik"][1].T
                o.qsa_pool(self.raw[li], L["ikn"], pos // CR, (pos + n) // CR, CR, s.R, s.theta, s.eps, self.pooled[li])
                iq = (h @ L["iq"][1].T).reshape(n, IH, ID)
                mask = o.qsa_select(iq, L["iqn"], self.pooled[li], pos, CR, BUDGET // CR, s.R, s.theta, s.eps, self.mw)
                att = o.attention_qsa(rq, kc, vc, pos, mask, CR, qg)
            else:
                att = o.attention(rq, kc, vc, pos, qg)
            x = x + att.reshape(n, s.NH * s.D) @ L["o"][1].T
        return rmsnorm(x, m.fnorm) @ m.out[1].T


def _driver():
    if not os.path.exists(cxx_build.BACKEND_OUT):
        if not os.path.exists(os.path.join(cxx_build.REF_SRC, "qwen4.h")):
            pytest.skip("backend_driver not built (it needs the reference's headers; tests/cxx/build.py builds it)")
        cxx_build.build_backend()
    return cxx_build.BACKEND_OUT


def _schedule(vocab, seed):
    """Backend calls: (code, n, tokens); the positions each op leaves; and the oracle's (tokens, pos, all rows)."""
    r = np.random.default_rng(seed)
    tok = lambda n: [int(t) for t in r.integers(0, vocab, n)]
    ops = [(0, 24, tok(24))] + [(0, 1, tok(1)) for _ in range(3)]
    ops += [(3, 0, None), (1, 4, tok(4)), (2, 2, None), (0, 1, tok(1)), (0, 1, tok(1)), (4, 0, None), (0, 3, tok(3))]
    ops += [(1, 4, tok(4)), (2, 1, None), (0, 1, tok(1)), (5, 0, None), (0, 5, tok(5)), (0, 1, tok(1))]
    pos, spec0, saved, positions, calls = 0, 0, 0, [], []
    for code, n, toks in ops:
        if code in (0, 1):
            calls.append((toks, pos, code == 1))
            if code == 1:
                spec0 = pos
            pos += n
        elif code == 2:
            pos = spec0 + n
        elif code == 3:
            saved = pos
        elif code == 4:
            pos = saved
        elif code == 5:
            pos = 0
        positions.append(pos)
    return ops, positions, calls


CASES = [(TINY_GGUF, 256, 0, 11), (TINY_GGUF, 256, 1, 12), (QWEN3_NEXT, 512, 1, 13)]


@pytest.mark.gpu
@pytest.mark.parametrize("s,hidden,q8,seed", CASES, ids=lambda v: repr(v))
def test_hip_backend_through_backend_interface(oracle, tmp_path, s, hidden, q8, seed):
    vocab, max_ctx = 256, 128
    model = Model(s, hidden, vocab, [0, CR], seed, q8)
    ops, positions, calls = _schedule(vocab, seed + 100)
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        model.write(f, max_ctx, ops)
    print(f"backend_driver {s} hidden={hidden} q8={q8}: {len(ops)} Backend calls", flush=True)
    r = subprocess.run([_driver(), str(inp), str(outp)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stderr)
    raw = np.fromfile(outp, dtype="<f4")
    n_logits = sum(len(t) if all_rows else 1 for t, _, all_rows in calls) * vocab
    got_pos = raw[n_logits:].view("<i4")
    assert list(got_pos) == positions
    orc = OracleRun(oracle, model, max_ctx)
    off, worst = 0, 0.0
    for i, (toks, pos, all_rows) in enumerate(calls):
        ref = orc.forward(toks, pos)
        if not all_rows:
            ref = ref[-1:]
        got = raw[off:off + ref.size].reshape(ref.shape)
        off += ref.size
        assert float(np.min(top2_margin(ref))) > 2e-3, f"call {i}: a near-tie in the oracle's logits"
        assert np.array_equal(np.argmax(got, -1), np.argmax(ref, -1)), f"call {i} pos={pos}"
        worst = max(worst, float(np.abs(got - ref).max()))
    print(f"backend_driver: worst logit difference {worst:.2e}", flush=True)
    assert worst <= 1e-3


def test_hip_backend_builds_against_reference_headers():
    """The program links HipBackend against the reference's Backend / Q4Config headers and libqwattn (where the
    reference sources are present; the built program is what the GPU test runs)."""
    if not os.path.exists(os.path.join(cxx_build.REF_SRC, "qwen4.h")):
        pytest.skip("reference sources not present")
    assert os.path.exists(cxx_build.build_backend())
