"""An attention-only tiny language model for end-to-end argmax parity.

The reference's own tiny model (tests/make_tiny_gguf.py, checked by tests/check_gguf.py:35-48) needs the
whole qwen4exp stack, which is outside the attention hot path. This model keeps only what feeds and
consumes attention: seeded embedding -> per layer [RMSNorm -> q|gate, k, v projections -> the attention
layer body (QK-RMSNorm with (1 + w), partial RoPE, fp16 K/V cache append, causal GQA attention, sigmoid
gate) -> o_proj, residual] -> final RMSNorm -> lm_head. The dense parts run in numpy fp32 on the host for
every backend, so two runs differ only in the attention layer body that is plugged in.
"""
import numpy as np


def rmsnorm(x, w, eps=1e-6):
    x = x.astype(np.float32)
    return (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w).astype(np.float32)


class TinyModel:
    def __init__(self, s, hidden, vocab, layers, seed):
        rng = np.random.default_rng(seed)
        f = np.float32
        self.s, self.hidden, self.vocab, self.layers = s, hidden, vocab, layers
        self.emb = rng.standard_normal((vocab, hidden)).astype(f)
        self.lw = []
        for _ in range(layers):
            self.lw.append(dict(
                norm=(1 + 0.1 * rng.standard_normal(hidden)).astype(f),
                wqg=(rng.standard_normal((hidden, s.NH * 2 * s.D)) / np.sqrt(hidden)).astype(f),
                wk=(rng.standard_normal((hidden, s.NKV * s.D)) / np.sqrt(hidden)).astype(f),
                wv=(rng.standard_normal((hidden, s.NKV * s.D)) / np.sqrt(hidden)).astype(f),
                wo=(rng.standard_normal((s.NH * s.D, hidden)) / np.sqrt(s.NH * s.D)).astype(f),
                qn=(0.1 * rng.standard_normal(s.D)).astype(f),  # QK-norm weights w: multiplier 1 + w
                kn=(0.1 * rng.standard_normal(s.D)).astype(f)))
        self.fnorm = (1 + 0.1 * rng.standard_normal(hidden)).astype(f)
        self.lm_head = (rng.standard_normal((hidden, vocab)) / np.sqrt(hidden)).astype(f)

    def forward(self, ids, pos, attend):
        """Logits [n, vocab] of tokens `ids` at positions pos .. pos+n-1. attend(layer, qg [n,NH,2D],
        k [n,NKV,D], v [n,NKV,D], qn, kn, pos, n) -> attention output [n, NH, D] (gate applied) and
        appends the tokens' K/V to that layer's cache."""
        s = self.s
        n = len(ids)
        x = self.emb[np.asarray(ids)]
        for li, w in enumerate(self.lw):
            h = rmsnorm(x, w["norm"])
            qg = (h @ w["wqg"]).reshape(n, s.NH, 2 * s.D)
            k = (h @ w["wk"]).reshape(n, s.NKV, s.D)
            v = (h @ w["wv"]).reshape(n, s.NKV, s.D)
            o = attend(li, qg, k, v, w["qn"], w["kn"], pos, n)
            x = x + np.asarray(o, np.float32).reshape(n, s.NH * s.D) @ w["wo"]
        return rmsnorm(x, self.fnorm) @ self.lm_head


class OracleAttention:
    """The attention layer body on the CPU oracle, with per-layer fp32 caches holding fp16-rounded rows
    (the cache is fp16 on every backend). chunk > 0 uses the oracle's split-KV + LSE-combine form."""

    def __init__(self, oracle, s, layers, max_ctx, chunk=0):
        self.o, self.s, self.chunk = oracle, s, chunk
        self.kc = [np.zeros((max_ctx, s.NKV, s.D), np.float32) for _ in range(layers)]
        self.vc = [np.zeros((max_ctx, s.NKV, s.D), np.float32) for _ in range(layers)]

    def __call__(self, li, qg, k, v, qn, kn, pos, n):
        s = self.s
        rq, rk, rv = self.o.qk_norm_rope(qg, k, v, 1 + qn, 1 + kn, pos, s.R, s.theta, s.eps)
        self.kc[li][pos:pos + n] = rk[pos:pos + n].astype(np.float16)
        self.vc[li][pos:pos + n] = rv[pos:pos + n].astype(np.float16)
        if self.chunk:
            return self.o.attention_split(rq, self.kc[li][:pos + n], self.vc[li][:pos + n], pos, self.chunk, qg)
        return self.o.attention(rq, self.kc[li][:pos + n], self.vc[li][:pos + n], pos, qg)


def run(model, attend, prompt, schedule):
    """Prefill `prompt`, then feed each chunk of `schedule` (lists of token ids; a chunk of several ids
    is a multi-token verify pass). Returns the logits of every fed token, in order."""
    out = [model.forward(prompt, 0, attend)]
    pos = len(prompt)
    for ids in schedule:
        out.append(model.forward(ids, pos, attend))
        pos += len(ids)
    return np.concatenate(out, axis=0)


def greedy_schedule(model, attend, prompt, steps, verify_at=None):
    """A decode schedule built greedily from the reference backend: each step feeds the argmax of the
    previous step; at step `verify_at` the next 4 greedy tokens go in as one verify pass instead."""
    logits = model.forward(prompt, 0, attend)
    pos = len(prompt)
    nxt = int(np.argmax(logits[-1]))
    sched = []
    while len(sched) < steps:
        if verify_at is not None and len(sched) == verify_at:
            ids = [nxt]
            for _ in range(3):  # draft tokens: greedy continuations, fed together
                ids.append((ids[-1] * 7 + 3) % model.vocab)
        else:
            ids = [nxt]
        lg = model.forward(ids, pos, attend)
        sched.append(ids)
        pos += len(ids)
        nxt = int(np.argmax(lg[-1]))
    return sched


def top2_margin(logits):
    part = np.partition(logits, -2, axis=-1)
    return part[..., -1] - part[..., -2]
