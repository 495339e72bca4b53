"""The reference's tiny qwen4exp model as its own CPU engine ran it (tests/golden/tiny_qwen4exp_attn.npz, written
by tests/golden/make_tiny_qwen4exp.py), and replays of its full-attention layer calls.

A replay walks the recorded schedule: forward calls in order, and a save/restore pair around a 4-token pass
(1 + 3 drafts) that rolls back and re-feeds the 2 kept tokens. Each call of a full-attention layer hands
the attention body the engine's own q|gate, k and v projections (and, on its QSA layers, the indexer's raw
key and query projections) and expects the engine's own attention output (the o_proj input).
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "tiny_qwen4exp_attn.npz")


class TinyGguf:
    def __init__(self, path=FIXTURE):
        f = np.load(path)
        self.f = f
        (self.hidden, self.n_layers, self.vocab, self.NH, self.NKV, self.D, self.R, self.IH, self.ID,
         self.budget) = (int(x) for x in f["shape"])
        self.eps, self.theta = (float(x) for x in f["eps_theta"])
        self.full = [int(x) for x in f["full_layers"]]
        self.compress = dict(zip(self.full, (int(x) for x in f["compress"])))
        self.ops = [tuple(int(x) for x in o) for o in f["ops"]]
        self.n_calls = sum(1 for o in self.ops if o[0] == 0)
        self.max_pos = max(o[1] + o[2] for o in self.ops)

    def norms(self, layer):
        """(q_norm, k_norm, idx_q_norm, idx_k_norm): the engine's gammas (already 1 + w)."""
        f = self.f
        return tuple(f[f"L{layer}_{k}"] for k in ("qn", "kn", "iqn", "ikn"))

    def calls(self):
        """(call index, pos, n) of every forward call, in order (save/restore leave no call of their own)."""
        ci = 0
        for op, n, pos in self.ops:
            if op == 0:
                yield ci, pos, n
                ci += 1

    def arr(self, ci, layer, kind):
        key = f"c{ci}_L{layer}_{kind}"
        return self.f[key] if key in self.f.files else None

    def logits(self, ci):
        return self.f[f"c{ci}_logits"]

    def tokens(self, ci):
        return self.f[f"c{ci}_tokens"]


def oracle_layer_replay(oracle, tg, layer):
    """The oracle's attention over the recorded calls of one layer, with fp32 K/V caches as the reference's CPU
    engine keeps them (src/qwen4_cpu.cpp:318-319) and, on a QSA layer, the oracle's indexer over the recorded
    raw indexer projections (selecting on the calls where the engine selected). Yields (ci, pos, n, out,
    recorded output)."""
    qn, kn, iqn, ikn = tg.norms(layer)
    cr = tg.compress[layer]
    rows = tg.max_pos + 32
    kc = np.zeros((rows, tg.NKV, tg.D), np.float32)
    vc = np.zeros((rows, tg.NKV, tg.D), np.float32)
    raw = np.zeros((rows, tg.ID), np.float32)
    pooled = np.zeros((rows // max(cr, 1) + 1, tg.ID), np.float32)
    mw = (rows // max(cr, 1) + 1 + 31) // 32
    for ci, pos, n in tg.calls():
        qg, k, v = tg.arr(ci, layer, "qg"), tg.arr(ci, layer, "k"), tg.arr(ci, layer, "v")
        rq, rk, rv = oracle.qk_norm_rope(qg, k, v, qn, kn, pos, tg.R, tg.theta, tg.eps)
        kc[pos:pos + n], vc[pos:pos + n] = rk[pos:pos + n], rv[pos:pos + n]
        iq = tg.arr(ci, layer, "iq")
        if cr:
            raw[pos:pos + n] = tg.arr(ci, layer, "ik")
            oracle.qsa_pool(raw, ikn, pos // cr, (pos + n) // cr, cr, tg.R, tg.theta, tg.eps, pooled)
        if cr and iq is not None:
            mask = oracle.qsa_select(iq, iqn, pooled, pos, cr, tg.budget // cr, tg.R, tg.theta, tg.eps, mw)
            out = oracle.attention_qsa(rq, kc[:pos + n], vc[:pos + n], pos, mask, cr, qg)
        else:
            out = oracle.attention(rq, kc[:pos + n], vc[:pos + n], pos, qg)
        yield ci, pos, n, out, tg.arr(ci, layer, "att")


class GpuLayers:
    """libqwattn as the attention body of the tiny model's full-attention layers: one context, one K/V slot per
    layer, and per QSA layer the indexer's raw and pooled key arrays; call() runs one layer call exactly as a
    HIP backend would (qwattn_qsa_pool, or qwattn_qsa_index when the engine's indexer selects, then
    qwattn_layer_attention_qsa; qwattn_layer_attention on a dense call)."""

    def __init__(self, qw, tg, device="cuda:0"):
        import torch
        self.torch, self.tg, self.dev = torch, tg, device
        self.cap = (tg.max_pos + 64 + 31) // 32 * 32
        self.att = qw.Attention(tg.NH, tg.NKV, tg.D, tg.R, tg.theta, tg.eps, max_ctx=self.cap, max_tokens=64,
                                max_splits=256)
        self.slot = {l: i for i, l in enumerate(tg.full)}
        self.att.kv_alloc(len(tg.full), self.cap)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)
        self.d = d
        self.w = {}
        self.qsa = {}
        for l in tg.full:
            qn, kn, iqn, ikn = tg.norms(l)
            # the library takes w with the multiplier 1 + w (the reference's upload stores gamma - 1,
            # src/qwen4_vk.cpp:444-448); the indexer's gammas are used as they are
            self.w[l] = (d(qn - 1.0), d(kn - 1.0), d(iqn), d(ikn))
            cr = tg.compress[l]
            if cr:
                self.qsa[l] = (torch.zeros((self.cap, tg.ID), device=device),
                               torch.zeros((self.cap // cr + 1, tg.ID), device=device))

    def call(self, layer, pos, n, qg, k, v, ik=None, iq=None):
        torch, tg, d = self.torch, self.tg, self.d
        qn, kn, iqn, ikn = self.w[layer]
        out = torch.zeros((n, tg.NH, tg.D), device=self.dev)
        cr = tg.compress[layer]
        if cr:
            raw, pooled = self.qsa[layer]
            if iq is not None:
                kbits = torch.zeros((n, (pos + n + 31) // 32), dtype=torch.int32, device=self.dev)
                self.att.qsa_index(d(ik), d(iq), ikn, iqn, cr, tg.budget, raw, pooled, self.cap, pos, n, None, kbits)
                self.att.layer_attention_qsa(self.slot[layer], d(qg), d(k), d(v), qn, kn, out, pos, n, kbits)
            else:
                self.att.qsa_pool(d(ik), ikn, cr, raw, pooled, self.cap, pos, n)
                self.att.layer_attention(self.slot[layer], d(qg), d(k), d(v), qn, kn, out, pos, n)
        else:
            self.att.layer_attention(self.slot[layer], d(qg), d(k), d(v), qn, kn, out, pos, n)
        self.att.sync_status()
        return out.cpu().numpy()

    def close(self):
        self.att.close()
