"""Writes tests/golden/tiny_qwen4exp_attn.npz: the reference's own qwen4exp engine on the reference's own tiny
model, as its tiny-model check runs it (tests/check_gguf.py:35-48 of the reference, on the output of
tests/make_tiny_gguf.py), observed at its full-attention layers.

Run in the container that holds the reference (not on the GPU box):
    python tests/golden/make_tiny_qwen4exp.py

Steps:
1. The reference's generator script writes the tiny random qwen4exp GGUF (4 layers, the fourth full
   attention with 2 query heads, 1 KV head, head_dim 256, rope 64, and a QSA indexer of 2 heads x 128 dims,
   blocks of 4, a budget of 16 keys) into oracle/_ref/tiny_qwen4exp.gguf. That file is not committed (it is
   the reference's data); it travels with oracle/_ref/ for the GPU test that runs the engine end to end.
2. The reference's CPU engine, compiled in place (oracle/_ref/libref_qwen4.so, see oracle/ref_qwen4_driver.cpp),
   runs a fixed schedule of forward calls: a 24-token prompt, decode steps, a 4-token pass (1 + 3 drafts)
   from a saved state that is then restored and fed its 2 kept tokens (the CPU engine's form of
   accept(2)), more decode steps and a 16-token chunk. The QSA indexer selects from the prompt's 20th token
   on (more than 16 / 4 complete blocks).
3. For every call: the last token's logits, and for the full-attention layer the arrays the engine produced:
   the q|gate, k, v projections, the indexer's raw key / query projections, and the attention body's
   output (the o_proj input). Plus the layer's norm gammas and the model's shape.

The fixture is data only (inputs and outputs); no reference source is copied.
"""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

REF_GEN = "/root/reference/tests/make_tiny_gguf.py"
OUT = os.path.join(ROOT, "tests", "golden", "tiny_qwen4exp_attn.npz")

# (op, n): "fwd" n tokens; "save" / "restore" the engine's state (Backend::save_state / restore_state)
SCHEDULE = ([("fwd", 24)] + [("fwd", 1)] * 6 + [("save", 0), ("fwd", 4), ("restore", 0), ("fwd", 2)]
            + [("fwd", 1)] * 3 + [("fwd", 16)] + [("fwd", 1)] * 2)


def main():
    os.makedirs(os.path.dirname(oracle.TINY_GGUF), exist_ok=True)
    subprocess.run([sys.executable, REF_GEN, oracle.TINY_GGUF], check=True)
    oracle.build(ref=True)
    eng = oracle.RefQwen4(oracle.TINY_GGUF, max_ctx=4096, threads=4)
    full = eng.full_layers()
    rng = np.random.default_rng(2024)
    # a verify pass re-fed after restore must see the same tokens: draw the stream once, index by position
    stream = rng.integers(0, eng.vocab, size=4096).astype(np.int32)
    out = {"shape": np.array([eng.hidden, eng.n_layers, eng.vocab, eng.NH, eng.NKV, eng.D, eng.R, eng.IH, eng.ID,
                              eng.budget], np.int32),
           "eps_theta": np.array([eng.eps, eng.theta], np.float32),
           "full_layers": np.array(full, np.int32),
           "compress": np.array([eng.layers[l][1] for l in full], np.int32)}
    for l in full:
        qn, kn, iqn, ikn = eng.norms(l)
        out[f"L{l}_qn"], out[f"L{l}_kn"], out[f"L{l}_iqn"], out[f"L{l}_ikn"] = qn, kn, iqn, ikn
    rec = {}

    def hook(layer, kind, pos, n, arr):
        rec[(layer, kind)] = arr.copy()

    eng.hook = hook
    ops, ci = [], 0
    for op, n in SCHEDULE:
        if op == "save":
            eng.save_state()
            ops.append((1, 0, eng.pos()))
            continue
        if op == "restore":
            eng.restore_state()
            ops.append((2, 0, eng.pos()))
            continue
        pos = eng.pos()
        rec.clear()
        logits = eng.forward(stream[pos:pos + n])
        out[f"c{ci}_tokens"] = stream[pos:pos + n].copy()
        out[f"c{ci}_logits"] = logits
        for (layer, kind), arr in rec.items():
            out[f"c{ci}_L{layer}_{kind}"] = arr
        ops.append((0, n, pos))
        ci += 1
    out["ops"] = np.array(ops, np.int32)  # (op 0 fwd / 1 save / 2 restore, n, pos before the op)
    eng.close()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {ci} forward calls, full-attention layers {full}, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
