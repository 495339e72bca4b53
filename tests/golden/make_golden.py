"""Writes tests/golden/attn_*.npz: seeded inputs and fp64 outputs of the full-attention hot path.

The generator is SplitMix64 + Box-Muller (portable: any host reproduces the same inputs from the seed).
The outputs are computed here in float64 numpy, independently of oracle/: per (token, head)
  y = x / sqrt(mean(x^2) + eps) * (1 + w)                          (src/qwen4_cpu.cpp:19-23)
  rotate-half on pairs (i, i + R/2), angle = fp32((float)p * inv_freq[i]) (src/qwen4_cpu.cpp:281-289)
  inv_freq[i] = (float)(1 / theta^(2i/R))                            (src/qwen4_cpu.cpp:38-39)
  out = softmax(q . K^T / sqrt(D)) V * sigmoid(gate), causal, GQA     (src/qwen4_cpu.cpp:346-372)
Run: python tests/golden/make_golden.py  (writes next to this file)
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


def splitmix64(seed, n):
    out = np.empty(n, dtype=np.uint64)
    s = seed & M64
    for i in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out[i] = z ^ (z >> 31)
    return out


def normal(seed, shape):
    n = int(np.prod(shape))
    u = splitmix64(seed, 2 * ((n + 1) // 2))
    u = (u >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log1p(-u1))  # 1 - u1 in (0, 1]
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return z.reshape(shape)


def inv_freq(R, theta):
    return np.array([np.float32(1.0 / theta ** (2.0 * i / R)) for i in range(R // 2)], np.float32)


def norm_rope(x, w, p, R, theta, eps):
    D = x.shape[-1]
    y = x / np.sqrt(np.mean(x * x) + eps) * (1.0 + w)
    inv = inv_freq(R, theta)
    ang = (np.float32(p) * inv).astype(np.float64)  # the fp32 product, then exact trigonometry
    a, b = y[:R // 2].copy(), y[R // 2:R].copy()
    y[:R // 2] = a * np.cos(ang) - b * np.sin(ang)
    y[R // 2:R] = b * np.cos(ang) + a * np.sin(ang)
    return y


def make(name, seed, NH, NKV, D, R, pos, n, theta=1e7, eps=1e-6):
    G = NH // NKV
    qg = normal(seed, (n, NH, 2 * D)).astype(np.float32)
    k = normal(seed + 1, (n, NKV, D)).astype(np.float32)
    v = normal(seed + 2, (n, NKV, D)).astype(np.float32)
    wq = (0.1 * normal(seed + 3, (D,))).astype(np.float32)
    wk = (0.1 * normal(seed + 4, (D,))).astype(np.float32)
    # cache rows before pos: post-norm keys and values, fp16-representable
    kc0 = normal(seed + 5, (pos, NKV, D)).astype(np.float16).astype(np.float32)
    vc0 = normal(seed + 6, (pos, NKV, D)).astype(np.float16).astype(np.float32)
    q_out = np.zeros((n, NH, D))
    k_new = np.zeros((n, NKV, D))
    for t in range(n):
        for h in range(NH):
            q_out[t, h] = norm_rope(qg[t, h, :D].astype(np.float64), wq.astype(np.float64), pos + t, R, theta, eps)
        for h in range(NKV):
            k_new[t, h] = norm_rope(k[t, h].astype(np.float64), wk.astype(np.float64), pos + t, R, theta, eps)
    K = np.concatenate([kc0.astype(np.float64), k_new])
    V = np.concatenate([vc0.astype(np.float64), v.astype(np.float64)])
    out = np.zeros((n, NH, D))
    for t in range(n):
        L = pos + t + 1
        for h in range(NH):
            s = K[:L, h // G] @ q_out[t, h] / np.sqrt(D)
            p = np.exp(s - s.max())
            o = (p[:, None] * V[:L, h // G]).sum(0) / p.sum()
            out[t, h] = o / (1.0 + np.exp(-qg[t, h, D:].astype(np.float64)))
    np.savez_compressed(os.path.join(HERE, f"attn_{name}.npz"), qg=qg, k=k, v=v, wq=wq, wk=wk,
                        kc0=kc0.astype(np.float16), vc0=vc0.astype(np.float16),
                        dims=np.array([NH, NKV, D, R, pos, n]), theta=np.float64(theta), eps=np.float64(eps),
                        seed=np.int64(seed), q_out=q_out, k_new=k_new, out=out)


def make_rope(seed, D=256, R=64, theta=1e7, eps=1e-6):
    """Norm + rope of single rows at positions up to the 256K context limit, where the fp32 angle
    (float)p * inv_freq differs from the exact product by up to ~1e-2 rad."""
    pos = np.array([0, 1, 2, 7, 1000, 4097, 32768, 100003, 262143], np.int32)
    x = normal(seed, (len(pos), D)).astype(np.float32)
    w = (0.1 * normal(seed + 1, (D,))).astype(np.float32)
    y = np.stack([norm_rope(x[i].astype(np.float64), w.astype(np.float64), int(p), R, theta, eps)
                  for i, p in enumerate(pos)])
    np.savez_compressed(os.path.join(HERE, "rope_longpos.npz"), x=x, w=w, pos=pos, y=y,
                        dims=np.array([D, R]), theta=np.float64(theta), eps=np.float64(eps))


if __name__ == "__main__":
    make("c1_tiny", 1001, 4, 1, 64, 16, 128, 1)
    make("gguf_tiny", 2002, 2, 1, 256, 64, 40, 3)      # the reference tiny model's attention shape
    make("qwen3next", 3003, 16, 2, 256, 64, 96, 4)     # Qwen3-Next shape, a 1+3 verify-sized pass
    make_rope(4004)
