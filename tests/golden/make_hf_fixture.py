"""Writes tests/golden/hf_qwen3next_attn.npz from the installed Hugging Face transformers
Qwen3NextAttention (a third-party implementation of the same attention, not the reference), as an
independent pin of the conventions the reference shares with it: the [query | gate] split per head,
(1 + w) QK-RMSNorm, partial rotate-half RoPE on the first R dims, GQA head grouping, causal softmax
with 1/sqrt(D) and the sigmoid output gate.

The projections are selection matrices, so the module sees exactly the fixture's qg/k/v; o_proj
selects the gated attention output. Runs in float64 (transformers' RMSNorm and rotary tables compute
in float32 internally). Run: python tests/golden/make_hf_fixture.py
"""
import os

import numpy as np
import torch
from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextAttention, Qwen3NextRotaryEmbedding

HERE = os.path.dirname(os.path.abspath(__file__))


def main(NH=4, NKV=2, D=64, R=16, T=24, theta=1e7, eps=1e-6, seed=77):
    r = np.random.default_rng(seed)
    qg = r.standard_normal((T, NH, 2 * D))
    k = r.standard_normal((T, NKV, D))
    v = r.standard_normal((T, NKV, D))
    wq = 0.1 * r.standard_normal(D)
    wk = 0.1 * r.standard_normal(D)
    H = NH * 2 * D + 2 * NKV * D
    cfg = Qwen3NextConfig(hidden_size=H, num_attention_heads=NH, num_key_value_heads=NKV, head_dim=D,
                          rms_norm_eps=eps, attention_bias=False,
                          rope_parameters={"rope_type": "default", "rope_theta": theta,
                                           "partial_rotary_factor": R / D})
    cfg._attn_implementation = "eager"
    att = Qwen3NextAttention(cfg, layer_idx=3).double().eval()
    with torch.no_grad():
        nq, nk = NH * 2 * D, NKV * D
        eye = torch.eye(H, dtype=torch.float64)
        att.q_proj.weight.copy_(eye[:nq])
        att.k_proj.weight.copy_(eye[nq:nq + nk])
        att.v_proj.weight.copy_(eye[nq + nk:])
        att.o_proj.weight.zero_()
        att.o_proj.weight[:NH * D].copy_(torch.eye(NH * D, dtype=torch.float64))
        att.q_norm.weight.copy_(torch.from_numpy(wq))
        att.k_norm.weight.copy_(torch.from_numpy(wk))
        x = torch.from_numpy(np.concatenate([qg.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], 1))[None]
        rot = Qwen3NextRotaryEmbedding(cfg)
        pos_ids = torch.arange(T)[None]
        cos, sin = rot(x, pos_ids)
        mask = torch.full((T, T), float("-inf"), dtype=torch.float64).triu(1)[None, None]
        out, _ = att(x, (cos, sin), mask)
    out = out[0, :, :NH * D].reshape(T, NH, D).numpy()
    np.savez_compressed(os.path.join(HERE, "hf_qwen3next_attn.npz"), qg=qg, k=k, v=v, wq=wq, wk=wk, out=out,
                        dims=np.array([NH, NKV, D, R, T]), theta=np.float64(theta), eps=np.float64(eps))


if __name__ == "__main__":
    main()
