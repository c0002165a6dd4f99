"""Write the golden fixtures under tests/golden/ (run in a container with transformers).

The reference ships no tests or vectors, so the fixtures pin the oracle against
an independent library implementation of the same math: HF transformers'
Qwen3-MoE decoder layer (transformers 5.15.0, modeling_qwen3_moe.py), built
from a tiny config in float32 with seeded random weights.  The decode step is
run with a prefilled DynamicCache and an additive mask that limits sequence b
to its first pos[b] cached positions (plus the new token), which is the
reference's position mask (attn_fused_nki.py:646-691).

Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))


def qwen_layer_fixture(seed: int = 2024):
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_moe import modeling_qwen3_moe as M
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig

    H, nq, nkv, d, E, K, I = 256, 4, 2, 64, 8, 2, 64
    B, S = 3, 40
    cfg = Qwen3MoeConfig(hidden_size=H, num_attention_heads=nq, num_key_value_heads=nkv,
                         head_dim=d, num_experts=E, num_experts_per_tok=K,
                         moe_intermediate_size=I, intermediate_size=128, num_hidden_layers=1,
                         rms_norm_eps=1e-6, norm_topk_prob=True, vocab_size=64,
                         rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    cfg._attn_implementation = "eager"
    cfg._experts_implementation = "eager"
    g = torch.Generator().manual_seed(seed)
    layer = M.Qwen3MoeDecoderLayer(cfg, 0).float()
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if "norm" in name:
                v = 1.0 + 0.1 * torch.randn(p.shape, generator=g)
            else:
                v = 0.05 * torch.randn(p.shape, generator=g)
            p.copy_(v.to(torch.bfloat16).float())   # bf16-representable inputs
    pos = torch.tensor([37, 5, 22], dtype=torch.int64)
    P = int(pos.max())
    bfv = lambda t: t.to(torch.bfloat16).float()
    x = bfv(torch.randn(B, H, generator=g))
    kc = bfv(torch.randn(B, nkv, S, d, generator=g))
    vc = bfv(torch.randn(B, nkv, S, d, generator=g))
    cache = DynamicCache(config=cfg)
    cache.update(kc[:, :, :P].clone(), vc[:, :, :P].clone(), 0)
    rot = M.Qwen3MoeRotaryEmbedding(cfg)
    cos, sin = rot(x[:, None, :], pos[:, None])
    mask = torch.full((B, 1, 1, P + 1), torch.finfo(torch.float32).min)
    for b in range(B):
        mask[b, 0, 0, :int(pos[b])] = 0.0
        mask[b, 0, 0, P] = 0.0
    with torch.no_grad():
        y = layer(x[:, None, :], attention_mask=mask, position_ids=pos[:, None],
                  past_key_values=cache, position_embeddings=(cos, sin))
        y = y[0] if isinstance(y, tuple) else y
    k_new = cache.layers[0].keys[:, :, P]          # [B, nkv, d] post-norm, post-RoPE
    v_new = cache.layers[0].values[:, :, P]
    bf = lambda t: t.detach().to(torch.bfloat16).contiguous()   # exact: values are bf16
    sd = {f"w.{n}": bf(p) for n, p in layer.named_parameters()}
    sd.update({"x": bf(x), "pos": pos.to(torch.int32), "k_cache": bf(kc), "v_cache": bf(vc),
               "y": y.reshape(B, H).contiguous(), "k_new": k_new.contiguous(),
               "v_new": v_new.contiguous(), "cos": cos.reshape(B, d).contiguous(),
               "sin": sin.reshape(B, d).contiguous()})
    save_file(sd, os.path.join(HERE, "qwen3moe_layer_fp32.safetensors"),
              metadata={"H": str(H), "nq": str(nq), "nkv": str(nkv), "d": str(d), "E": str(E),
                        "K": str(K), "I": str(I), "eps": "1e-6", "theta": "1e6",
                        "source": "transformers 5.15.0 Qwen3MoeDecoderLayer fp32 eager"})


if __name__ == "__main__":
    qwen_layer_fixture()
    print("wrote", os.listdir(HERE))
