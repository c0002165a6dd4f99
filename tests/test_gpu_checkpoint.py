"""HF safetensors checkpoints through checkpoint.load_qwen3_moe / load_gpt_oss give
bit-identical greedy decode steps (logits, next ids, KV caches) to models built
directly from the same weights: Qwen3-MoE per-expert HF keys fused into the
[E, 2I, H] experts, untied lm_head, two shards; GPT-OSS MXFP4 expert blocks
decoded by the loader vs bf16 experts decoded independently by the oracle's
E2M1 formula (so the nibble order, scale and transposes are all checked)."""
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import mx as omx

pytestmark = pytest.mark.gpu


def _save(path, tensors, n_shards, config):
    names = sorted(tensors)
    wm = {}
    for i in range(n_shards):
        part = {k: tensors[k].contiguous() for k in names[i::n_shards]}
        fn = f"model-{i + 1:05d}-of-{n_shards:05d}.safetensors"
        save_file(part, str(path / fn))
        wm.update({k: fn for k in part})
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    (path / "config.json").write_text(json.dumps(config))


def _two_steps(m, ids, pos):
    l1, n1 = m(ids, pos)
    l2, n2 = m(n1, pos + 1)
    torch.cuda.synchronize()
    return l1.cpu(), n1.cpu(), l2.cpu(), n2.cpu()


def test_qwen3_checkpoint_decode_matches_direct(mk, dev, tmp_path):
    from nki_moe_megakernel_amd import checkpoint as C
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    print("qwen3 checkpoint: E=16 I=256 2 layers B=2", flush=True)
    hf_cfg = dict(model_type="qwen3_moe", hidden_size=2048, num_attention_heads=32, num_key_value_heads=4,
                  head_dim=128, num_experts=16, num_experts_per_tok=8, moe_intermediate_size=256,
                  num_hidden_layers=2, vocab_size=1024, rms_norm_eps=1e-6, rope_theta=1e6,
                  norm_topk_prob=True, tie_word_embeddings=False)
    cfg = C.qwen3_moe_config(hf_cfg, max_batch=2, max_seq=256)
    I = cfg.moe_intermediate_size
    t, layers_hf = {}, []
    for l in range(2):
        hf = Q.random_layer_hf(cfg, l, 11, "cpu")
        layers_hf.append(hf)
        p = f"model.layers.{l}."
        for n in "qkvo":
            t[p + f"self_attn.{n}_proj.weight"] = hf[f"{n}_proj"]
        t[p + "self_attn.q_norm.weight"] = hf["q_norm"]
        t[p + "self_attn.k_norm.weight"] = hf["k_norm"]
        t[p + "input_layernorm.weight"] = hf["input_layernorm"]
        t[p + "post_attention_layernorm.weight"] = hf["post_attention_layernorm"]
        t[p + "mlp.gate.weight"] = hf["gate"]
        for e in range(cfg.num_experts):
            t[p + f"mlp.experts.{e}.gate_proj.weight"] = hf["gate_up_proj"][e, :I]
            t[p + f"mlp.experts.{e}.up_proj.weight"] = hf["gate_up_proj"][e, I:]
            t[p + f"mlp.experts.{e}.down_proj.weight"] = hf["down_proj"][e]
    g = torch.Generator().manual_seed(5)
    embed = (torch.randn(1024, 2048, generator=g) * 0.5).to(torch.bfloat16)
    ln_f = (1 + 0.02 * torch.randn(2048, generator=g)).to(torch.bfloat16)
    lm = (0.02 * torch.randn(1024, 2048, generator=g)).to(torch.bfloat16)
    t.update({"model.embed_tokens.weight": embed, "model.norm.weight": ln_f, "lm_head.weight": lm})
    _save(tmp_path, t, 2, hf_cfg)

    m1 = C.load_qwen3_moe(str(tmp_path), batch=2, device=dev, max_seq=256)
    assert m1.cfg == cfg
    m2 = Q.Qwen3MoeMegakernelModel(
        cfg, [Q.pack_layer({k: v.to(dev) for k, v in h.items()}) for h in layers_hf], 2, dev,
        embed=embed.to(dev), ln_f=ln_f.to(dev), lm_head=lm.to(dev))
    ids = torch.tensor([3, 1000], dtype=torch.int32, device=dev)
    pos = torch.tensor([100, 7], dtype=torch.int32, device=dev)
    a, b = _two_steps(m1, ids, pos), _two_steps(m2, ids, pos)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert torch.isfinite(a[0]).all() and a[0].abs().max() > 0
    for l in range(2):
        assert torch.equal(m1.kv_mgr.k(l).cpu(), m2.kv_mgr.k(l).cpu())
        assert torch.equal(m1.kv_mgr.v(l).cpu(), m2.kv_mgr.v(l).cpu())


def _e2m1_pack(codes):
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


def test_gpt_oss_mxfp4_checkpoint_decode_matches_direct(mk, dev, tmp_path):
    from nki_moe_megakernel_amd import checkpoint as C
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    print("gpt-oss mxfp4 checkpoint: E=8 I=1024 2 layers B=1", flush=True)
    hf_cfg = dict(model_type="gpt_oss", hidden_size=2880, num_attention_heads=64, num_key_value_heads=8,
                  head_dim=64, num_local_experts=8, num_experts_per_tok=4, intermediate_size=1024,
                  num_hidden_layers=2, vocab_size=1024, rms_norm_eps=1e-5, sliding_window=128,
                  swiglu_limit=7.0, rope_theta=150000.0,
                  rope_scaling=dict(rope_type="yarn", factor=32.0, beta_fast=32.0, beta_slow=1.0,
                                    original_max_position_embeddings=4096, truncate=False),
                  layer_types=["sliding_attention", "full_attention"], tie_word_embeddings=False)
    cfg = C.gpt_oss_config(hf_cfg, max_batch=1, max_seq=512)
    H, I, E = cfg.hidden_size, cfg.intermediate_size, cfg.num_experts
    rng = np.random.default_rng(9)
    t, layers_hf = {}, []
    for l in range(2):
        hf = G.random_layer_hf(cfg, l, 13, "cpu")
        p = f"model.layers.{l}."
        for n in "qkvo":
            for k in ("weight", "bias"):
                t[p + f"self_attn.{n}_proj.{k}"] = hf[f"{n}_proj.{k}"]
        t[p + "self_attn.sinks"] = hf["sinks"]
        t[p + "input_layernorm.weight"] = hf["input_layernorm"]
        t[p + "post_attention_layernorm.weight"] = hf["post_attention_layernorm"]
        t[p + "mlp.router.weight"] = hf["router.weight"]
        t[p + "mlp.router.bias"] = hf["router.bias"]
        t[p + "mlp.experts.gate_up_proj_bias"] = hf["experts.gate_up_proj_bias"]
        t[p + "mlp.experts.down_proj_bias"] = hf["experts.down_proj_bias"]
        for proj, (N, K) in (("gate_up_proj", (2 * I, H)), ("down_proj", (H, I))):
            codes = rng.integers(0, 16, (E, N, K), dtype=np.int64)
            scales = rng.integers(118, 124, (E, N, K // 32), dtype=np.int64).astype(np.uint8)
            vals = omx.dequantize_mx(codes, scales, "e2m1")                 # [E, N, K] oracle decode
            t[p + f"mlp.experts.{proj}_blocks"] = torch.from_numpy(
                _e2m1_pack(codes).reshape(E, N, K // 32, 16))
            t[p + f"mlp.experts.{proj}_scales"] = torch.from_numpy(scales)
            hf[f"experts.{proj}"] = torch.from_numpy(vals).transpose(1, 2).to(torch.bfloat16).contiguous()
        layers_hf.append(hf)
    g = torch.Generator().manual_seed(6)
    embed = (torch.randn(1024, H, generator=g) * 0.5).to(torch.bfloat16)
    ln_f = (1 + 0.02 * torch.randn(H, generator=g)).to(torch.bfloat16)
    lm = (0.02 * torch.randn(1024, H, generator=g)).to(torch.bfloat16)
    t.update({"model.embed_tokens.weight": embed, "model.norm.weight": ln_f, "lm_head.weight": lm})
    _save(tmp_path, t, 2, hf_cfg)

    m1 = C.load_gpt_oss(str(tmp_path), batch=1, device=dev, max_seq=512)
    assert m1.cfg == cfg
    m2 = G.GptOssMegakernelModel(
        cfg, [G.pack_layer({k: v.to(dev) for k, v in h.items()}, cfg) for h in layers_hf], 1, dev,
        embed=embed.to(dev), ln_f=ln_f.to(dev), lm_head=lm.to(dev))
    ids = torch.tensor([77], dtype=torch.int32, device=dev)
    pos = torch.tensor([300], dtype=torch.int32, device=dev)

    def steps(m):
        outs = []
        for k in range(2):
            hidden = torch.empty(1, cfg.hidden_pad, dtype=torch.bfloat16, device=dev)
            logits = torch.empty(1, cfg.vocab_size, dtype=torch.float32, device=dev)
            nxt = torch.empty(1, dtype=torch.int32, device=dev)
            m.step(ids if k == 0 else outs[-1][1].to(dev), pos + k, hidden, logits, nxt)
            torch.cuda.synchronize()
            outs.append((logits.cpu(), nxt.cpu()))
        return outs

    a, b = steps(m1), steps(m2)
    for (la, na), (lb, nb) in zip(a, b):
        assert torch.equal(la, lb) and torch.equal(na, nb)
    assert torch.isfinite(a[0][0]).all() and a[0][0].abs().max() > 0
