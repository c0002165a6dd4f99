"""The module-level drop-in surface, driven the way NxDI drives the reference.

* Qwen3: NxDI's per-layer loop over ``Qwen3MoeDecoderLayerMK.forward``
  (qwen_with_megakernel.py:422-526).  Token generation: layer 0 runs the whole
  stack and returns (Y, (K0, V0), cos, sin, None), layers 1.. pass through and
  hand back their own cache handles, which alias ``kv_mgr.past_key_values``.
  Context encoding: every layer runs itself over the prompt (the stock CTE layer
  path), padded slots of a [B, S] attention mask pass through.
* GPT-OSS: ``get_model_output`` with the reference's parameter list
  (gpt_oss_with_megakernel.py:577-598), keyword and positional, TKG and CTE.

Hidden states against the CPU oracle within 2e-2, routed like the GPU's routing
log (the routing itself checked against the oracle router on the GPU residual).
"""
import pytest
import torch

from conftest import max_abs_rel
from oracle import ref
from prompt_oracle import qwen_prompt_chain, qwen_ref_layers
from routing_checks import check_oracle_flips, check_qwen_routing

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _small_qwen(dev, B, layers=2, max_seq=128, seed=5):
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    cfg = Q.Qwen3MoeMKConfig(hidden_size=512, num_attention_heads=8, num_key_value_heads=2,
                             head_dim=128, num_experts=16, num_experts_per_tok=4,
                             moe_intermediate_size=128, num_hidden_layers=layers, vocab_size=1000,
                             max_batch=B, max_seq=max_seq)
    hfs = [Q.random_layer_hf(cfg, l, seed, "cpu") for l in range(layers)]
    model = Q.Qwen3MoeMegakernelModel(cfg, [Q.pack_layer({k: v.to(dev) for k, v in h.items()}) for h in hfs],
                                      B, dev)
    shape = ref.QwenShape(H=512, q_heads=8, kv_heads=2, d=128, E=16, K=4, I=128)
    return cfg, hfs, model, shape


def test_qwen_decoder_layer_loop_token_generation(mk, dev):
    cfg, hfs, model, shape = _small_qwen(dev, 3)
    B, Ln = 3, cfg.num_hidden_layers
    model.enable_route_log(B)
    g = torch.Generator().manual_seed(9)
    kc = [torch.randn(B, 2, 128, 128, generator=g).to(torch.bfloat16) for _ in range(Ln)]
    vc = [torch.randn(B, 2, 128, 128, generator=g).to(torch.bfloat16) for _ in range(Ln)]
    for l in range(Ln):
        model.kv_mgr.k(l).copy_(kc[l].to(dev))
        model.kv_mgr.v(l).copy_(vc[l].to(dev))
    x = torch.randn(B, 1, cfg.hidden_size, generator=g).to(torch.bfloat16)
    pos = torch.tensor([[10], [64], [127]], dtype=torch.int64)
    hidden = x.to(dev)
    for l, layer in enumerate(model.layers):
        out = layer(hidden, attention_mask=None, position_ids=pos.to(dev), past_key_value=None,
                    kv_mgr=model.kv_mgr, idx=l, is_for_context_encoding=False)
        assert isinstance(out, tuple) and len(out) == 5 and out[4] is None
        k_l, v_l = out[1]
        assert k_l is model.kv_mgr.past_key_values[2 * l] and v_l is model.kv_mgr.past_key_values[2 * l + 1]
        if l == 0:
            assert out[2].shape == (B, 1, 128) and out[3].shape == (B, 1, 128)
        else:
            assert out[0] is hidden and out[2] is None
        hidden = out[0]
    torch.cuda.synchronize()
    logs = model.route_log(B)
    lws = qwen_ref_layers(hfs)
    cos, sin = ref.rope_cos_sin(pos.reshape(-1), 128, cfg.rope_theta)
    y = x.reshape(B, -1).float()
    for l in range(Ln):
        check_qwen_routing(logs[l], lws[l], 1e-6, 4)
        kr = kc[l].clone()
        y, _ = ref.qwen_decoder_layer(y, lws[l], kr, vc[l].clone(), cos, sin, pos.reshape(-1), shape,
                                      force_idx=logs[l]["idx"].long())
        kn = model.kv_mgr.k(l).cpu()
        for b in range(B):
            p = int(pos[b])
            assert (kn[b] != kc[l][b]).any(-1).any(0).nonzero().flatten().tolist() == [p]
            assert max_abs_rel(kn[b, :, p], kr[b, :, p]) < TOL
    assert max_abs_rel(hidden.reshape(B, -1), y) < TOL


def test_qwen_decoder_layer_loop_context_encoding(mk, dev):
    """Per-layer CTE over two prompts in one [B, S] batch (the second left-padded by
    3 slots), then one decode step through the TKG loop reads the encoded rows."""
    cfg, hfs, model, shape = _small_qwen(dev, 2)
    B, S, pad, Ln = 2, 24, 3, cfg.num_hidden_layers
    g = torch.Generator().manual_seed(13)
    x = torch.randn(B, S, cfg.hidden_size, generator=g).to(torch.bfloat16)
    mask = torch.ones(B, S, dtype=torch.int64)
    mask[1, :pad] = 0
    pos = torch.arange(S).repeat(B, 1)
    pos[1] = torch.clamp(torch.arange(S) - pad, min=0)
    hidden = x.to(dev)
    for l, layer in enumerate(model.layers):
        out = layer(hidden, attention_mask=mask.to(dev), position_ids=pos.to(dev), kv_mgr=model.kv_mgr,
                    is_for_context_encoding=True)
        assert len(out) == 5 and out[1][0] is model.kv_mgr.past_key_values[2 * l]
        hidden = out[0]
    torch.cuda.synchronize()
    hid = hidden.cpu()
    assert torch.equal(hid[1, :pad], x[1, :pad])                     # padded slots pass through
    lws = qwen_ref_layers(hfs)
    for b in range(B):
        c0 = pad if b == 1 else 0
        T = S - c0
        kcs = [torch.zeros(1, 2, 128, 128) for _ in range(Ln)]
        vcs = [torch.zeros(1, 2, 128, 128) for _ in range(Ln)]
        y_own, _ = qwen_prompt_chain(x[b, c0:], lws, kcs, vcs, 0, shape)
        e = max_abs_rel(hid[b, c0:], y_own)
        print(f"sequence {b}: CTE through the layer loop vs the oracle chain {e:.2e}", flush=True)
        assert e < TOL
        for l in range(Ln):
            assert max_abs_rel(model.kv_mgr.k(l).cpu()[b, :, :T], kcs[l][0, :, :T]) < TOL
            assert max_abs_rel(model.kv_mgr.v(l).cpu()[b, :, :T], vcs[l][0, :, :T]) < TOL
            assert not model.kv_mgr.k(l).cpu()[b, :, T:].any()


def _small_gpt_oss(dev, B, seed=3):
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    cfg = G.GptOssMKConfig(num_hidden_layers=2, max_batch=B, max_seq=256, vocab_size=1024,
                           num_experts=8, intermediate_size=1024, expert_format="bf16")
    hfs = [G.random_layer_hf(cfg, l, seed, "cpu") for l in range(2)]
    g = torch.Generator().manual_seed(seed)
    embed = (torch.randn(1024, cfg.hidden_size, generator=g) * 0.5).to(torch.bfloat16)
    ln_f = (1 + 0.02 * torch.randn(cfg.hidden_size, generator=g)).to(torch.bfloat16)
    lm = (0.02 * torch.randn(1024, cfg.hidden_size, generator=g)).to(torch.bfloat16)
    model = G.GptOssMegakernelModel(cfg, [G.pack_layer({k: v.to(dev) for k, v in h.items()}, cfg) for h in hfs],
                                    B, dev, embed=embed.to(dev), ln_f=ln_f.to(dev), lm_head=lm.to(dev))
    return cfg, hfs, model, embed, ln_f


def _gpt_oss_ref_layer(hf):
    return ref.GptOssLayer(
        wq=hf["q_proj.weight"], bq=hf["q_proj.bias"], wk=hf["k_proj.weight"], bk=hf["k_proj.bias"],
        wv=hf["v_proj.weight"], bv=hf["v_proj.bias"], wo=hf["o_proj.weight"], bo=hf["o_proj.bias"],
        sinks=hf["sinks"], ln_in=hf["input_layernorm"], ln_post=hf["post_attention_layernorm"],
        router_w=hf["router.weight"], router_b=hf["router.bias"], gate_up=hf["experts.gate_up_proj"],
        gate_up_b=hf["experts.gate_up_proj_bias"], down=hf["experts.down_proj"],
        down_b=hf["experts.down_proj_bias"])


def test_gpt_oss_get_model_output_reference_signature(mk, dev):
    """CTE of a 5-token prompt for two sequences, then a TKG step, through
    get_model_output called with the reference's keywords (and once
    positionally: input_ids, seq_ids, attention_mask, position_ids); the
    returned norm(Y) and caches against the oracle decoding token by token."""
    cfg, hfs, model, embed, ln_f = _small_gpt_oss(dev, 2)
    B, S = 2, 5
    model.enable_route_log(B)
    model.route_log_history = []     # every CTE pass's routing: pass b * S + t is token t of sequence b
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(0, 1024, (B, S + 1), generator=g)
    pos = torch.arange(S).repeat(B, 1)
    y_cte, cache = model.get_model_output(input_ids=ids[:, :S].to(dev), seq_ids=torch.arange(B).to(dev),
                                          attention_mask=torch.ones(B, S, device=dev),
                                          position_ids=pos.to(dev), past_key_values=None,
                                          is_for_context_encoding=True)
    assert y_cte.shape == (B, S, cfg.hidden_size) and len(cache) == 4
    assert all(a is b for a, b in zip(cache, model.kv_mgr.past_key_values))
    y_tkg, _ = model.get_model_output(ids[:, S:].to(dev), torch.arange(B).to(dev), None,
                                      torch.full((B, 1), S).to(dev))
    torch.cuda.synchronize()
    logs = model.route_log(B)
    hist = model.route_log_history
    model.route_log_history = None
    assert len(hist) == B * S
    # oracle: token by token through both layers (sliding window 128, full), routed like
    # the GPU -- the CTE tokens like their own passes, the last (TKG) token like the
    # TKG call -- with every flip of the oracle's own top-k a near-tie
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    lws = [_gpt_oss_ref_layer(h) for h in hfs]
    inv, scl = G.yarn_inv_freq(cfg)
    shape = ref.GptOssShape(E=8, I=1024)
    caches = [(torch.zeros(B, 8, 128 if cfg.is_sliding(l) else 256, 64),
               torch.zeros(B, 8, 128 if cfg.is_sliding(l) else 256, 64)) for l in range(2)]
    outs = []
    for t in range(S + 1):
        p = torch.full((B,), t)
        fr = p.reshape(-1, 1).float() * inv[None, :]
        cos, sin = fr.cos() * scl, fr.sin() * scl
        x = embed[ids[:, t]].float()
        for l in range(2):
            if t == S:
                rec_idx, rec_lg = logs[l]["idx"], logs[l]["logits"]
            else:
                rec_idx = torch.cat([hist[b * S + t][l]["idx"] for b in range(B)])
                rec_lg = torch.cat([hist[b * S + t][l]["logits"] for b in range(B)])
            x, aux = ref.gpt_oss_decoder_layer(x, lws[l], caches[l][0], caches[l][1], cos, sin, p,
                                               128 if cfg.is_sliding(l) else 0, shape,
                                               force_idx=rec_idx.long())
            check_oracle_flips(rec_idx, rec_lg, aux["logits"], 4)
        outs.append(ref._bf(ref.rmsnorm_tkg(x, ln_f, cfg.rms_norm_eps)))
    e_cte = max(max_abs_rel(y_cte[:, t], outs[t]) for t in range(S))
    e_tkg = max_abs_rel(y_tkg[:, 0], outs[S])
    print(f"get_model_output: CTE vs oracle {e_cte:.2e}, TKG vs oracle {e_tkg:.2e}", flush=True)
    assert e_cte < TOL and e_tkg < TOL
    for l in range(2):
        assert max_abs_rel(model.kv_mgr.k(l).cpu()[:, :, :S + 1], caches[l][0][:, :, :S + 1]) < TOL
    with pytest.raises(NotImplementedError):
        model.get_model_output(ids[:, S:].to(dev), torch.tensor([1, 0]).to(dev), None,
                               torch.full((B, 1), S).to(dev))
