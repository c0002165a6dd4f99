"""CPU checks of host-side logic of the package (no GPU): RoPE tables and
weight-layout conversions that run before any kernel."""
import pytest
import torch


def test_gpt_oss_yarn_matches_hf(mk):
    """YaRN frequencies and attention scaling == transformers' "yarn" rope init for
    the GPT-OSS config (truncate=False)."""
    from transformers import GptOssConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    inv, sc = G.yarn_inv_freq(G.GptOssMKConfig())
    inv_hf, sc_hf = ROPE_INIT_FUNCTIONS["yarn"](GptOssConfig(head_dim=64), "cpu")
    torch.testing.assert_close(inv, inv_hf.float(), rtol=1e-6, atol=0)
    assert sc == pytest.approx(sc_hf, rel=1e-12)


def test_gpt_oss_converter_deinterleaves_and_folds_up_bias(mk):
    """HF gate_up [E, H, 2I] interleaved -> gate rows then up rows; up bias + 1;
    H zero-padded (gpt_oss_with_megakernel.py:554-560)."""
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    cfg = G.GptOssMKConfig(hidden_size=96, hidden_pad=512, num_attention_heads=4, num_key_value_heads=2,
                           head_dim=16, num_experts=3, intermediate_size=8)
    hf = G.random_layer_hf(cfg, 0, 1, "cpu")
    c = G.convert_layer(hf, cfg)
    gu = hf["experts.gate_up_proj"]
    I = 8
    assert torch.equal(c["gate_up"][:, :I, :96], gu[:, :, 0::2].transpose(1, 2))
    assert torch.equal(c["gate_up"][:, I:, :96], gu[:, :, 1::2].transpose(1, 2))
    assert not c["gate_up"][:, :, 96:].any()
    b = hf["experts.gate_up_proj_bias"].float()
    assert torch.equal(c["gate_up_bias"][:, 0].float(), b[:, 0::2].bfloat16().float())
    assert torch.equal(c["gate_up_bias"][:, 1].float(), (b[:, 1::2] + 1).bfloat16().float())
    assert torch.equal(c["down"][:, :96], hf["experts.down_proj"].transpose(1, 2))
    assert not c["w_qkv"][:, 96:].any() and not c["ln_in"][96:].any()


def test_prefill_rejects_bad_requests_before_any_gpu_call(mk):
    """model.prefill's host checks: the sequence slot must exist and the prompt must
    fit the caches; a model without embedding / lm_head cannot prefill."""
    from types import SimpleNamespace
    from nki_moe_megakernel_amd.qwen_with_megakernel import _prefill
    cfg = SimpleNamespace(max_seq=16, vocab_size=32)
    m = SimpleNamespace(embed_tokens=torch.zeros(1), lm_head_packed=torch.zeros(1), batch=2, cfg=cfg,
                        device=torch.device("cpu"))
    ids = torch.arange(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="sequence 2"):
        _prefill(m, ids, 0, 2, 128, 8, 8, 2, lambda p: (None, None))
    with pytest.raises(ValueError, match="does not fit"):
        _prefill(m, ids, 13, 0, 128, 8, 8, 2, lambda p: (None, None))
    with pytest.raises(ValueError, match="does not fit"):
        _prefill(m, ids[:0], 0, 0, 128, 8, 8, 2, lambda p: (None, None))
    with pytest.raises(ValueError, match="embedding"):
        _prefill(SimpleNamespace(**{**m.__dict__, "lm_head_packed": None}), ids, 0, 0, 128, 8, 8, 2,
                 lambda p: (None, None))
