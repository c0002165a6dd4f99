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
