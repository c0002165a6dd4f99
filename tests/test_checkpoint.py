"""CPU checks of the HF safetensors checkpoint reader (no GPU): lazy sharded
reads, config.json mapping, and the MXFP4 expert decoding, which is pinned
against the OCP E2M1 bit formula of the oracle's MX codec for every byte value
and shown to survive the OCP re-quantisation exactly."""
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import mx as omx


def _C():
    from nki_moe_megakernel_amd import checkpoint as C
    return C


def test_mxfp4_decode_every_byte_matches_e2m1_formula(mk):
    """All 256 byte values under scales 2^-3, 2^0 and 2^5: low nibble is element
    2i, high nibble 2i + 1, value = E2M1(code) * 2^(scale - 127)."""
    C = _C()
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(16, 16)      # 16 blocks of 16 bytes
    for sbyte in (124, 127, 132):
        s = torch.full((16,), sbyte, dtype=torch.uint8)
        got = C.mxfp4_dequantize(b, s).float().numpy().reshape(16, 32)            # K = 512
        lo = omx.decode_elements(b.numpy() & 0x0F, "e2m1")
        hi = omx.decode_elements(b.numpy() >> 4, "e2m1")
        want = np.stack([lo, hi], -1).reshape(16, 32) * 2.0 ** (sbyte - 127)
        np.testing.assert_array_equal(got, want.astype(np.float32))
        # -0.0 keeps its sign (code 8)
        assert np.signbit(got[0, 16]) and got[0, 16] == 0.0    # byte 0x08: low code 8 = -0.0


def test_mxfp4_known_block():
    """Hand-decoded block: bytes 0x21 0xF7 under scale byte 128 (x2)."""
    from nki_moe_megakernel_amd import checkpoint as C
    blk = torch.zeros(1, 1, 16, dtype=torch.uint8)
    blk[0, 0, 0], blk[0, 0, 1] = 0x21, 0xF7
    v = C.mxfp4_dequantize(blk, torch.tensor([[128]], dtype=torch.uint8))
    assert v.shape == (1, 32)
    assert v[0, :4].tolist() == [1.0, 2.0, 12.0, -12.0]
    assert bool((v[0, 4:] == 0).all())


def test_mxfp4_rejects_bad_scales_and_shapes(mk):
    C = _C()
    blk = torch.zeros(2, 3, 16, dtype=torch.uint8)
    with pytest.raises(ValueError):
        C.mxfp4_dequantize(blk, torch.full((2, 3), 255, dtype=torch.uint8))
    with pytest.raises(ValueError):
        C.mxfp4_dequantize(blk, torch.zeros(2, 4, dtype=torch.uint8))


def test_mxfp4_requantisation_is_exact(mk):
    """Random MXFP4 blocks (every code, scales 100..150): decode -> OCP MX
    quantise (the oracle's rule, bit-identical to the library's quantiser) ->
    decode gives the same values, so MX models keep the checkpoint's weights."""
    C = _C()
    g = torch.Generator().manual_seed(3)
    blk = torch.randint(0, 256, (64, 8, 16), generator=g, dtype=torch.int32).to(torch.uint8)
    blk[0, 0] = 0x11                                            # block of 0.5s only
    blk[1, 1] = 0                                               # all-zero block
    sc = torch.randint(100, 151, (64, 8), generator=g, dtype=torch.int32).to(torch.uint8)
    v = C.mxfp4_dequantize(blk, sc).float().numpy()            # [64, 256]
    codes, scales = omx.quantize_mx(v, "e2m1")
    back = omx.dequantize_mx(codes, scales, "e2m1")
    np.testing.assert_array_equal(back, v)


def _write_sharded(tmp_path, tensors, n_shards, config=None):
    names = sorted(tensors)
    wm = {}
    for i in range(n_shards):
        part = {k: tensors[k].contiguous() for k in names[i::n_shards]}
        fn = f"model-{i + 1:05d}-of-{n_shards:05d}.safetensors"
        save_file(part, str(tmp_path / fn))
        wm.update({k: fn for k in part})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    if config is not None:
        (tmp_path / "config.json").write_text(json.dumps(config))


def test_sharded_checkpoint_reads_lazily(mk, tmp_path):
    C = _C()
    g = torch.Generator().manual_seed(0)
    t = {f"model.layers.{l}.w{i}": torch.randn(3, 5, generator=g).to(torch.bfloat16)
         for l in range(2) for i in range(3)}
    t["blocks"] = torch.randint(0, 255, (2, 4, 16), generator=g, dtype=torch.int32).to(torch.uint8)
    _write_sharded(tmp_path, t, 3, {"model_type": "x"})
    ck = C.SafetensorsCheckpoint(str(tmp_path))
    assert len(ck) == len(t) and set(ck.keys()) == set(t)
    assert ck.config == {"model_type": "x"}
    for k, v in t.items():
        assert k in ck and torch.equal(ck[k], v)
    assert "missing" not in ck and ck.get("missing") is None
    with pytest.raises(KeyError):
        ck["missing"]
    # single file, no index
    save_file({"a": torch.ones(2)}, str(tmp_path / "one.safetensors"))
    one = C.SafetensorsCheckpoint(str(tmp_path / "one.safetensors"))
    assert list(one.keys()) == ["a"] and torch.equal(one["a"], torch.ones(2))


def test_qwen3_moe_config_maps_hf_fields(mk):
    from transformers import Qwen3MoeConfig
    C = _C()
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    hf = Qwen3MoeConfig(hidden_size=2048, num_attention_heads=32, num_key_value_heads=4, head_dim=128,
                        num_experts=128, num_experts_per_tok=8, moe_intermediate_size=768,
                        num_hidden_layers=48, vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1e6,
                        norm_topk_prob=True).to_dict()
    cfg = C.qwen3_moe_config(hf, max_batch=4, max_seq=4096)
    want = Q.Qwen3MoeMKConfig(max_batch=4, max_seq=4096)     # defaults: the 30B-A3B shape
    assert cfg == want
    with pytest.raises(ValueError):
        C.qwen3_moe_config(dict(hf, norm_topk_prob=False))
    with pytest.raises(ValueError):
        C.qwen3_moe_config(dict(hf, mlp_only_layers=[3]))


def test_gpt_oss_config_maps_hf_fields(mk):
    from transformers import GptOssConfig
    C = _C()
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    hf = GptOssConfig(num_hidden_layers=24, num_local_experts=32, num_experts_per_tok=4,
                      hidden_size=2880, intermediate_size=2880, head_dim=64, num_attention_heads=64,
                      num_key_value_heads=8, vocab_size=201088, sliding_window=128,
                      rope_theta=150000.0).to_dict()
    cfg = C.gpt_oss_config(hf)
    assert cfg == G.GptOssMKConfig()                          # defaults: the 20B shape
    assert C.gpt_oss_config(dict(hf, hidden_size=2880 + 600)).hidden_pad == 3584
    types = ["full_attention", "sliding_attention"] * 12
    assert C.gpt_oss_config(dict(hf, layer_types=types)).first_sliding is False
    with pytest.raises(ValueError):
        C.gpt_oss_config(dict(hf, layer_types=["sliding_attention"] * 24))


def test_gpt_oss_layer_from_mxfp4_checkpoint(mk, tmp_path):
    """MXFP4 expert tensors -> the converter's [E, H, 2I] / [E, I, H] bf16 layouts."""
    C = _C()
    E, H, I, nq, nkv, d = 2, 64, 32, 2, 1, 16
    g = torch.Generator().manual_seed(1)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    u8 = lambda *s, lo=0, hi=256: torch.randint(lo, hi, s, generator=g, dtype=torch.int32).to(torch.uint8)
    p = "model.layers.0."
    t = {p + f"self_attn.{n}_proj.weight": r(o, i) for n, o, i in
         (("q", nq * d, H), ("k", nkv * d, H), ("v", nkv * d, H), ("o", H, nq * d))}
    t.update({p + f"self_attn.{n}_proj.bias": r(o) for n, o in (("q", nq * d), ("k", nkv * d),
                                                                 ("v", nkv * d), ("o", H))})
    t.update({p + "self_attn.sinks": torch.randn(nq, generator=g), p + "input_layernorm.weight": r(H),
              p + "post_attention_layernorm.weight": r(H), p + "mlp.router.weight": r(E, H),
              p + "mlp.router.bias": r(E), p + "mlp.experts.gate_up_proj_bias": r(E, 2 * I),
              p + "mlp.experts.down_proj_bias": r(E, H),
              p + "mlp.experts.gate_up_proj_blocks": u8(E, 2 * I, H // 32, 16),
              p + "mlp.experts.gate_up_proj_scales": u8(E, 2 * I, H // 32, lo=120, hi=130),
              p + "mlp.experts.down_proj_blocks": u8(E, H, I // 32, 16),
              p + "mlp.experts.down_proj_scales": u8(E, H, I // 32, lo=120, hi=130)})
    _write_sharded(tmp_path, t, 2)
    ck = C.SafetensorsCheckpoint(str(tmp_path))
    hf = C.gpt_oss_layer_hf(ck, 0, "cpu")
    gu = C.mxfp4_dequantize(t[p + "mlp.experts.gate_up_proj_blocks"], t[p + "mlp.experts.gate_up_proj_scales"])
    dn = C.mxfp4_dequantize(t[p + "mlp.experts.down_proj_blocks"], t[p + "mlp.experts.down_proj_scales"])
    assert hf["experts.gate_up_proj"].shape == (E, H, 2 * I)
    assert torch.equal(hf["experts.gate_up_proj"], gu.transpose(1, 2))
    assert hf["experts.down_proj"].shape == (E, I, H)
    assert torch.equal(hf["experts.down_proj"], dn.transpose(1, 2))
    assert torch.equal(hf["q_proj.bias"], t[p + "self_attn.q_proj.bias"])
    assert hf["sinks"].dtype == torch.float32
    del t[p + "mlp.router.bias"]
    _write_sharded(tmp_path, t, 2)
    with pytest.raises(KeyError):
        C.gpt_oss_layer_hf(C.SafetensorsCheckpoint(str(tmp_path)), 0, "cpu")
