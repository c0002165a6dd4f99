"""HF safetensors checkpoints -> the library's packed decode models.

The reference turns HF state dicts into its kernels' layouts inside NxDI
(convert_qwen3_moe_hf_to_neuron_state_dict, megakernels/qwen3_moe/
qwen_with_megakernel.py:171-271; convert_gpt_oss_hf_to_neuron_state_dict,
megakernels/gpt_oss/gpt_oss_with_megakernel.py:290-327, which pads H to 3072
and defers the rest to NxDI's GPT-OSS converter).  Here a checkpoint directory
(``config.json`` + ``model.safetensors`` or sharded ``model-*.safetensors``
with ``model.safetensors.index.json``) is read lazily, one tensor at a time,
and each layer is converted and packed on the device before the next is read,
so host memory holds at most one layer's tensors.

Supported on-disk forms:
  Qwen3-MoE  per-expert ``mlp.experts.{e}.{gate,up,down}_proj.weight`` (HF) or
             fused ``mlp.experts.gate_up_proj`` [E, 2I, H] / ``down_proj`` [E, H, I];
             ``lm_head.weight`` or tied embeddings.
  GPT-OSS    bf16 experts ``mlp.experts.gate_up_proj`` [E, H, 2I] (gate / up
             columns interleaved) / ``down_proj`` [E, I, H], or the released
             MXFP4 form ``*_proj_blocks`` [E, N, K/32, 16] (two E2M1 codes per
             byte, low nibble first) + ``*_proj_scales`` [E, N, K/32] (E8M0).

MXFP4 experts are decoded to bf16 on the device and re-quantised by the
library's OCP quantiser when the model keeps MX experts.  That round trip is
exact: for a block whose largest code magnitude is c_max (0.5 .. 6) under
scale 2^s, the OCP rule picks 2^(s - (2 - floor(log2 c_max))), and every
E2M1 value times 2^(2 - floor(log2 c_max)) that stays <= 6 is again an E2M1
value.
"""
from __future__ import annotations

import json
import os
from typing import Dict, Iterator, Optional

import torch

from . import gpt_oss_with_megakernel as G
from . import qwen_with_megakernel as Q

# OCP MX v1.0 E2M1 element values by 4-bit code (sign bit 3, exponent bits 2:1
# with bias 1, mantissa bit 0; code 0b0001 is the subnormal 0.5).
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


class SafetensorsCheckpoint:
    """Read-only, lazy name -> tensor mapping over a checkpoint directory (or one
    .safetensors file).  Tensors are read on access; nothing is cached."""

    def __init__(self, path: str):
        from safetensors import safe_open
        self._open = safe_open
        self.path = path
        self.config: dict = {}
        if os.path.isdir(path):
            cfg = os.path.join(path, "config.json")
            if os.path.exists(cfg):
                with open(cfg) as f:
                    self.config = json.load(f)
            index = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(index):
                with open(index) as f:
                    wm = json.load(f)["weight_map"]
                self._where = {k: os.path.join(path, v) for k, v in wm.items()}
            else:
                files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
                if not files:
                    raise FileNotFoundError(f"no .safetensors files in {path}")
                self._where = {}
                for fn in files:
                    full = os.path.join(path, fn)
                    with safe_open(full, framework="pt") as h:
                        for k in h.keys():
                            self._where[k] = full
        else:
            self._where = {}
            with safe_open(path, framework="pt") as h:
                for k in h.keys():
                    self._where[k] = path
        self._handles: Dict[str, object] = {}

    def _handle(self, fn: str):
        h = self._handles.get(fn)
        if h is None:
            h = self._open(fn, framework="pt")
            self._handles[fn] = h
        return h

    def __contains__(self, name: str) -> bool:
        return name in self._where

    def __getitem__(self, name: str) -> torch.Tensor:
        if name not in self._where:
            raise KeyError(name)
        return self._handle(self._where[name]).get_tensor(name)

    def get(self, name: str, default=None):
        return self[name] if name in self._where else default

    def keys(self) -> Iterator[str]:
        return iter(self._where)

    def __len__(self) -> int:
        return len(self._where)


def _rope(hf: dict, default_theta: float):
    """(theta, scaling dict) from either config.json form: top-level rope_theta +
    rope_scaling (released checkpoints) or rope_parameters (newer transformers)."""
    rp = hf.get("rope_parameters") or {}
    theta = float(hf.get("rope_theta", rp.get("rope_theta", default_theta)))
    rs = hf.get("rope_scaling") or {}
    if not rs and rp.get("rope_type", "default") != "default":
        rs = rp
    return theta, rs


def _checked(hf: dict, key: str, want, what: str):
    v = hf.get(key, want)
    if v != want:
        raise ValueError(f"{what}: config {key}={v!r} is not supported (needs {want!r})")


def qwen3_moe_config(hf: dict, **overrides) -> Q.Qwen3MoeMKConfig:
    """HF Qwen3-MoE config.json fields -> Qwen3MoeMKConfig (+ runtime overrides such
    as max_batch, max_seq, expert_format, kv_block_len)."""
    if hf.get("model_type", "qwen3_moe") != "qwen3_moe":
        raise ValueError(f"not a Qwen3-MoE config (model_type={hf.get('model_type')!r})")
    _checked(hf, "norm_topk_prob", True, "Qwen3-MoE")
    _checked(hf, "decoder_sparse_step", 1, "Qwen3-MoE")
    if hf.get("mlp_only_layers"):
        raise ValueError("Qwen3-MoE: dense (mlp_only_layers) layers are not supported")
    H, nq = hf["hidden_size"], hf["num_attention_heads"]
    theta, rs = _rope(hf, 1e6)
    if rs:
        raise ValueError(f"Qwen3-MoE: rope scaling {rs!r} is not supported")
    kw = dict(hidden_size=H, num_attention_heads=nq,
              num_key_value_heads=hf.get("num_key_value_heads", nq),
              head_dim=hf.get("head_dim", H // nq),
              num_experts=hf.get("num_experts", hf.get("num_local_experts")),
              num_experts_per_tok=hf["num_experts_per_tok"],
              moe_intermediate_size=hf["moe_intermediate_size"],
              num_hidden_layers=hf["num_hidden_layers"], vocab_size=hf["vocab_size"],
              rms_norm_eps=float(hf.get("rms_norm_eps", 1e-6)), rope_theta=theta)
    kw.update(overrides)
    return Q.Qwen3MoeMKConfig(**kw)


def gpt_oss_config(hf: dict, **overrides) -> G.GptOssMKConfig:
    """HF GPT-OSS config.json fields -> GptOssMKConfig (hidden padded to a multiple
    of 512, as the reference pads 2880 to 3072; YaRN rope parameters; sliding /
    full layer alternation from layer_types)."""
    if hf.get("model_type", "gpt_oss") != "gpt_oss":
        raise ValueError(f"not a GPT-OSS config (model_type={hf.get('model_type')!r})")
    H, nq = hf["hidden_size"], hf["num_attention_heads"]
    L = hf["num_hidden_layers"]
    types = hf.get("layer_types")
    first_sliding = True
    if types:
        first_sliding = types[0] == "sliding_attention"
        for l, t in enumerate(types):
            if (t == "sliding_attention") != ((l % 2 == 0) == first_sliding):
                raise ValueError("GPT-OSS: only alternating sliding / full layers are supported")
    theta, rs = _rope(hf, 150000.0)
    if rs and rs.get("rope_type", rs.get("type")) != "yarn":
        raise ValueError(f"GPT-OSS: rope_scaling {rs!r} is not supported (YaRN only)")
    kw = dict(hidden_size=H, hidden_pad=(H + 511) // 512 * 512, num_attention_heads=nq,
              num_key_value_heads=hf.get("num_key_value_heads", nq), head_dim=hf.get("head_dim", H // nq),
              num_experts=hf.get("num_local_experts", hf.get("num_experts")),
              num_experts_per_tok=hf.get("num_experts_per_tok", hf.get("experts_per_token")),
              intermediate_size=hf["intermediate_size"], num_hidden_layers=L, vocab_size=hf["vocab_size"],
              rms_norm_eps=float(hf.get("rms_norm_eps", 1e-5)),
              sliding_window=hf.get("sliding_window", 128), swiglu_limit=float(hf.get("swiglu_limit", 7.0)),
              rope_theta=theta, first_sliding=first_sliding)
    if rs:
        kw.update(rope_factor=float(rs.get("factor", 32.0)), rope_beta_fast=float(rs.get("beta_fast", 32.0)),
                  rope_beta_slow=float(rs.get("beta_slow", 1.0)),
                  rope_original_max=int(rs.get("original_max_position_embeddings", 4096)),
                  rope_truncate=bool(rs.get("truncate", False)))
    kw.update(overrides)
    return G.GptOssMKConfig(**kw)


def mxfp4_dequantize(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """MXFP4 blocks [..., N, K/32, 16] uint8 (two E2M1 codes per byte, low nibble
    first) + scales [..., N, K/32] uint8 (E8M0: 2^(byte - 127)) -> bf16 [..., N, K].
    Runs on the tensors' device."""
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise ValueError("MXFP4 blocks and scales must be uint8")
    if blocks.shape[-1] != 16 or tuple(blocks.shape[:-1]) != tuple(scales.shape):
        raise ValueError(f"MXFP4 blocks {tuple(blocks.shape)} do not match scales {tuple(scales.shape)}")
    if bool((scales == 255).any()):
        raise ValueError("MXFP4 scale byte 0xFF (NaN) in the checkpoint")
    lut = torch.tensor(_E2M1, dtype=torch.float32, device=blocks.device)
    lo = lut[(blocks & 0x0F).long()]
    hi = lut[(blocks >> 4).long()]
    vals = torch.stack([lo, hi], -1).flatten(-2)                      # [..., N, K/32, 32]
    vals = torch.ldexp(vals, scales.to(torch.int32).unsqueeze(-1) - 127)
    return vals.flatten(-2).to(torch.bfloat16)


def _qwen_head(ck: SafetensorsCheckpoint, device):
    embed = ck.get("model.embed_tokens.weight")
    ln_f = ck.get("model.norm.weight")
    lm = ck.get("lm_head.weight")
    if lm is None and ck.config.get("tie_word_embeddings", False):
        lm = embed
    to = lambda t: t.to(device=device, dtype=torch.bfloat16).contiguous() if t is not None else None
    return to(embed), to(ln_f), to(lm)


def load_qwen3_moe(path: str, batch: int = 1, device="cuda", **overrides) -> Q.Qwen3MoeMegakernelModel:
    """Qwen3-MoE checkpoint directory -> Qwen3MoeMegakernelModel on `device`
    (layers converted and packed one at a time)."""
    ck = SafetensorsCheckpoint(path)
    overrides.setdefault("max_batch", batch)
    cfg = qwen3_moe_config(ck.config, **overrides)
    layers = Q.convert_qwen3_moe_hf_to_mkd(ck, cfg, device)
    embed, ln_f, lm = _qwen_head(ck, device)
    return Q.Qwen3MoeMegakernelModel(cfg, layers, batch, device, embed=embed, ln_f=ln_f, lm_head=lm)


def gpt_oss_layer_hf(ck, layer: int, device) -> Dict[str, torch.Tensor]:
    """One GPT-OSS layer of an HF checkpoint in the key layout of
    gpt_oss_with_megakernel.random_layer_hf (experts [E, H, 2I] interleaved and
    [E, I, H]; MXFP4 experts decoded to bf16 on `device`)."""
    p = f"model.layers.{layer}."
    if p + "self_attn.q_proj.weight" not in ck:
        p = f"layers.{layer}."

    def t(name, dtype=torch.bfloat16):
        if p + name not in ck:
            raise KeyError(f"layer {layer}: missing {p + name}")
        return ck[p + name].to(device=device, dtype=dtype)

    def experts(proj):
        if p + f"mlp.experts.{proj}_blocks" in ck:
            w = mxfp4_dequantize(t(f"mlp.experts.{proj}_blocks", torch.uint8),
                                 t(f"mlp.experts.{proj}_scales", torch.uint8))   # [E, N, K]
            return w.transpose(1, 2).contiguous()                                # [E, K, N]
        return t(f"mlp.experts.{proj}")

    hf = {f"{n}_proj.{k}": t(f"self_attn.{n}_proj.{k}") for n in "qkvo" for k in ("weight", "bias")}
    hf.update({
        "sinks": t("self_attn.sinks", torch.float32),
        "input_layernorm": t("input_layernorm.weight"),
        "post_attention_layernorm": t("post_attention_layernorm.weight"),
        "router.weight": t("mlp.router.weight"), "router.bias": t("mlp.router.bias"),
        "experts.gate_up_proj": experts("gate_up_proj"),
        "experts.gate_up_proj_bias": t("mlp.experts.gate_up_proj_bias"),
        "experts.down_proj": experts("down_proj"),
        "experts.down_proj_bias": t("mlp.experts.down_proj_bias"),
    })
    return hf


def load_gpt_oss(path: str, batch: int = 1, device="cuda", **overrides) -> G.GptOssMegakernelModel:
    """GPT-OSS checkpoint directory (bf16 or MXFP4 experts) -> GptOssMegakernelModel
    on `device` (layers decoded, converted and packed one at a time)."""
    ck = SafetensorsCheckpoint(path)
    overrides.setdefault("max_batch", batch)
    cfg = gpt_oss_config(ck.config, **overrides)
    layers = []
    for l in range(cfg.num_hidden_layers):
        layers.append(G.pack_layer(gpt_oss_layer_hf(ck, l, device), cfg))
    embed, ln_f, lm = _qwen_head(ck, device)
    return G.GptOssMegakernelModel(cfg, layers, batch, device, embed=embed, ln_f=ln_f, lm_head=lm)
