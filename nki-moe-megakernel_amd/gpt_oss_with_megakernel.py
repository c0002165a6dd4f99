"""GPT-OSS-20B-shaped decode on the MI355X library (the reference's
megakernels/gpt_oss/gpt_oss_with_megakernel.py + transformer_gpt_oss.py).

Model boundary: ``GptOssMegakernelModel.get_model_output(input_ids,
position_ids)`` returns ``(norm(Y), [K0, V0, K1, V1, ...])`` like
NeuronGptOssModelV1.get_model_output (gpt_oss_with_megakernel.py:577-690), and
``step`` runs a whole greedy decode step into caller buffers (graph-capturable).

Layer flow (transformer_gpt_oss.py:239-522), all layers in one
``mkd_qwen3_decode_layers`` call with ``variant = MKD_VARIANT_GPT_OSS``:
rmsnorm_tkg (eps 1e-5, hidden 2880 zero-padded to 3072, divisor 2880) ->
QKV (+bias) -> RoPE (YaRN tables) -> GQA attention with learned sinks, even
layers sliding-window 128 (ring cache of 128 rows, new row at pos % 127),
odd layers full -> o_proj (+bias) -> residual -> rmsnorm_tkg -> router (bias,
top-4 on logits, softmax over the top-4) -> experts (Swish alpha 1.702, gate
<= 7, up + 1 in [-6, 8], biases; bf16, MXFP8 or MXFP4 weights) -> residual.

Weight conversion (gpt_oss_with_megakernel.py:290-327, 397-454, 490-567):
HF's expert gate_up [E, H, 2I] interleaves gate / up columns ([..., ::2],
[..., 1::2]); they are de-interleaved into gate rows then up rows, the HF
``up + 1`` is folded into the up bias, H is zero-padded to a multiple of 512.
"""
from __future__ import annotations

import math
from ctypes import c_int as C_int
from dataclasses import dataclass
from typing import Dict, List, Optional

import torch
from torch import nn

from . import _lib as L
from . import packing
from .qwen_with_megakernel import (EXPERT_FORMATS, _LayerStack, _prefill, check_waits, pack_experts_mx,
                                   randn_bf16, tensor_seed)

VARIANT_GPT_OSS = 1


@dataclass
class GptOssMKConfig:
    hidden_size: int = 2880
    hidden_pad: int = 3072             # multiple of 512 (the reference pads H to 3072)
    num_attention_heads: int = 64
    num_key_value_heads: int = 8
    head_dim: int = 64
    num_experts: int = 32
    num_experts_per_tok: int = 4
    intermediate_size: int = 2880
    num_hidden_layers: int = 24
    vocab_size: int = 201088
    rms_norm_eps: float = 1e-5
    sliding_window: int = 128
    swiglu_limit: float = 7.0
    alpha: float = 1.702
    rope_theta: float = 150000.0
    rope_factor: float = 32.0
    rope_beta_fast: float = 32.0
    rope_beta_slow: float = 1.0
    rope_original_max: int = 4096
    rope_truncate: bool = False        # GPT-OSS keeps the correction range unrounded
    max_batch: int = 1
    max_seq: int = 4224                # full-attention cache rows per sequence
    expert_format: str = "mxfp4"
    first_sliding: bool = True         # layer 0 slides, then alternate

    def is_sliding(self, layer: int) -> bool:
        # even layers slide (transformer_gpt_oss.py:366)
        return (layer % 2 == 0) == self.first_sliding


def yarn_inv_freq(cfg: GptOssMKConfig):
    """YaRN RoPE frequencies and attention scaling (the published YaRN rule as used by
    HF's "yarn" rope type): per dimension pair, interpolate between the extrapolated
    frequency theta^(-2i/d) and the interpolated one (/ factor) with a linear ramp
    between the dims whose wavelength completes beta_fast and beta_slow rotations
    over the original context (rounded outwards only with rope_truncate); cos / sin
    are scaled by 0.1 * ln(factor) + 1.  Returns (inv_freq [d/2] fp32,
    attention_scaling)."""
    d = cfg.head_dim
    base, factor = cfg.rope_theta, cfg.rope_factor
    pos_freqs = base ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
    extra = 1.0 / pos_freqs
    inter = 1.0 / (factor * pos_freqs)

    def corr_dim(rot):
        return (d * math.log(cfg.rope_original_max / (rot * 2 * math.pi))) / (2 * math.log(base))

    low, high = corr_dim(cfg.rope_beta_fast), corr_dim(cfg.rope_beta_slow)
    if cfg.rope_truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0), min(high, d - 1)
    if low == high:
        high += 0.001
    ramp = ((torch.arange(d // 2, dtype=torch.float64) - low) / (high - low)).clamp(0, 1)
    extra_factor = 1 - ramp
    inv_freq = inter * (1 - extra_factor) + extra * extra_factor
    return inv_freq.float(), 0.1 * math.log(factor) + 1.0


def random_layer_hf(cfg: GptOssMKConfig, layer: int, seed: int, device) -> Dict[str, torch.Tensor]:
    """HF-layout GPT-OSS layer weights (modeling_gpt_oss.py): linears and biases
    N(0, 0.02), norm gammas 1 + N(0, 0.02), sinks N(0, 1); experts gate_up
    [E, H, 2I] with interleaved gate / up columns."""
    H, nq, nkv, d = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    E, I = cfg.num_experts, cfg.intermediate_size
    r = lambda name, shape, **kw: randn_bf16(shape, tensor_seed(seed, layer, name), device, **kw)
    return {
        "q_proj.weight": r("q_proj", (nq * d, H)), "q_proj.bias": r("q_bias", (nq * d,)),
        "k_proj.weight": r("k_proj", (nkv * d, H)), "k_proj.bias": r("k_bias", (nkv * d,)),
        "v_proj.weight": r("v_proj", (nkv * d, H)), "v_proj.bias": r("v_bias", (nkv * d,)),
        "o_proj.weight": r("o_proj", (H, nq * d)), "o_proj.bias": r("o_bias", (H,)),
        "sinks": r("sinks", (nq,), std=1.0).float(),
        "input_layernorm": r("input_layernorm", (H,), mean=1.0),
        "post_attention_layernorm": r("post_attention_layernorm", (H,), mean=1.0),
        "router.weight": r("router", (E, H)), "router.bias": r("router_bias", (E,)),
        "experts.gate_up_proj": r("gate_up_proj", (E, H, 2 * I)),
        "experts.gate_up_proj_bias": r("gate_up_bias", (E, 2 * I)),
        "experts.down_proj": r("down_proj", (E, I, H)),
        "experts.down_proj_bias": r("down_bias", (E, H)),
    }


@dataclass
class PackedGptOssLayer:
    w_qkv: torch.Tensor
    b_qkv: torch.Tensor
    w_o: torch.Tensor
    b_o: torch.Tensor
    sinks: torch.Tensor
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    router: torch.Tensor
    router_bias: torch.Tensor
    gate_up: torch.Tensor
    gate_up_bias: torch.Tensor
    down: torch.Tensor
    down_bias: torch.Tensor
    gate_up_scales: Optional[torch.Tensor] = None
    down_scales: Optional[torch.Tensor] = None


def _pad_cols(w: torch.Tensor, n: int) -> torch.Tensor:
    out = torch.zeros(*w.shape[:-1], n, dtype=w.dtype, device=w.device)
    out[..., : w.shape[-1]] = w
    return out


def _pad_rows(w: torch.Tensor, n: int, dim: int = 0) -> torch.Tensor:
    shape = list(w.shape)
    shape[dim] = n
    out = torch.zeros(shape, dtype=w.dtype, device=w.device)
    out.narrow(dim, 0, w.shape[dim]).copy_(w)
    return out


def convert_layer(hf: Dict[str, torch.Tensor], cfg: GptOssMKConfig) -> Dict[str, torch.Tensor]:
    """HF layer -> padded, de-interleaved tensors in this build's logical layouts:
    w_qkv [(nq+2nkv)d, Hp], w_o [Hp, nq d], gate_up rows [E, 2I, Hp] (gate then up),
    gate_up bias [E, 2, I] (up bias + 1), down [E, Hp, I], down bias [E, Hp]."""
    Hp = cfg.hidden_pad
    wqkv = torch.cat([hf["q_proj.weight"], hf["k_proj.weight"], hf["v_proj.weight"]], 0)
    bqkv = torch.cat([hf["q_proj.bias"], hf["k_proj.bias"], hf["v_proj.bias"]], 0)
    gu = hf["experts.gate_up_proj"]                               # [E, H, 2I] interleaved
    gub = hf["experts.gate_up_proj_bias"].float()                 # [E, 2I] interleaved
    gate, up = gu[..., 0::2], gu[..., 1::2]                       # [E, H, I]
    rows = torch.cat([gate.transpose(1, 2), up.transpose(1, 2)], 1)   # [E, 2I, H]
    bias = torch.stack([gub[:, 0::2], gub[:, 1::2] + 1.0], 1).to(torch.bfloat16)
    down = hf["experts.down_proj"].transpose(1, 2)                # [E, H, I]
    return {
        "w_qkv": _pad_cols(wqkv, Hp).contiguous(),
        "b_qkv": bqkv.contiguous(),
        "w_o": _pad_rows(hf["o_proj.weight"], Hp).contiguous(),
        "b_o": _pad_rows(hf["o_proj.bias"], Hp).contiguous(),
        "sinks": hf["sinks"].float().contiguous(),
        "ln_in": _pad_rows(hf["input_layernorm"], Hp).contiguous(),
        "ln_post": _pad_rows(hf["post_attention_layernorm"], Hp).contiguous(),
        "router": _pad_cols(hf["router.weight"], Hp).contiguous(),
        "router_bias": hf["router.bias"].contiguous(),
        "gate_up": _pad_cols(rows, Hp).contiguous(),
        "gate_up_bias": bias.contiguous(),
        "down": _pad_rows(down, Hp, 1).contiguous(),
        "down_bias": _pad_rows(hf["experts.down_proj_bias"], Hp, 1).contiguous(),
    }


def pack_layer(hf: Dict[str, torch.Tensor], cfg: GptOssMKConfig) -> PackedGptOssLayer:
    c = convert_layer(hf, cfg)
    fmt = EXPERT_FORMATS[cfg.expert_format]
    if fmt:
        gu, gus, dn, dns = pack_experts_mx(c["gate_up"], c["down"], fmt)
    else:
        gu = packing.pack_experts_gate_up_hf(c["gate_up"])
        dn = packing.pack_experts_down_hf(c["down"])
        gus = dns = None
    return PackedGptOssLayer(
        w_qkv=packing.pack_out_in(c["w_qkv"]), b_qkv=c["b_qkv"], w_o=packing.pack_out_in(c["w_o"]),
        b_o=c["b_o"], sinks=c["sinks"], ln_in=c["ln_in"], ln_post=c["ln_post"],
        router=packing.pack_out_in(c["router"]), router_bias=c["router_bias"],
        gate_up=gu, gate_up_bias=c["gate_up_bias"], down=dn, down_bias=c["down_bias"],
        gate_up_scales=gus, down_scales=dns)


class GptOssKVCache:
    """Per-layer caches: sliding layers [B, nkv, W, d] (ring), full layers
    [B, nkv, max_seq, d]; ``past_key_values`` is flat [K0, V0, K1, V1, ...]."""

    def __init__(self, cfg: GptOssMKConfig, batch: int, device):
        self.rows = [cfg.sliding_window if cfg.is_sliding(l) else cfg.max_seq
                     for l in range(cfg.num_hidden_layers)]
        self.past_key_values = []
        for l in range(cfg.num_hidden_layers):
            shape = (batch, cfg.num_key_value_heads, self.rows[l], cfg.head_dim)
            self.past_key_values.append(torch.zeros(shape, dtype=torch.bfloat16, device=device))
            self.past_key_values.append(torch.zeros(shape, dtype=torch.bfloat16, device=device))

    def k(self, l):
        return self.past_key_values[2 * l]

    def v(self, l):
        return self.past_key_values[2 * l + 1]


class GptOssMegakernelModel(_LayerStack, nn.Module):
    """GPT-OSS decoder stack + decode-step epilogue on the MI355X library."""

    def __init__(self, cfg: GptOssMKConfig, layers: List[PackedGptOssLayer], batch: int, device,
                 embed: Optional[torch.Tensor] = None, ln_f: Optional[torch.Tensor] = None,
                 lm_head: Optional[torch.Tensor] = None):
        super().__init__()
        if cfg.hidden_pad % 512 or cfg.hidden_pad < cfg.hidden_size:
            raise ValueError("hidden_pad must be a multiple of 512 and >= hidden_size")
        self.cfg = cfg
        self.batch = batch
        self.device = torch.device(device)
        self.packed = layers
        self.kv_mgr = GptOssKVCache(cfg, batch, device)
        Hp = cfg.hidden_pad
        self.embed_tokens = _pad_cols(embed, Hp).contiguous() if embed is not None else None
        self.ln_f = _pad_rows(ln_f, Hp).contiguous() if ln_f is not None else None
        self.lm_head_packed = packing.pack_out_in(_pad_cols(lm_head, Hp).contiguous()) \
            if lm_head is not None else None
        inv, self.attn_scaling = yarn_inv_freq(cfg)
        self.inv_freq = inv.to(device)
        self._build_struct()
        lib = L.load()
        self.ws = torch.zeros(max(lib.mkd_qwen3_workspace_bytes(self._model, batch), 256),
                              dtype=torch.uint8, device=device)
        self.lm_ws = torch.empty(max(lib.mkd_lm_head_workspace_bytes(batch, Hp, cfg.vocab_size), 256),
                                 dtype=torch.uint8, device=device)
        self.cos = torch.empty(batch, cfg.head_dim, dtype=torch.float32, device=device)
        self.sin = torch.empty(batch, cfg.head_dim, dtype=torch.float32, device=device)

    def _build_struct(self):
        cfg, Ln = self.cfg, self.cfg.num_hidden_layers
        arr = lambda ts: (L.vp * Ln)(*[t.data_ptr() if t is not None else None for t in ts])
        p = self.packed
        fmt = EXPERT_FORMATS[cfg.expert_format]
        self._arrays = {
            "w_qkv": arr([x.w_qkv for x in p]), "w_o": arr([x.w_o for x in p]),
            "ln_in": arr([x.ln_in for x in p]), "ln_post": arr([x.ln_post for x in p]),
            "router": arr([x.router for x in p]), "gate_up": arr([x.gate_up for x in p]),
            "down": arr([x.down for x in p]),
            "k_cache": arr([self.kv_mgr.k(l) for l in range(Ln)]),
            "v_cache": arr([self.kv_mgr.v(l) for l in range(Ln)]),
            "b_qkv": arr([x.b_qkv for x in p]), "b_o": arr([x.b_o for x in p]),
            "sinks": arr([x.sinks for x in p]), "router_bias": arr([x.router_bias for x in p]),
            "gate_up_bias": arr([x.gate_up_bias for x in p]),
            "down_bias": arr([x.down_bias for x in p]),
        }
        if fmt:
            self._arrays["gate_up_scales"] = arr([x.gate_up_scales for x in p])
            self._arrays["down_scales"] = arr([x.down_scales for x in p])
        self._window = (C_int * Ln)(*[cfg.sliding_window if cfg.is_sliding(l) else 0 for l in range(Ln)])
        self._rows = (C_int * Ln)(*self.kv_mgr.rows)
        self._model = L.Qwen3Model(
            num_layers=Ln, H=cfg.hidden_pad, nq=cfg.num_attention_heads,
            nkv=cfg.num_key_value_heads, d=cfg.head_dim, E=cfg.num_experts,
            K=cfg.num_experts_per_tok, I=cfg.intermediate_size, S_max=cfg.max_seq,
            eps=cfg.rms_norm_eps, inv_freq=None, expert_format=fmt,
            variant=VARIANT_GPT_OSS, H_actual=cfg.hidden_size, window=self._window,
            layer_s_max=self._rows, act_alpha=cfg.alpha, gate_hi=cfg.swiglu_limit,
            gate_lo=-math.inf, up_hi=cfg.swiglu_limit + 1.0, up_lo=-cfg.swiglu_limit + 1.0,
            **self._arrays)

    def rope_cos_sin(self, position_ids: torch.Tensor, cos=None, sin=None):
        """YaRN cos/sin [B, d] (halves duplicated, attention scaling folded in)."""
        freqs = position_ids.reshape(-1, 1).float() * self.inv_freq[None, :]
        emb = torch.cat([freqs, freqs], -1)
        c = emb.cos() * self.attn_scaling
        s = emb.sin() * self.attn_scaling
        if cos is not None:
            cos.copy_(c)
            sin.copy_(s)
            return cos, sin
        return c, s

    def decode_layers(self, hidden: torch.Tensor, position_ids: torch.Tensor, layers=None):
        """All layers (or the range `layers` = (lo, hi)) in place on hidden [B, hidden_pad]
        bf16 (padded columns zero)."""
        B = hidden.shape[0]
        if B > self.batch:
            raise ValueError(f"batch {B} exceeds the configured max batch {self.batch}")
        if hidden.dtype != torch.bfloat16 or not hidden.is_contiguous() or hidden.shape[1] != self.cfg.hidden_pad:
            raise ValueError(f"hidden must be a contiguous bf16 [B, {self.cfg.hidden_pad}] tensor")
        pos = position_ids.reshape(-1)
        if pos.dtype != torch.int32:
            raise ValueError("position_ids must be int32")
        cos, sin = self.rope_cos_sin(pos, self.cos[:B], self.sin[:B])
        rc = L.load().mkd_qwen3_decode_layers(
            self._struct_for(layers), B, hidden.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(),
            self.ws.data_ptr(), self.ws.numel(), L.stream_ptr(self.device))
        L.check(rc, "gpt_oss decode_layers")
        return hidden

    def step(self, token_ids, position_ids, hidden, logits, next_tokens):
        """Greedy decode step into caller buffers (no allocation; graph-capturable)."""
        lib = L.load()
        B = hidden.shape[0]
        Hp = self.cfg.hidden_pad
        s = L.stream_ptr(self.device)
        L.check(lib.mkd_embed(token_ids.data_ptr(), self.embed_tokens.data_ptr(), hidden.data_ptr(),
                              B, Hp, self.embed_tokens.shape[0], s), "embed")
        self.decode_layers(hidden, position_ids)
        L.check(lib.mkd_lm_head_greedy(hidden.data_ptr(), self.ln_f.data_ptr(), self.cfg.rms_norm_eps,
                                       self.lm_head_packed.data_ptr(), B, Hp, self.cfg.vocab_size,
                                       self.cfg.hidden_size, 1, logits.data_ptr(),
                                       next_tokens.data_ptr(), self.lm_ws.data_ptr(),
                                       self.lm_ws.numel(), s), "lm_head")
        return next_tokens

    def prefill(self, input_ids: torch.Tensor, start_pos: int = 0, seq: int = 0, chunk: int = 4096):
        """Context encoding of one sequence: input_ids [T] fill the caches of sequence
        `seq` from start_pos, then the step epilogue on the last token: (logits [V]
        fp32, next id [1] int32).  The sliding-window layers' ring caches take one
        token per pass, so a model with them prefills token by token."""
        if any(self.cfg.is_sliding(l) for l in range(self.cfg.num_hidden_layers)):
            chunk = 1
        return _prefill(self, input_ids, start_pos, seq, chunk, self.cfg.hidden_pad, self.cfg.hidden_size,
                        1, lambda pos: self.rope_cos_sin(pos))

    def get_model_output(self, input_ids: Optional[torch.Tensor] = None, seq_ids=None,
                         attention_mask=None, position_ids: Optional[torch.Tensor] = None,
                         past_key_values=None, active_mask=None, inputs_embeds=None, prev_hidden=None,
                         adapter_ids=None, rotary_position_ids=None, update_cache: bool = False,
                         is_for_context_encoding: bool = False, vision_embeddings=None,
                         vision_mask=None, deepstack_vision_embeds=None, local_attn_mask=None,
                         windowed_context_encoding_window_idx: int = -1, padding_mask=None, **kwargs):
        """NeuronGptOssModelV1.get_model_output (gpt_oss_with_megakernel.py:577-690):
        embed (or inputs_embeds [B, S, H]) -> all layers -> final norm; returns
        (norm(Y) [B, S, H], [K0, V0, K1, V1, ...]) with the caches updated in place.
        Token generation (S = 1) runs the decode layers at position_ids [B, 1];
        context encoding runs each sequence's S tokens at consecutive
        position_ids (one token per pass: the sliding-window layers' ring rows).
        As in the reference's TKG path, attention masks, active_mask,
        past_key_values (the model's own caches are used), update_cache and
        rotary_position_ids carry no extra information; LoRA adapters, vision
        inputs, windowed context encoding and cache slots other than the batch
        rows (seq_ids != arange(B)) are not supported."""
        for name, v in (("adapter_ids", adapter_ids), ("vision_embeddings", vision_embeddings),
                        ("vision_mask", vision_mask), ("deepstack_vision_embeds", deepstack_vision_embeds),
                        ("local_attn_mask", local_attn_mask), ("prev_hidden", prev_hidden)):
            if v is not None:
                raise NotImplementedError(f"get_model_output: {name} is not supported")
        if windowed_context_encoding_window_idx != -1:
            raise NotImplementedError("get_model_output: windowed context encoding is not supported")
        if position_ids is None:
            raise ValueError("get_model_output needs position_ids")
        cfg, Hp = self.cfg, self.cfg.hidden_pad
        if inputs_embeds is not None:
            B, S = inputs_embeds.shape[:2]
        else:
            ids = input_ids.reshape(input_ids.shape[0], -1)
            B, S = ids.shape
        if seq_ids is not None and not torch.equal(seq_ids.reshape(-1).cpu().long(), torch.arange(B)):
            raise NotImplementedError("get_model_output: seq_ids must be arange(B) (batch row b is cache slot b)")
        if B > self.batch:
            raise ValueError(f"batch {B} exceeds the configured max batch {self.batch}")
        hidden = torch.zeros(B * S, Hp, dtype=torch.bfloat16, device=self.device)
        s = L.stream_ptr(self.device)
        if inputs_embeds is not None:
            hidden[:, : cfg.hidden_size] = inputs_embeds.reshape(B * S, -1)[:, : cfg.hidden_size].to(torch.bfloat16)
        else:
            L.check(L.load().mkd_embed(ids.reshape(-1).to(device=self.device, dtype=torch.int32).contiguous().data_ptr(),
                                       self.embed_tokens.data_ptr(), hidden.data_ptr(), B * S, Hp,
                                       self.embed_tokens.shape[0], s), "embed")
        pos = position_ids.reshape(B, S).to(device=self.device, dtype=torch.int32)
        if not is_for_context_encoding:
            if S != 1:
                raise NotImplementedError("token generation takes one token per sequence")
            self.decode_layers(hidden, pos.reshape(-1).contiguous())
            check_waits(self, B, self.ws)
        else:
            from .qwen_with_megakernel import prefill_rows
            hv = hidden.reshape(B, S, Hp)
            pc = pos.cpu().long()
            for b in range(B):
                if not torch.equal(pc[b], torch.arange(int(pc[b, 0]), int(pc[b, 0]) + S)):
                    raise NotImplementedError("context encoding needs consecutive position_ids")
                for t in range(S):   # sliding-window ring rows: one token per pass
                    row = hv[b, t:t + 1].contiguous()
                    prefill_rows(self, row, int(pc[b, t]), b, rope=lambda p: self.rope_cos_sin(p))
                    hv[b, t] = row[0]
                    if self.route_log_history is not None:
                        self.route_log_history.append(self.route_log(1))
        normed = torch.empty_like(hidden)
        L.check(L.load().mkd_rmsnorm_tkg(hidden.data_ptr(), L.DT_BF16, self.ln_f.data_ptr(),
                                         normed.data_ptr(), L.DT_BF16, B * S, Hp, cfg.hidden_size,
                                         cfg.rms_norm_eps, s), "final norm")
        return normed.reshape(B, S, Hp)[:, :, : cfg.hidden_size], list(self.kv_mgr.past_key_values)


NeuronGptOssForCausalLM = GptOssMegakernelModel
