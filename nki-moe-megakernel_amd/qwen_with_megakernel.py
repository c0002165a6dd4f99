"""Qwen3-MoE decode through the MI355X megakernel library.

Mirrors megakernels/qwen3_moe/qwen_with_megakernel.py:
  * ``convert_qwen3_moe_hf_to_mkd`` <- convert_qwen3_moe_hf_to_neuron_state_dict
    (:171-271): HF state dict -> the library's packed layouts.
  * ``Qwen3MoeDecoderLayerMK.forward`` <- NeuronQwen3MoeDecoderLayerV3.forward
    (:422-526): on token generation layer 0 runs the whole L-layer stack in one
    library call (mkd_qwen3_decode_layers, the counterpart of
    transformer_qwen3_moe_tkg_multilayer) and the other layers pass through;
    returns (Y, (K0, V0), cos, sin, None).
  * ``Qwen3MoeMegakernelModel`` <- NeuronQwen3MoeModelV3 (:560-594) plus the
    NxDI decode-step pieces the reference delegates (embedding, final norm,
    lm_head :533-553, greedy sampling main.py:390-398), with an optional
    HIP-graph capture of the whole step.

KV caches are [B, kv_heads, S_max, d] bf16 per layer and are updated in place
at position_ids (the reference's [B, 1, S_prior, d] per TP rank).
"""
from __future__ import annotations

import ctypes as C
import hashlib
import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch
from torch import nn

from . import _lib as L
from . import packing


def set_decode_path(mode: str = "multi_kernel") -> None:
    """Decode-layer execution (process-global): "multi_kernel" (default) runs
    each layer as a short kernel sequence (at one token with bf16 experts the
    router top-k, gate/up and down projections share one launch, the down
    blocks waiting inside it for their expert's gate/up blocks); "persistent"
    runs each layer as one persistent kernel launch where the model and batch
    allow it; "separate_launches" is "multi_kernel" with every stage a launch
    of its own."""
    modes = {"multi_kernel": 0, "persistent": 1, "separate_launches": 2}
    if mode not in modes:
        raise ValueError(f"decode path {mode!r} not in {sorted(modes)}")
    L.check(L.load().mkd_set_decode_path(modes[mode]), "set_decode_path")


@dataclass
class Qwen3MoeMKConfig:
    hidden_size: int = 2048
    num_attention_heads: int = 32
    num_key_value_heads: int = 4
    head_dim: int = 128
    num_experts: int = 128
    num_experts_per_tok: int = 8
    moe_intermediate_size: int = 768
    num_hidden_layers: int = 48
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_batch: int = 1
    max_seq: int = 2304           # KV capacity per sequence
    expert_format: str = "bf16"   # "bf16", "mxfp8" (E4M3) or "mxfp4" (E2M1) expert weights
    kv_block_len: int = 0         # > 0: paged KV cache with blocks of this many positions

    @property
    def qkv_out(self) -> int:
        return (self.num_attention_heads + 2 * self.num_key_value_heads) * self.head_dim


def tensor_seed(base: int, layer: int, name: str) -> int:
    """Deterministic per-tensor seed from (base seed, layer, tensor name)."""
    h = hashlib.sha256(f"{base}/{layer}/{name}".encode()).digest()
    return int.from_bytes(h[:8], "little") & ((1 << 63) - 1)


def randn_bf16(shape, seed: int, device, std: float = 0.02, mean: float = 0.0) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    return (t * std + mean).to(torch.bfloat16)


def random_layer_hf(cfg: Qwen3MoeMKConfig, layer: int, seed: int, device) -> Dict[str, torch.Tensor]:
    """HF-layout weights of one layer: linears N(0, 0.02), norm gammas 1 + N(0, 0.02)
    (HF initialises gammas to 1; the perturbation keeps the gamma multiply non-trivial)."""
    H, nq, nkv, d = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    E, I = cfg.num_experts, cfg.moe_intermediate_size
    r = lambda name, shape, **kw: randn_bf16(shape, tensor_seed(seed, layer, name), device, **kw)
    return {
        "q_proj": r("q_proj", (nq * d, H)),
        "k_proj": r("k_proj", (nkv * d, H)),
        "v_proj": r("v_proj", (nkv * d, H)),
        "o_proj": r("o_proj", (H, nq * d)),
        "q_norm": r("q_norm", (d,), mean=1.0),
        "k_norm": r("k_norm", (d,), mean=1.0),
        "input_layernorm": r("input_layernorm", (H,), mean=1.0),
        "post_attention_layernorm": r("post_attention_layernorm", (H,), mean=1.0),
        "gate": r("gate", (E, H)),
        "gate_up_proj": r("gate_up_proj", (E, 2 * I, H)),
        "down_proj": r("down_proj", (E, H, I)),
    }


@dataclass
class PackedLayer:
    w_qkv: torch.Tensor
    w_o: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    router: torch.Tensor
    gate_up: torch.Tensor
    down: torch.Tensor
    gate_up_scales: Optional[torch.Tensor] = None   # MX experts only
    down_scales: Optional[torch.Tensor] = None


EXPERT_FORMATS = {"bf16": 0, "mxfp8": 1, "mxfp4": 2}


def pack_experts_mx(gate_up: torch.Tensor, down: torch.Tensor, fmt: int):
    """HF expert weights gate_up [E, 2I, H], down [E, H, I] (bf16) -> MX quantised
    (OCP rule, one E8M0 per 32 along the contraction) and packed:
    (gate_up, gate_up_scales, down, down_scales)."""
    from . import mx
    E, N2, H = gate_up.shape
    I = N2 // 2
    gc, gs = mx.quantize_mx(gate_up.reshape(E * N2, H), fmt, H)
    gu, gus = mx.pack_mx(gc.reshape(E, N2, -1), gs.reshape(E, N2, -1), fmt, H, I)
    dc, ds = mx.quantize_mx(down.reshape(E * H, I), fmt, (I + 127) // 128 * 128)
    dn, dns = mx.pack_mx(dc.reshape(E, H, -1), ds.reshape(E, H, -1), fmt, I)
    return gu, gus, dn, dns


def pack_layer(hf: Dict[str, torch.Tensor], expert_format: str = "bf16") -> PackedLayer:
    """One layer of HF weights -> packed (convert_qwen3_moe_hf_to_neuron_state_dict's role).
    expert_format "mxfp8" / "mxfp4" quantises the experts to MX first."""
    wqkv = torch.cat([hf["q_proj"], hf["k_proj"], hf["v_proj"]], 0).contiguous()
    fmt = EXPERT_FORMATS[expert_format]
    if fmt:
        gu, gus, dn, dns = pack_experts_mx(hf["gate_up_proj"].contiguous(), hf["down_proj"].contiguous(), fmt)
    else:
        gu = packing.pack_experts_gate_up_hf(hf["gate_up_proj"].contiguous())
        dn = packing.pack_experts_down_hf(hf["down_proj"].contiguous())
        gus = dns = None
    return PackedLayer(
        w_qkv=packing.pack_out_in(wqkv),
        w_o=packing.pack_out_in(hf["o_proj"].contiguous()),
        q_norm=hf["q_norm"].contiguous(), k_norm=hf["k_norm"].contiguous(),
        ln_in=hf["input_layernorm"].contiguous(),
        ln_post=hf["post_attention_layernorm"].contiguous(),
        router=packing.pack_out_in(hf["gate"].contiguous()),
        gate_up=gu, down=dn, gate_up_scales=gus, down_scales=dns,
    )


def convert_qwen3_moe_hf_to_mkd(state_dict: Dict[str, torch.Tensor], cfg: Qwen3MoeMKConfig,
                                device) -> List[PackedLayer]:
    """HF Qwen3-MoE state dict (``model.layers.{l}...`` or ``layers.{l}...`` keys;
    experts either fused [E, 2I, H] / [E, H, I] or per-expert gate/up/down) ->
    packed layers on `device`."""
    def get(l, *names):
        for pre in (f"model.layers.{l}.", f"layers.{l}."):
            for n in names:
                if pre + n in state_dict:
                    return state_dict[pre + n].to(device=device, dtype=torch.bfloat16)
        return None

    layers = []
    for l in range(cfg.num_hidden_layers):
        gu = get(l, "mlp.experts.gate_up_proj")
        dn = get(l, "mlp.experts.down_proj")
        if gu is None:
            gates = [get(l, f"mlp.experts.{e}.gate_proj.weight") for e in range(cfg.num_experts)]
            ups = [get(l, f"mlp.experts.{e}.up_proj.weight") for e in range(cfg.num_experts)]
            downs = [get(l, f"mlp.experts.{e}.down_proj.weight") for e in range(cfg.num_experts)]
            gu = torch.stack([torch.cat([g, u], 0) for g, u in zip(gates, ups)])
            dn = torch.stack(downs)
        hf = {
            "q_proj": get(l, "self_attn.q_proj.weight"),
            "k_proj": get(l, "self_attn.k_proj.weight"),
            "v_proj": get(l, "self_attn.v_proj.weight"),
            "o_proj": get(l, "self_attn.o_proj.weight"),
            "q_norm": get(l, "self_attn.q_norm.weight"),
            "k_norm": get(l, "self_attn.k_norm.weight"),
            "input_layernorm": get(l, "input_layernorm.weight"),
            "post_attention_layernorm": get(l, "post_attention_layernorm.weight"),
            "gate": get(l, "mlp.gate.weight"),
            "gate_up_proj": gu, "down_proj": dn,
        }
        missing = [k for k, v in hf.items() if v is None]
        if missing:
            raise KeyError(f"layer {l}: missing {missing}")
        layers.append(pack_layer(hf, cfg.expert_format))
    return layers


class KVCacheManager:
    """Holds per-layer K/V caches; ``past_key_values`` is flat [K0, V0, K1, V1, ...]
    like the NxDI kv_mgr the reference reads (qwen_with_megakernel.py:410-420).

    Flat caches are [B, kv_heads, max_seq, d].  With cfg.kv_block_len > 0 the
    caches are a block pool [num_blocks, block_len, kv_heads, d] per layer and
    ``block_table`` [B, blocks_per_seq] (int32, shared by all layers) maps
    sequence b's positions t to row t % block_len of block
    block_table[b, t // block_len] -- the paged layout of
    attention_block_tkg.py:199-206.  Blocks are handed out as a seeded random
    permutation, so sequences own scattered blocks."""

    def __init__(self, cfg: Qwen3MoeMKConfig, batch: int, device, seed: int = 0):
        self.block_len = cfg.kv_block_len
        self.block_table = None
        if self.block_len:
            if cfg.max_seq % self.block_len:
                raise ValueError(f"max_seq {cfg.max_seq} must be a multiple of kv_block_len {self.block_len}")
            self.blocks_per_seq = cfg.max_seq // self.block_len
            self.num_blocks = batch * self.blocks_per_seq
            g = torch.Generator().manual_seed(seed)
            perm = torch.randperm(self.num_blocks, generator=g).to(torch.int32)
            self.block_table = perm.reshape(batch, self.blocks_per_seq).contiguous().to(device)
            shape = (self.num_blocks, self.block_len, cfg.num_key_value_heads, cfg.head_dim)
        else:
            self.blocks_per_seq = self.num_blocks = 0
            shape = (batch, cfg.num_key_value_heads, cfg.max_seq, cfg.head_dim)
        self.past_key_values = []
        for _ in range(cfg.num_hidden_layers):
            self.past_key_values.append(torch.zeros(shape, dtype=torch.bfloat16, device=device))
            self.past_key_values.append(torch.zeros(shape, dtype=torch.bfloat16, device=device))

    def k(self, l):
        return self.past_key_values[2 * l]

    def v(self, l):
        return self.past_key_values[2 * l + 1]


_PTR_FIELDS = ("w_qkv", "w_o", "q_norm", "k_norm", "ln_in", "ln_post", "router", "gate_up", "down",
               "k_cache", "v_cache", "gate_up_scales", "down_scales", "b_qkv", "b_o", "sinks",
               "router_bias", "gate_up_bias", "down_bias")


class _LayerStack:
    """Shared by the Qwen3 and GPT-OSS models: a view of a contiguous range of
    the layers, and the routing log (what each layer's router produced)."""

    # A list here (with the routing log enabled) collects route_log(1) after every
    # one-token pass of a token-by-token context encoding, in pass order
    # (synchronises per pass; for tests that route an oracle like the GPU).
    route_log_history: Optional[list] = None

    def decode_plan(self, batch: Optional[int] = None) -> str:
        """The decode path for this batch under the current mode: "persistent",
        "joined_experts" (multi-kernel layers, gate/up and down in one launch) or
        "multi_kernel"."""
        plan = C.c_int32(0)
        L.check(L.load().mkd_qwen3_decode_plan(self._model, batch or self.batch, C.byref(plan)),
                "qwen3_decode_plan")
        return "persistent" if plan.value & 1 else ("joined_experts" if plan.value & 2 else "multi_kernel")

    def joined_attention(self, batch: Optional[int] = None) -> bool:
        """Whether the multi-kernel layers run attention, chunk combine and output
        projection as one launch for this batch under the current mode."""
        plan = C.c_int32(0)
        L.check(L.load().mkd_qwen3_decode_plan(self._model, batch or self.batch, C.byref(plan)),
                "qwen3_decode_plan")
        return bool(plan.value & 4)

    def router_in_attention(self, batch: Optional[int] = None) -> bool:
        """Whether the joined attention launch also runs the residual add, the
        post-attention norm and the router GEMM (no router launch) for this batch."""
        plan = C.c_int32(0)
        L.check(L.load().mkd_qwen3_decode_plan(self._model, batch or self.batch, C.byref(plan)),
                "qwen3_decode_plan")
        return bool(plan.value & 8)

    def layer_kernel_status(self, batch: Optional[int] = None):
        """(persistent layer kernel planned for this batch, an in-launch wait -- a grid
        barrier or the joined expert launch's flags -- timed out).  Synchronises the device."""
        used, timeout = C.c_int32(0), C.c_int32(0)
        rc = L.load().mkd_qwen3_layer_kernel_status(self._model, batch or self.batch, self.ws.data_ptr(),
                                                   self.ws.numel(), C.byref(used), C.byref(timeout))
        L.check(rc, "qwen3_layer_kernel_status")
        return bool(used.value), bool(timeout.value)

    def _struct_for(self, layers):
        """The model struct, or a copy covering layers [lo, hi) only (host pointer
        arrays offset to lo; the persistent path's device table is left out)."""
        if layers is None:
            return self._model
        lo, hi = layers
        n = self._model.num_layers
        if not 0 <= lo < hi <= n:
            raise ValueError(f"layer range {layers} outside [0, {n})")
        sub = L.Qwen3Model()
        C.memmove(C.addressof(sub), C.addressof(self._model), C.sizeof(sub))
        sub.num_layers = hi - lo
        vsz = C.sizeof(L.vp)
        for f in _PTR_FIELDS:
            arr = getattr(self._model, f)
            if arr:
                setattr(sub, f, C.cast(C.cast(arr, C.c_void_p).value + lo * vsz, C.POINTER(L.vp)))
        for f in ("window", "layer_s_max"):
            arr = getattr(self._model, f)
            if arr:
                setattr(sub, f, C.cast(C.cast(arr, C.c_void_p).value + lo * C.sizeof(C.c_int),
                                       C.POINTER(C.c_int)))
        sub.layer_table = None
        if self._model.route_log:
            stride = self._route_log_offsets(self._route_log_batch)[4]
            sub.route_log = self._model.route_log + lo * stride
            sub.route_log_bytes = self._model.route_log_bytes - lo * stride
        return sub

    def _route_log_offsets(self, B):
        offs = (C.c_size_t * 5)()
        L.check(L.load().mkd_qwen3_route_log_layout(self._model, B, offs), "route_log_layout")
        return list(offs)

    def enable_route_log(self, batch: Optional[int] = None):
        """Record, per layer, the expert indices / weights / router logits and the
        post-attention residual of every decode call of up to `batch` tokens (the
        record layout follows the batch of each call).  Capture a step graph after
        this call for the graph to record too."""
        B = batch or self.batch
        n = L.load().mkd_qwen3_route_log_bytes(self._model, B)
        self._route_log = torch.zeros(n, dtype=torch.uint8, device=self.device)
        self._route_log_batch = B
        self._model.route_log = self._route_log.data_ptr()
        self._model.route_log_bytes = n

    def disable_route_log(self):
        self._model.route_log = None
        self._model.route_log_bytes = 0
        self._route_log = None

    def route_log(self, B: int):
        """Per-layer routing records of the last call of B tokens (synchronises):
        a list of dicts idx [B, K] int32, w [B, K] fp32, logits [B, E] fp32,
        r [B, H] bf16 (CPU tensors)."""
        if getattr(self, "_route_log", None) is None:
            raise ValueError("enable_route_log() first")
        o_idx, o_w, o_lg, o_r, stride = self._route_log_offsets(B)
        m = self._model
        K, E, H = m.K, m.E, m.H
        buf = self._route_log.cpu()
        out = []
        for l in range(m.num_layers):
            b = l * stride
            if b + stride > buf.numel():
                break
            out.append({
                "idx": buf[b + o_idx: b + o_idx + 4 * B * K].view(torch.int32).reshape(B, K).clone(),
                "w": buf[b + o_w: b + o_w + 4 * B * K].view(torch.float32).reshape(B, K).clone(),
                "logits": buf[b + o_lg: b + o_lg + 4 * B * E].view(torch.float32).reshape(B, E).clone(),
                "r": buf[b + o_r: b + o_r + 2 * B * H].view(torch.bfloat16).reshape(B, H).clone(),
            })
        return out


class Qwen3MoeMegakernelModel(_LayerStack, nn.Module):
    """Decoder stack + decode-step epilogue on the MI355X library."""

    def __init__(self, cfg: Qwen3MoeMKConfig, layers: List[PackedLayer], batch: int, device,
                 embed: Optional[torch.Tensor] = None, ln_f: Optional[torch.Tensor] = None,
                 lm_head: Optional[torch.Tensor] = None):
        super().__init__()
        self.cfg = cfg
        self.batch = batch
        self.device = torch.device(device)
        self.packed = layers
        self.kv_mgr = KVCacheManager(cfg, batch, device)
        self.embed_tokens = embed                    # [V, H] bf16 or None
        self.ln_f = ln_f                             # [H] bf16 or None
        self.lm_head_packed = packing.pack_out_in(lm_head) if lm_head is not None else None
        d = cfg.head_dim
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))).to(device)
        self._build_struct()
        lib = L.load()
        # device table of the per-layer pointers (persistent decode path)
        self.layer_table = torch.empty(max(lib.mkd_qwen3_layer_table_bytes(self._model), 8),
                                       dtype=torch.uint8, device=device)
        L.check(lib.mkd_qwen3_write_layer_table(self._model, self.layer_table.data_ptr(),
                                                self.layer_table.numel()), "qwen3_write_layer_table")
        self._model.layer_table = self.layer_table.data_ptr()
        self.ws = torch.zeros(max(lib.mkd_qwen3_workspace_bytes(self._model, batch), 256),
                              dtype=torch.uint8, device=device)
        self.lm_ws = torch.empty(max(lib.mkd_lm_head_workspace_bytes(batch, cfg.hidden_size, cfg.vocab_size), 256),
                                 dtype=torch.uint8, device=device)
        self.layers = nn.ModuleList(
            [Qwen3MoeDecoderLayerMK(cfg, i, self) for i in range(cfg.num_hidden_layers)])
        self._graph = None

    # -- ctypes model struct (host arrays of device pointers) --
    def _build_struct(self):
        cfg, Ln = self.cfg, self.cfg.num_hidden_layers
        arr = lambda ts: (L.vp * Ln)(*[t.data_ptr() for t in ts])
        p = self.packed
        self._arrays = {
            "w_qkv": arr([x.w_qkv for x in p]), "w_o": arr([x.w_o for x in p]),
            "q_norm": arr([x.q_norm for x in p]), "k_norm": arr([x.k_norm for x in p]),
            "ln_in": arr([x.ln_in for x in p]), "ln_post": arr([x.ln_post for x in p]),
            "router": arr([x.router for x in p]), "gate_up": arr([x.gate_up for x in p]),
            "down": arr([x.down for x in p]),
            "k_cache": arr([self.kv_mgr.k(l) for l in range(Ln)]),
            "v_cache": arr([self.kv_mgr.v(l) for l in range(Ln)]),
        }
        fmt = EXPERT_FORMATS[cfg.expert_format]
        if fmt:
            if any(x.gate_up_scales is None or x.down_scales is None for x in p):
                raise ValueError(f"expert_format {cfg.expert_format!r} needs layers packed with MX experts")
            self._arrays["gate_up_scales"] = arr([x.gate_up_scales for x in p])
            self._arrays["down_scales"] = arr([x.down_scales for x in p])
        kv = self.kv_mgr
        self._model = L.Qwen3Model(
            num_layers=Ln, H=cfg.hidden_size, nq=cfg.num_attention_heads,
            nkv=cfg.num_key_value_heads, d=cfg.head_dim, E=cfg.num_experts,
            K=cfg.num_experts_per_tok, I=cfg.moe_intermediate_size, S_max=cfg.max_seq,
            eps=cfg.rms_norm_eps, inv_freq=self.inv_freq.data_ptr(), expert_format=fmt,
            block_table=L.ptr(kv.block_table), blocks_per_seq=kv.blocks_per_seq,
            block_len=kv.block_len, num_blocks=kv.num_blocks, **self._arrays)

    def rope_cos_sin(self, position_ids: torch.Tensor):
        """cos/sin [B, d] at position_ids (HF rotary: fp32 angles, halves duplicated)."""
        freqs = position_ids.reshape(-1, 1).float() * self.inv_freq[None, :]
        emb = torch.cat([freqs, freqs], -1)
        return emb.cos(), emb.sin()

    def decode_layers(self, hidden: torch.Tensor, position_ids: torch.Tensor,
                      cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                      layers=None):
        """Run all layers (or the range `layers` = (lo, hi)) in place on hidden [B, H]
        bf16 (the multilayer kernel call)."""
        B = hidden.shape[0]
        if B > self.batch:
            raise ValueError(f"batch {B} exceeds the configured max batch {self.batch}")
        if hidden.dtype != torch.bfloat16 or not hidden.is_contiguous():
            raise ValueError("hidden must be a contiguous bf16 [B, H] tensor")
        pos = position_ids.reshape(-1)
        if pos.dtype != torch.int32:
            raise ValueError("position_ids must be int32")
        rc = L.load().mkd_qwen3_decode_layers(
            self._struct_for(layers), B, hidden.data_ptr(), pos.data_ptr(), L.ptr(cos), L.ptr(sin),
            self.ws.data_ptr(), self.ws.numel(), L.stream_ptr(self.device))
        L.check(rc, "qwen3_decode_layers")
        return hidden

    def step(self, token_ids: torch.Tensor, position_ids: torch.Tensor, hidden: torch.Tensor,
             logits: torch.Tensor, next_tokens: torch.Tensor):
        """Full greedy decode step into caller buffers (no allocation; graph-capturable)."""
        lib = L.load()
        B, H = hidden.shape
        s = L.stream_ptr(self.device)
        L.check(lib.mkd_embed(token_ids.data_ptr(), self.embed_tokens.data_ptr(), hidden.data_ptr(),
                              B, H, self.embed_tokens.shape[0], s), "embed")
        self.decode_layers(hidden, position_ids)
        L.check(lib.mkd_lm_head_greedy(hidden.data_ptr(), self.ln_f.data_ptr(), self.cfg.rms_norm_eps,
                                       self.lm_head_packed.data_ptr(), B, H, self.cfg.vocab_size, H, 2,
                                       logits.data_ptr(), next_tokens.data_ptr(),
                                       self.lm_ws.data_ptr(), self.lm_ws.numel(), s), "lm_head")
        return next_tokens

    def prefill(self, input_ids: torch.Tensor, start_pos: int = 0, seq: int = 0, chunk: int = 4096):
        """Context encoding of one sequence (the reference's CTE layer path,
        qwen_with_megakernel.py:496-526): input_ids [T] fill cache rows start_pos ..
        start_pos + T - 1 of sequence `seq`, in passes of up to `chunk` (<= 4096)
        tokens through all layers (mkd_qwen3_prefill_layers; passes above 128 tokens
        run the experts as LDS-tiled MFMA GEMMs), then the step epilogue on the last
        token: (logits [V] fp32, next id [1] int32)."""
        return _prefill(self, input_ids, start_pos, seq, chunk, self.cfg.hidden_size,
                        self.cfg.hidden_size, 2, lambda pos: (None, None))

    def forward(self, input_ids: torch.Tensor, position_ids: torch.Tensor):
        """Greedy decode step: input_ids [B] -> (logits [B, V] fp32, next ids [B] int32).
        Synchronises and raises RuntimeError when an in-launch wait of the step ran
        out (the step's results are then invalid); `step` is the graph-capturable
        form without that check."""
        B = input_ids.shape[0]
        hidden = torch.empty(B, self.cfg.hidden_size, dtype=torch.bfloat16, device=self.device)
        logits = torch.empty(B, self.cfg.vocab_size, dtype=torch.float32, device=self.device)
        nxt = torch.empty(B, dtype=torch.int32, device=self.device)
        self.step(input_ids.to(torch.int32).contiguous(), position_ids.to(torch.int32).contiguous(),
                  hidden, logits, nxt)
        check_waits(self, B, self.ws)
        return logits, nxt


# Passes of more tokens than this plan no in-launch waits (the joined launches
# and the persistent kernel take at most 4 tokens).
_MAX_WAIT_TOKENS = 4


def check_waits(model, B: int, ws: torch.Tensor, struct=None):
    """Raise RuntimeError when an in-launch wait of the last decode / prefill call
    of B tokens on workspace `ws` ran out of polls (a grid barrier, a flag or a
    data-polled exchange): the kernels then drain but that call's results are
    invalid.  Synchronises the device."""
    used, timeout = C.c_int32(0), C.c_int32(0)
    L.check(L.load().mkd_qwen3_layer_kernel_status(struct or model._model, B, ws.data_ptr(), ws.numel(),
                                                   C.byref(used), C.byref(timeout)),
            "qwen3_layer_kernel_status")
    if timeout.value:
        raise RuntimeError("an in-launch wait of the decode layers timed out: the step's results are invalid")


def prefill_rows(model, hidden: torch.Tensor, start_pos: int, seq: int = 0, layers=None, rope=None):
    """Context encoding of rows already embedded: hidden [T, H] bf16 (contiguous,
    T <= 4096) holds consecutive tokens of sequence `seq` at positions start_pos ..
    start_pos + T - 1 and is run through all layers (or the range `layers` =
    (lo, hi)) in one pass, in place; those layers' cache rows are written.
    `rope(pos)` gives the (cos, sin) tables or (None, None)."""
    T = hidden.shape[0]
    if hidden.dtype != torch.bfloat16 or not hidden.is_contiguous() or hidden.dim() != 2:
        raise ValueError("hidden must be a contiguous bf16 [T, H] tensor")
    if not 1 <= T <= 4096:
        raise ValueError(f"{T} tokens per pass; the library takes 1..4096")
    if not 0 <= seq < model.batch:
        raise ValueError(f"sequence {seq} outside the model's {model.batch} cache slots")
    if start_pos < 0 or start_pos + T > model.cfg.max_seq:
        raise ValueError(f"{T} tokens at {start_pos} do not fit max_seq {model.cfg.max_seq}")
    lib = L.load()
    st = model._struct_for(layers)
    ws = getattr(model, "_prefill_ws", None)
    need = max(lib.mkd_qwen3_workspace_bytes(st, T), 256)
    if ws is None or ws.numel() < need:
        ws = model._prefill_ws = torch.zeros(need, dtype=torch.uint8, device=model.device)
    pos = torch.arange(start_pos, start_pos + T, dtype=torch.int32, device=model.device)
    cos, sin = rope(pos) if rope is not None else (None, None)
    L.check(lib.mkd_qwen3_prefill_layers(st, seq, T, hidden.data_ptr(), pos.data_ptr(), L.ptr(cos),
                                         L.ptr(sin), ws.data_ptr(), ws.numel(),
                                         L.stream_ptr(model.device)), "qwen3_prefill_layers")
    if T <= _MAX_WAIT_TOKENS:
        check_waits(model, T, ws, st)
    return hidden


def _prefill(model, input_ids, start_pos, seq, chunk, H, h_actual, norm_order, rope):
    """Shared prefill loop of the Qwen3 and GPT-OSS models (same C entry point)."""
    if model.embed_tokens is None or model.lm_head_packed is None:
        raise ValueError("prefill needs the embedding table and lm_head")
    if not 0 <= seq < model.batch:
        raise ValueError(f"sequence {seq} outside the model's {model.batch} cache slots")
    ids = input_ids.reshape(-1).to(device=model.device, dtype=torch.int32).contiguous()
    T = ids.numel()
    if T < 1 or start_pos < 0 or start_pos + T > model.cfg.max_seq:
        raise ValueError(f"prompt of {T} tokens at {start_pos} does not fit max_seq {model.cfg.max_seq}")
    chunk = max(1, min(int(chunk), 4096, T))
    lib = L.load()
    ws = getattr(model, "_prefill_ws", None)
    need = max(lib.mkd_qwen3_workspace_bytes(model._model, chunk), 256)
    if ws is None or ws.numel() < need:
        ws = model._prefill_ws = torch.zeros(need, dtype=torch.uint8, device=model.device)
    V = model.cfg.vocab_size
    hidden = torch.empty(chunk, H, dtype=torch.bfloat16, device=model.device)
    s = L.stream_ptr(model.device)
    n = 0
    for c0 in range(0, T, chunk):
        n = min(chunk, T - c0)
        pos = torch.arange(start_pos + c0, start_pos + c0 + n, dtype=torch.int32, device=model.device)
        h = hidden[:n]
        L.check(lib.mkd_embed(ids[c0:].data_ptr(), model.embed_tokens.data_ptr(), h.data_ptr(), n, H,
                              model.embed_tokens.shape[0], s), "embed")
        cos, sin = rope(pos)
        L.check(lib.mkd_qwen3_prefill_layers(model._model, seq, n, h.data_ptr(), pos.data_ptr(),
                                             L.ptr(cos), L.ptr(sin), ws.data_ptr(), ws.numel(), s),
                "qwen3_prefill_layers")
        if n <= _MAX_WAIT_TOKENS:
            check_waits(model, n, ws)
    logits = torch.empty(1, V, dtype=torch.float32, device=model.device)
    nxt = torch.empty(1, dtype=torch.int32, device=model.device)
    L.check(lib.mkd_lm_head_greedy(hidden[n - 1:n].data_ptr(), model.ln_f.data_ptr(), model.cfg.rms_norm_eps,
                                   model.lm_head_packed.data_ptr(), 1, H, V, h_actual, norm_order,
                                   logits.data_ptr(), nxt.data_ptr(), model.lm_ws.data_ptr(),
                                   model.lm_ws.numel(), s), "lm_head")
    return logits[0], nxt


class Qwen3MoeDecoderLayerMK(nn.Module):
    """Decoder-layer boundary of NeuronQwen3MoeDecoderLayerV3 (qwen_with_megakernel.py:422-526)."""

    def __init__(self, cfg: Qwen3MoeMKConfig, layer_idx: int, parent: Qwen3MoeMegakernelModel):
        super().__init__()
        self.layer_idx = layer_idx
        self._num_hidden_layers = cfg.num_hidden_layers
        import weakref
        self._parent_model_ref = weakref.ref(parent)

    @property
    def _parent_model(self):
        return self._parent_model_ref()

    def forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None,
                past_key_value=None, padding_mask=None, kv_mgr=None, idx: int = 0,
                is_for_context_encoding: bool = True, **kwargs):
        parent = self._parent_model
        kv_mgr = kv_mgr if kv_mgr is not None else parent.kv_mgr
        if kv_mgr is not parent.kv_mgr:
            raise ValueError("kv_mgr must be the model's KVCacheManager (its caches are bound to the step)")
        if is_for_context_encoding:
            return self._context_encoding(hidden_states, attention_mask, position_ids, kv_mgr,
                                          kwargs.get("seq_ids"))
        Ln = self._num_hidden_layers
        if self.layer_idx == 0:
            B, S, H = hidden_states.shape
            if S != 1:
                raise NotImplementedError("token generation takes one token per sequence")
            pos = position_ids.reshape(-1).to(torch.int32).contiguous()
            cos, sin = parent.rope_cos_sin(pos)
            y = hidden_states.reshape(B, H).to(torch.bfloat16).contiguous().clone()
            parent.decode_layers(y, pos)
            K_out = [kv_mgr.k(l) for l in range(Ln)]
            V_out = [kv_mgr.v(l) for l in range(Ln)]
            parent._tkg_kv_out = (K_out, V_out)
            return (y.reshape(B, S, H), (K_out[0], V_out[0]), cos[:, None, :], sin[:, None, :], None)
        K_out, V_out = parent._tkg_kv_out
        return (hidden_states, (K_out[self.layer_idx], V_out[self.layer_idx]), None, None, None)

    def _context_encoding(self, hidden_states, attention_mask, position_ids, kv_mgr, seq_ids):
        """CTE through this one layer, as the reference's stock layer path
        (qwen_with_megakernel.py:496-526): hidden_states [B, S, H] -> this layer's
        output for every token, the layer's cache rows of each sequence written.
        Sequence b's tokens are the positions where attention_mask[b] (a [B, S]
        0/1 padding mask, default all ones) is 1 -- one contiguous run at
        consecutive position_ids [B, S]; padded slots pass through unchanged."""
        parent = self._parent_model
        B, S, H = hidden_states.shape
        if position_ids is None:
            raise ValueError("context encoding needs position_ids [B, S]")
        pos = position_ids.reshape(B, S).to(torch.int64).cpu()
        if attention_mask is not None and attention_mask.dim() == 2:
            keep = attention_mask.reshape(B, S).to(torch.bool).cpu()
        elif attention_mask is None:
            keep = torch.ones(B, S, dtype=torch.bool)
        else:
            raise NotImplementedError("context encoding takes a [B, S] padding mask (causal masking is implied)")
        seqs = seq_ids.reshape(-1).tolist() if seq_ids is not None else list(range(B))
        y = hidden_states.to(torch.bfloat16).clone()
        l = self.layer_idx
        for b in range(B):
            cols = keep[b].nonzero().flatten()
            if cols.numel() == 0:
                continue
            c0, c1 = int(cols[0]), int(cols[-1]) + 1
            if cols.numel() != c1 - c0:
                raise NotImplementedError("each sequence's tokens must be one contiguous run")
            p = pos[b, c0:c1]
            if not torch.equal(p, torch.arange(int(p[0]), int(p[0]) + p.numel())):
                raise NotImplementedError("context encoding needs consecutive position_ids")
            rows = y[b, c0:c1].contiguous()
            prefill_rows(parent, rows, int(p[0]), int(seqs[b]), layers=(l, l + 1))
            y[b, c0:c1] = rows
        cos, sin = parent.rope_cos_sin(pos.reshape(-1).to(torch.int32).to(parent.device))
        return (y, (kv_mgr.k(l), kv_mgr.v(l)), cos.reshape(B, S, -1), sin.reshape(B, S, -1), None)


# Alias mirroring the reference module's export (qwen_with_megakernel.py:728).
NeuronQwen3MoeForCausalLM = Qwen3MoeMegakernelModel
