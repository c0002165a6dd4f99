"""Torch CPU restatement of the reference decode path (TEST INFRASTRUCTURE ONLY).

Every function cites the reference file:line it restates.  Reference paths are
relative to the KevGomes1403/nki-moe-megakernel checkout.  All math is fp32 on
the CPU; ``_bf`` marks the places where the reference rounds through bf16.

Two families live here:

* the generic vendored primitives (``rmsnorm_tkg``, ``router_topk``,
  ``moe_tkg``, ``attention_block_tkg``) with the reference operator argument
  meaning, in the reference HBM layouts;
* the Qwen3-MoE fused layer flow (``qwen_*``) that the Qwen megakernel runs,
  with the bf16 rounding points it emulates, in HF weight layouts
  ([out, in] linears, experts gate_up [E, 2I, H], down [E, H, I]).

``emulate_bf16=False`` turns every rounding point off; the result is then the
plain fp32 math, which is what the HF-module pins check.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

F32_MIN = torch.finfo(torch.float32).min


def _bf(x: torch.Tensor, on: bool = True) -> torch.Tensor:
    """Round an fp32 tensor through bf16 (round-to-nearest-even) and back."""
    return x.to(torch.bfloat16).to(torch.float32) if on else x


def stable_topk(x: torch.Tensor, k: int):
    """Top-k along the last dim, descending; equal values keep the lower index first.

    The reference selects with max8 + nc_find_index8 (router_topk.py:626-646),
    which returns values in descending order and the first index holding each
    value.  For distinct values both rules agree; for exact ties this one keeps
    distinct indices (the parity contract excludes near-ties anyway).
    """
    order = torch.sort(-x, dim=-1, stable=True).indices[..., :k]
    return torch.gather(x, -1, order), order


# ---------------------------------------------------------------------------
# a1: rmsnorm_tkg  (nki_kernels/norm/rmsnorm_tkg.py:49-147, math :318-454)
# ---------------------------------------------------------------------------
def rmsnorm_tkg(x: torch.Tensor, gamma: torch.Tensor, eps: float = 1e-6,
                hidden_actual: Optional[int] = None) -> torch.Tensor:
    """fp32 ``(x * gamma) * rsqrt(sum(x^2) / H_actual + eps)``.

    Square + reduce (:369-379), gamma multiply (:413-418), rsqrt with
    ``scale=1/hidden_actual`` and ``bias=eps`` (:432-439), final product
    (:442-447).  ``hidden_actual`` is the true width when x is zero-padded.
    Returns fp32; the caller casts to the io dtype.
    """
    xf = x.float()
    h = hidden_actual if hidden_actual is not None else xf.shape[-1]
    ss = (xf * xf).sum(-1, keepdim=True)
    rinv = torch.rsqrt(ss * (1.0 / h) + eps)
    return (xf * gamma.float().reshape(-1)) * rinv


# ---------------------------------------------------------------------------
# a6: router_topk  (nki_kernels/moe/router_topk.py:69-207, 400-1076, 1772-1858)
# ---------------------------------------------------------------------------
def _act(x: torch.Tensor, act_fn: str) -> torch.Tensor:
    # compute_activation router_topk.py:1772-1858: softmax = exp(x - max) * 1/sum
    if act_fn == "softmax":
        m = x.max(-1, keepdim=True).values
        e = torch.exp(x - m)
        return e * (1.0 / e.sum(-1, keepdim=True))
    if act_fn == "sigmoid":
        return torch.sigmoid(x)
    raise ValueError(act_fn)


def router_topk(x: torch.Tensor, w: torch.Tensor, w_bias: Optional[torch.Tensor],
                act_fn: str, k: int, router_pre_norm: bool = True,
                norm_topk_prob: bool = False):
    """Router logits, top-k expert ids and affinities.

    x [T, H] (io dtype), w [H, E] (router_topk.py:103), bias [1, E] or [E].
    logits = x @ w (+ bias) accumulated in fp32 (:400-493).
    Pipelines (:519-562):
      router_pre_norm=True              -> ACT1 -> topK (-> Norm -> scatter)
      router_pre_norm=False             -> topK -> ACT2 -> scatter
    Returns (router_logits [T,E] fp32, expert_index [T,k] int64,
             expert_affinities [T,E] fp32, topk_affinities [T,k] fp32).
    With (ACT1, topK) and no Norm the stored affinities are the full
    activation (:577-597); otherwise they are the top-k values scattered into
    zeros (:750-1076).
    """
    logits = x.float() @ w.float()
    if w_bias is not None:
        logits = logits + w_bias.float().reshape(1, -1)
    T, E = logits.shape
    if router_pre_norm:
        full = _act(logits, act_fn)
        vals, idx = stable_topk(full, k)
        if norm_topk_prob:
            vals = vals * (1.0 / vals.sum(-1, keepdim=True))          # :786-806
            aff = torch.zeros(T, E).scatter_(1, idx, vals)
        else:
            aff = full
    else:
        top_logits, idx = stable_topk(logits, k)
        vals = _act(top_logits, act_fn)                                # :757-785
        aff = torch.zeros(T, E).scatter_(1, idx, vals)
    return logits, idx, aff, vals


def qwen_router(x_f32: torch.Tensor, w_he: torch.Tensor, k: int, emulate_bf16: bool = True,
                force_idx: Optional[torch.Tensor] = None):
    """Qwen fused router (megakernels/qwen3_moe/moe_fused_nki.py:159-276, 404-418).

    fp32 normed input x [T, H], router weight [H, E] (bf16 values, fp32 math).
    Top-k is taken on the fp32 logits (:241-250), the softmax value at each
    selected index is recovered as exp(l - max) * 1/sum(exp(l - max))
    (:252-268), cast to bf16 (:270-272) and L1-renormalised: fp32 sum of the
    bf16 values, reciprocal, product rounded to bf16 (:404-418).
    Returns (logits fp32 [T,E], idx [T,k], weights [T,k] fp32 holding bf16 values).
    """
    return qwen_router_from_logits(x_f32.float() @ w_he.float(), k, emulate_bf16, force_idx)


def qwen_router_from_logits(logits: torch.Tensor, k: int, emulate_bf16: bool = True,
                            force_idx: Optional[torch.Tensor] = None):
    """The selection and weights of ``qwen_router`` given its fp32 logits [T, E]
    (moe_fused_nki.py:241-272, 404-418).  Returns (logits, idx [T,k], weights [T,k]).

    ``force_idx`` [T, k] replaces the top-k selection by the given experts (in
    that rank order); the weights are then the same formula at those experts.
    Tests use it to compare the continuous math of two flows whose routing a
    near-tie decided differently (the selection itself is checked separately)."""
    logits = logits.float()
    m = logits.max(-1, keepdim=True).values
    inv = 1.0 / torch.exp(logits - m).sum(-1, keepdim=True)
    if force_idx is not None:
        idx = force_idx.long()
        top = torch.gather(logits, -1, idx)
    else:
        top, idx = stable_topk(logits, k)
    vals = _bf(torch.exp(top - m) * inv, emulate_bf16)
    s = vals.sum(-1, keepdim=True)
    w = _bf(vals * (1.0 / s), emulate_bf16)
    return logits, idx, w


# ---------------------------------------------------------------------------
# a7: moe_tkg selective experts  (nki_kernels/moe/moe_tkg.py:56-293,
#     selective_expert_impl.py:84-519, mlp_tkg_gate_up_projection.py:1163-1277,
#     mlp_tkg_down_projection.py:455-638)
# ---------------------------------------------------------------------------
def act_fn_apply(g: torch.Tensor, act: str) -> torch.Tensor:
    if act == "silu":
        return g * torch.sigmoid(g)
    if act == "swish":          # GPT-OSS: g * sigmoid(1.702 g) (HF modeling_gpt_oss.py:82-88)
        return g * torch.sigmoid(1.702 * g)
    if act == "gelu":           # erf form (nl.gelu)
        return torch.nn.functional.gelu(g)
    if act == "gelu_tanh":      # tanh approximation (nl.gelu_apprx_tanh)
        return torch.nn.functional.gelu(g, approximate="tanh")
    raise ValueError(act)


def moe_tkg(hidden: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor,
            affinities: torch.Tensor, index: torch.Tensor,
            gate_up_bias: Optional[torch.Tensor] = None,
            down_bias: Optional[torch.Tensor] = None,
            scaling_mode: str = "none", act: str = "silu",
            gate_clamp_upper: Optional[float] = None, gate_clamp_lower: Optional[float] = None,
            up_clamp_upper: Optional[float] = None, up_clamp_lower: Optional[float] = None,
            emulate_bf16: bool = True) -> torch.Tensor:
    """Selective-expert MoE over the reference layouts; returns fp32 [T, H].

    hidden [T,H]; gate_up [E,H,2,I]; down [E,I,H]; affinities [T,E];
    index [T,K]; gate_up_bias [E,2,I]; down_bias [E,H].
    Per (t, k): g,u = x @ W[e] (+b) in fp32; gate clamps then activation,
    up clamps, h = act(g) * u (:1231-1277) rounded to the io dtype (bf16) as
    the down-projection input; y = h @ Wd[e] (+bd) in fp32; POST_SCALE
    multiplies by affinities[t, e] (selective_expert_impl.py:484-500); fp32
    accumulation over k.
    """
    T, H = hidden.shape
    K = index.shape[1]
    x = hidden.float()
    out = torch.zeros(T, H)
    for t in range(T):
        for j in range(K):
            e = int(index[t, j])
            g = x[t] @ gate_up[e, :, 0, :].float()
            u = x[t] @ gate_up[e, :, 1, :].float()
            if gate_up_bias is not None:
                g = g + gate_up_bias[e, 0].float()
                u = u + gate_up_bias[e, 1].float()
            if gate_clamp_upper is not None:
                g = torch.clamp(g, max=gate_clamp_upper)
            if gate_clamp_lower is not None:
                g = torch.clamp(g, min=gate_clamp_lower)
            g = act_fn_apply(g, act)
            if up_clamp_upper is not None:
                u = torch.clamp(u, max=up_clamp_upper)
            if up_clamp_lower is not None:
                u = torch.clamp(u, min=up_clamp_lower)
            h = _bf(g * u, emulate_bf16)
            y = h @ down[e].float()
            if down_bias is not None:
                y = y + down_bias[e].float()
            if scaling_mode == "post":
                y = y * affinities[t, e].float()
            out[t] += y
    return out


def moe_tkg_fp8_row(hidden, gate_up, down, gate_up_scale, down_scale, affinities, index,
                    gate_up_bias=None, down_bias=None, scaling_mode="none", act="silu",
                    emulate_bf16=True) -> torch.Tensor:
    """FP8 row-quantised experts (moe_tkg.py:119-123, 296-328;
    mlp_tkg_gate_up_projection.py:188-275; mlp_tkg_down_projection.py:418-560):
    e4m3 weights gate_up [E,H,2,I] / down [E,I,H], fp32 scales gate_up_scale
    [E,2,I] / down_scale [E,H].  Each projection is accumulated in fp32 over the
    bf16 activations and the e4m3 weight values, every output column multiplied
    by its scale, then the bias; the rest as moe_tkg.  Returns fp32 [T, H]."""
    T, H = hidden.shape
    K = index.shape[1]
    x = hidden.float()
    out = torch.zeros(T, H)
    for t in range(T):
        for j in range(K):
            e = int(index[t, j])
            g = (x[t] @ gate_up[e, :, 0, :].float()) * gate_up_scale[e, 0].float()
            u = (x[t] @ gate_up[e, :, 1, :].float()) * gate_up_scale[e, 1].float()
            if gate_up_bias is not None:
                g = g + gate_up_bias[e, 0].float()
                u = u + gate_up_bias[e, 1].float()
            h = _bf(act_fn_apply(g, act) * u, emulate_bf16)
            y = (h @ down[e].float()) * down_scale[e].float()
            if down_bias is not None:
                y = y + down_bias[e].float()
            if scaling_mode == "post":
                y = y * affinities[t, e].float()
            out[t] += y
    return out


def mx_qdq(x: torch.Tensor, fmt: str = "e4m3") -> torch.Tensor:
    """Quantise the rows of x to MX (blocks of 32 along the last dim) and back to fp32."""
    from . import mx
    c, s = mx.quantize_mx(x.float().numpy(), fmt)
    return torch.from_numpy(mx.dequantize_mx(c, s, fmt))


def moe_tkg_mx(hidden: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor,
               affinities: torch.Tensor, index: torch.Tensor,
               gate_up_bias: Optional[torch.Tensor] = None,
               down_bias: Optional[torch.Tensor] = None,
               scaling_mode: str = "post", act: str = "silu",
               gate_clamp_upper: Optional[float] = None, gate_clamp_lower: Optional[float] = None,
               up_clamp_upper: Optional[float] = None,
               up_clamp_lower: Optional[float] = None) -> torch.Tensor:
    """MX selective-expert MoE (selective_expert_mx_impl.py:60-531); returns fp32 [T, H].

    gate_up [E, 2I, H] and down [E, H, I] are the DEQUANTISED MX weights (fp32,
    gate rows then up rows).  Activations go through MXFP8 (E4M3) before each
    projection: the hidden rows (selective_expert_mx_impl.py:143-149) and the
    bf16 intermediate act(g)*u (down_projection_mx_shard_H.py:74-79).  Products
    and sums in fp32; down bias added before the affinity scale, which equals
    the reference's aff[T,E] @ b[E,H] term (selective_expert_mx_impl.py:457-497);
    fp32 accumulation over k (the reference accumulates in the io dtype,
    :421-440 -- a difference well inside the MX tolerance).
    """
    T, H = hidden.shape
    K = index.shape[1]
    I = gate_up.shape[1] // 2
    x = mx_qdq(_bf(hidden.float(), True))
    out = torch.zeros(T, H)
    for t in range(T):
        for j in range(K):
            e = int(index[t, j])
            g = gate_up[e, :I].float() @ x[t]
            u = gate_up[e, I:].float() @ x[t]
            if gate_up_bias is not None:
                g = g + gate_up_bias[e, 0].float()
                u = u + gate_up_bias[e, 1].float()
            if gate_clamp_upper is not None:
                g = torch.clamp(g, max=gate_clamp_upper)
            if gate_clamp_lower is not None:
                g = torch.clamp(g, min=gate_clamp_lower)
            g = act_fn_apply(g, act)
            if up_clamp_upper is not None:
                u = torch.clamp(u, max=up_clamp_upper)
            if up_clamp_lower is not None:
                u = torch.clamp(u, min=up_clamp_lower)
            h = mx_qdq(_bf(g * u, True)[None])[0]
            y = down[e].float() @ h
            if down_bias is not None:
                y = y + down_bias[e].float()
            if scaling_mode == "post":
                y = y * affinities[t, e].float()
            out[t] += y
    return out


def qwen_experts(x_bf: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor,
                 idx: torch.Tensor, weights: torch.Tensor, emulate_bf16: bool = True) -> torch.Tensor:
    """Qwen fused experts (moe_fused_nki.py:282-762), HF layouts.

    x_bf [T,H] (bf16 values), gate_up [E, 2I, H] (gate rows then up rows),
    down [E, H, I], idx/weights [T,K].  gate/up accumulate in fp32 and are
    cast to bf16 (:506-510); SiLU of the bf16 gate is rounded to bf16
    (:517-519); gate*up in bf16 (:525-527); down in fp32; scaled by the bf16
    affinity in fp32 and accumulated in fp32 over the K experts (:542-568);
    the sum is cast to bf16 once (:748-759, cast done by the caller).
    Returns fp32 [T, H].
    """
    T, H = x_bf.shape
    I = down.shape[2]
    out = torch.zeros(T, H)
    x = x_bf.float()
    for t in range(T):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            gu = x[t] @ gate_up[e].float().t()
            g = _bf(gu[:I], emulate_bf16)
            u = _bf(gu[I:], emulate_bf16)
            s = _bf(g * torch.sigmoid(g), emulate_bf16)
            h = _bf(s * u, emulate_bf16)
            y = h @ down[e].float().t()
            out[t] += y * weights[t, j].float()
    return out


# ---------------------------------------------------------------------------
# RoPE (HF modeling_qwen3_moe.py:51-80; reference RoPE in bf16 attn_fused_nki.py:426-446)
# ---------------------------------------------------------------------------
def rope_inv_freq(d: int, theta: float) -> torch.Tensor:
    """inv_freq = 1 / theta^(2i/d) in fp32 (HF compute_default_rope_parameters)."""
    return 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))


def rope_cos_sin(pos: torch.Tensor, d: int, theta: float):
    """cos/sin [B, d] fp32 at integer positions, halves duplicated (HF rotary forward)."""
    inv = rope_inv_freq(d, theta)
    freqs = pos.float()[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], -1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], -1)


def rope_apply(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, emulate_bf16: bool = True):
    """x*cos + rotate_half(x)*sin; with emulation each product and the sum are
    rounded to bf16 and cos/sin are bf16 (attn_fused_nki.py:426-446)."""
    c = _bf(cos, emulate_bf16)
    s = _bf(sin, emulate_bf16)
    return _bf(_bf(x * c, emulate_bf16) + _bf(rotate_half(x) * s, emulate_bf16), emulate_bf16)


def head_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Per-head RMSNorm over the last dim: (x * rsqrt(mean(x^2)+eps)) * w in fp32
    (attn_fused_nki.py:400-424 K path, :510-541 Q path)."""
    rinv = torch.rsqrt((x * x).sum(-1, keepdim=True) * (1.0 / x.shape[-1]) + eps)
    return (x * rinv) * w.float()


# ---------------------------------------------------------------------------
# Qwen3 fused attention (megakernels/qwen3_moe/attn_fused_nki.py:50-973),
# generalised from one kv head / B=1 to kv_heads >= 1, B >= 1, per-sequence
# positions.
# ---------------------------------------------------------------------------
@dataclass
class QwenShape:
    H: int = 2048
    q_heads: int = 32
    kv_heads: int = 4
    d: int = 128
    E: int = 128
    K: int = 8
    I: int = 768
    eps: float = 1e-6
    theta: float = 1e6
    vocab: int = 151936


def qwen_attention(h_bf: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor,
                   wo: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor,
                   k_cache: torch.Tensor, v_cache: torch.Tensor, cos: torch.Tensor,
                   sin: torch.Tensor, pos: torch.Tensor, eps: float = 1e-6,
                   emulate_bf16: bool = True, update_cache: bool = True):
    """One decode step of attention for B sequences.

    h_bf [B,H] (normed, bf16 values); wq [nq*d, H], wk/wv [nkv*d, H],
    wo [H, nq*d] (HF [out, in]); k_cache/v_cache [B, nkv, S_max, d] mutated in
    place at row pos[b] when update_cache; cos/sin [B, d] fp32; pos [B] int.

    Rounding flow (emulate_bf16): projections fp32 -> bf16 (:393-398, :494-498);
    q/k RMSNorm fp32 -> bf16 (:426-429, :543-546); RoPE in bf16; scores
    fp32 -> bf16 -> *1/sqrt(d) in bf16 -> fp32 (:611-619, :716-726); prior
    positions t < pos[b] (mask :646-691); max over prior + active; exp, fp32
    sum, reciprocal (:760-800); probabilities cast to bf16 before PV (:808-826);
    prior and active PV each rounded to bf16 then summed in bf16 (:852-865);
    o_proj fp32 -> bf16.  KV rows written after attention (:958-973).
    Returns out [B, H] fp32 (bf16 values when emulating), plus (q, k, v) used.
    """
    B, H = h_bf.shape
    nkv, d = k_cache.shape[1], k_cache.shape[3]
    nq = wq.shape[0] // d
    gqa = nq // nkv
    bf = lambda t: _bf(t, emulate_bf16)
    x = h_bf.float()
    q = bf(x @ wq.float().t()).reshape(B, nq, d)
    k = bf(x @ wk.float().t()).reshape(B, nkv, d)
    v = bf(x @ wv.float().t()).reshape(B, nkv, d)
    q = bf(head_rmsnorm(q, q_norm, eps))
    k = bf(head_rmsnorm(k, k_norm, eps))
    c = cos.float()[:, None, :]
    s = sin.float()[:, None, :]
    q = rope_apply(q, c, s, emulate_bf16)
    k = rope_apply(k, c, s, emulate_bf16)
    scale = 1.0 / math.sqrt(d)
    out = torch.zeros(B, nq, d)
    for b in range(B):
        p = int(pos[b])
        for g in range(nkv):
            Kp = k_cache[b, g, :p].float()            # [p, d]
            Vp = v_cache[b, g, :p].float()
            qh = q[b, g * gqa:(g + 1) * gqa]          # [gqa, d]
            sp = bf(bf(qh @ Kp.t()) * scale)          # [gqa, p]
            sa = bf(bf((qh * k[b, g]).sum(-1)) * scale)  # [gqa]
            m = torch.maximum(sp.max(-1).values if p > 0 else torch.full((gqa,), -1e9), sa)
            ep = torch.exp(sp - m[:, None])
            ea = torch.exp(sa - m)
            inv = 1.0 / (ep.sum(-1) + ea)
            prior = bf(bf(ep * inv[:, None]) @ Vp)
            act = bf(bf(ea * inv)[:, None] * v[b, g][None, :])
            out[b, g * gqa:(g + 1) * gqa] = bf(prior + act)
    o = bf(out.reshape(B, nq * d) @ wo.float().t())
    if update_cache:
        for b in range(B):
            p = int(pos[b])
            k_cache[b, :, p] = k[b].to(k_cache.dtype)
            v_cache[b, :, p] = v[b].to(v_cache.dtype)
    return o, (q, k, v)


# ---------------------------------------------------------------------------
# Qwen3 decoder layer / step (megakernels/qwen3_moe/transformer_qwen.py:218-378)
# ---------------------------------------------------------------------------
@dataclass
class QwenLayer:
    """HF-layout weights of one decoder layer."""
    wq: torch.Tensor        # [nq*d, H]
    wk: torch.Tensor        # [nkv*d, H]
    wv: torch.Tensor        # [nkv*d, H]
    wo: torch.Tensor        # [H, nq*d]
    q_norm: torch.Tensor    # [d]
    k_norm: torch.Tensor    # [d]
    ln_in: torch.Tensor     # [H]
    ln_post: torch.Tensor   # [H]
    router: torch.Tensor    # [E, H]
    gate_up: torch.Tensor   # [E, 2I, H]
    down: torch.Tensor      # [E, H, I]


def qwen_decoder_layer(x_bf: torch.Tensor, lw: QwenLayer, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       pos: torch.Tensor, shape: QwenShape, emulate_bf16: bool = True,
                       mx_experts: bool = False, force_idx: Optional[torch.Tensor] = None):
    """Residual stream in bf16 (transformer_qwen.py:117-127, adds :332, :371).

    Pre-attn RMSNorm is fused in attention as (x*rinv)*gamma -> bf16
    (attn_fused_nki.py:263-316); the post-attn RMSNorm is (x*gamma)*rinv with an
    fp32 copy for the router and a bf16 copy for the experts
    (moe_fused_nki.py:70-153).  mx_experts: lw.gate_up / lw.down hold the
    dequantised MX expert weights and the experts follow moe_tkg_mx (MXFP8
    activations) with the router's top-k weights as POST scales.
    force_idx [B, K]: route to these experts instead of the top-k (weights from
    the router formula at them; see qwen_router_from_logits).
    Returns (x_out, aux dict).
    """
    bf = lambda t: _bf(t, emulate_bf16)
    x = x_bf.float()
    H = x.shape[-1]
    rinv = torch.rsqrt((x * x).sum(-1, keepdim=True) * (1.0 / H) + shape.eps)
    h = bf((x * rinv) * lw.ln_in.float())
    attn, _ = qwen_attention(h, lw.wq, lw.wk, lw.wv, lw.wo, lw.q_norm, lw.k_norm,
                             k_cache, v_cache, cos, sin, pos, shape.eps, emulate_bf16)
    r = bf(x + attn)
    n32 = rmsnorm_tkg(r, lw.ln_post, shape.eps)
    n_bf = bf(n32)
    logits, idx, w = qwen_router(n32, lw.router.float().t(), shape.K, emulate_bf16, force_idx)
    if mx_experts:
        aff = torch.zeros(logits.shape).scatter_(1, idx, w)
        moe = bf(moe_tkg_mx(n_bf, lw.gate_up, lw.down, aff, idx, scaling_mode="post"))
    else:
        moe = bf(qwen_experts(n_bf, lw.gate_up, lw.down, idx, w, emulate_bf16))
    out = bf(r + moe)
    return out, {"h": h, "attn": attn, "r": r, "n32": n32, "logits": logits, "idx": idx,
                 "w": w, "moe": moe}


def final_norm_lm_head(x_bf: torch.Tensor, ln_f: torch.Tensor, lm_head: torch.Tensor,
                       eps: float, emulate_bf16: bool = True):
    """Final RMSNorm -> lm_head -> greedy argmax (qwen_with_megakernel.py:533-594;
    sampling main.py:390-398).  lm_head [V, H]; logits fp32 [B, V]."""
    n = _bf(rmsnorm_tkg(x_bf, ln_f, eps), emulate_bf16)
    logits = n @ lm_head.float().t()
    return logits, torch.argmax(logits, -1)


# ---------------------------------------------------------------------------
# Generic attention_block_tkg (nki_kernels/attention/attention_block_tkg.py:83-583)
# ---------------------------------------------------------------------------
def block_kv_to_flat(cache: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """Block KV cache [num_blocks, block_len, ...] + active_blocks_table [B, n]
    -> flat [B, n * block_len, ...]: position t of sequence b is row
    t % block_len of block table[b, t // block_len]
    (attention_block_tkg.py:199-206, 699-707; entries outside [0, num_blocks)
    give zero rows)."""
    nb, blk = cache.shape[0], cache.shape[1]
    B, n = table.shape
    out = torch.zeros((B, n * blk) + tuple(cache.shape[2:]), dtype=cache.dtype)
    for b in range(B):
        for j in range(n):
            e = int(table[b, j])
            if 0 <= e < nb:
                out[b, j * blk:(j + 1) * blk] = cache[e]
    return out


KV_FP8_MAX = 240.0   # _FP8_E4M3_MAX of the reference's float8_e4m3 (attention_block_tkg.py:1690)


def kv_fp8_quant(x: torch.Tensor, scale: float) -> torch.Tensor:
    """FP8 KV quantisation (attention_block_tkg.py:1694-1737 _quantize_to_fp8):
    e4m3(clip(x * scale, -240, 240)), round to nearest even, as a
    torch.float8_e4m3fn tensor.  The reference's float8_e4m3 reserves the top
    exponent for infinities (largest finite 240); on [-240, 240] its codes and
    values equal float8_e4m3fn's, which torch implements."""
    y = (x.float() * float(scale)).clamp(-KV_FP8_MAX, KV_FP8_MAX)
    return y.to(torch.float8_e4m3fn)


def static_fp8_linear(x: torch.Tensor, W: torch.Tensor, col_w_scale: torch.Tensor,
                      in_scale: float, bias=None) -> torch.Tensor:
    """Static FP8 projection (qkv_tkg.py:289-305, 849-862, 946-986, 1094-1098;
    output_projection_tkg.py:185-200, 549-566): the bf16 input is quantised as
    e4m3(clip(x * (1 / in_scale), +-240)), multiplied by the e4m3 weights
    W [k_in, n_out] in fp32, each column dequantised by its weight scale times
    in_scale (col_w_scale [n_out]), then the bias is added."""
    inv = float(torch.tensor(1.0, dtype=torch.float32) / torch.tensor(in_scale, dtype=torch.float32))
    xq = kv_fp8_quant(x.to(torch.bfloat16), inv).float()
    comb = col_w_scale.float() * torch.tensor(in_scale, dtype=torch.float32)
    y = (xq @ W.float()) * comb.reshape(1, -1)
    if bias is not None:
        y = y + bias.float().reshape(1, -1)
    return y


def attention_block_tkg(X, W_qkv, rmsnorm_X_gamma, rmsnorm_X_eps, bias_qkv,
                        q_norm_w, k_norm_w, qk_eps, cos, sin, K_cache, V_cache,
                        attention_mask, sink, update_cache, kv_cache_update_idx,
                        W_out, bias_out, softmax_scale=None, q_norm_post_w=None,
                        k_norm_post_w=None, qk_post_eps=None, k_scale=None, v_scale=None,
                        K_cache_transposed=False, qkv_static=None, out_static=None):
    """Generic attention block (fp32 math, kv_heads = 1 as in the reference :353).

    X [B, S_tkg, H]; W_qkv [H, d*(nq+2)] packed Q | K | V (:363-384);
    optional pre-attention RMSNorm (:359-366); pre-RoPE per-head RMSNorm
    (:880-900); RoPE with cos/sin [d/2, B, S_tkg] contiguous halves (:905);
    optional post-RoPE per-head RMSNorm with q_norm_post_w / k_norm_post_w [d]
    and qk_post_eps (:906-910, 1093-1138; a None weight skips that norm);
    scores over the cache window [0, S_ctx - S_tkg) followed by the S_tkg
    active tokens, uint8-style 0/1 mask [S_ctx, B, nq, S_tkg]
    (attention_tkg.py:1019-1046, 1892-1893); optional sink logit per head in
    the denominator (attention_tkg.py:3285-3366); KV rows written at
    kv_cache_update_idx[b] + s after attention, uint32 max = skip
    (attention_block_tkg.py:1144-1470); output projection
    attn [B*S, nq*d] @ W_out [nq*d, H] (+ bias).

    K_cache_transposed (:112, :197-202): K_cache is [B, d, S_max].  k_scale and
    v_scale (floats) both given (:749-754): the caches are float8_e4m3fn, the
    new k / v rows are taken in bf16 (their io dtype, :979-1084), quantised by
    kv_fp8_quant, written as such, and the attention uses the stored values
    as they are, the new tokens' own quantised rows included (:1073-1084;
    attention_tkg.py:749-821).  qkv_static = (w_scale [3] for the Q / K / V
    columns, in_scale) and out_static = (w_scale, in_scale): the STATIC FP8
    projections of static_fp8_linear with e4m3 W_qkv / W_out (:94-97, :124-127).
    Returns (out [B*S_tkg, H] fp32, K_cache, V_cache).
    """
    B, S, H = X.shape
    d = V_cache.shape[-1]
    nq = W_qkv.shape[1] // d - 2
    x = X.float().reshape(B * S, H)
    if rmsnorm_X_gamma is not None:
        x = rmsnorm_tkg(x, rmsnorm_X_gamma, rmsnorm_X_eps)
    if qkv_static is not None:
        ws, s_in = qkv_static
        ws = torch.as_tensor(ws, dtype=torch.float32).reshape(-1)
        seg = torch.cat([torch.full((nq * d,), 0), torch.full((d,), 1), torch.full((d,), 2)])
        qkv = static_fp8_linear(x, W_qkv, ws[seg], s_in, bias_qkv)
    else:
        qkv = x @ W_qkv.float()
        if bias_qkv is not None:
            qkv = qkv + bias_qkv.float().reshape(1, -1)
    q = qkv[:, :nq * d].reshape(B, S, nq, d)
    k = qkv[:, nq * d:(nq + 1) * d].reshape(B, S, d)
    v = qkv[:, (nq + 1) * d:].reshape(B, S, d)
    if q_norm_w is not None:
        q = head_rmsnorm(q, q_norm_w.reshape(-1), qk_eps)
        k = head_rmsnorm(k, k_norm_w.reshape(-1), qk_eps)
    if cos is not None:
        c = torch.cat([cos, cos], 0).permute(1, 2, 0).float()   # [B, S, d]
        s_ = torch.cat([sin, sin], 0).permute(1, 2, 0).float()
        q = q * c[:, :, None, :] + rotate_half(q) * s_[:, :, None, :]
        k = k * c + rotate_half(k) * s_
    if q_norm_post_w is not None:
        q = head_rmsnorm(q, q_norm_post_w.reshape(-1), qk_post_eps)
    if k_norm_post_w is not None:
        k = head_rmsnorm(k, k_norm_post_w.reshape(-1), qk_post_eps)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    S_ctx = attention_mask.shape[0]
    # [B, S_max, d] views (a transposed K cache read through its transpose)
    Kc = K_cache.transpose(1, 2) if K_cache_transposed else \
        (K_cache.reshape(K_cache.shape[0], -1, d) if K_cache.dim() == 4 else K_cache)
    Vc = V_cache.reshape(V_cache.shape[0], -1, d) if V_cache.dim() == 4 else V_cache
    kv_quant = k_scale is not None and v_scale is not None
    if kv_quant:   # the new rows as stored
        k = kv_fp8_quant(k.to(torch.bfloat16), k_scale).float()
        v = kv_fp8_quant(v.to(torch.bfloat16), v_scale).float()
    n_prior = S_ctx - S
    out = torch.zeros(B, S, nq, d)
    for b in range(B):
        keys = torch.cat([Kc[b, :n_prior].float(), k[b]], 0)      # [S_ctx, d]
        vals = torch.cat([Vc[b, :n_prior].float(), v[b]], 0)
        for si in range(S):
            sc = (q[b, si] @ keys.t()) * scale                    # [nq, S_ctx]
            valid = attention_mask[:, b, :, si].t().bool()        # [nq, S_ctx]
            sc = torch.where(valid, sc, torch.full_like(sc, -float("inf")))
            m = sc.max(-1, keepdim=True).values
            if sink is not None:
                m = torch.maximum(m, sink.float().reshape(-1, 1)[:nq])
            e = torch.exp(sc - m)
            den = e.sum(-1, keepdim=True)
            if sink is not None:
                den = den + torch.exp(sink.float().reshape(-1, 1)[:nq] - m)
            out[b, si] = (e / den) @ vals
    if update_cache:
        for b in range(B):
            p = int(kv_cache_update_idx.reshape(-1)[b])
            if p == 0xFFFFFFFF or p < 0:
                continue
            for si in range(S):
                Kc[b, p + si] = k[b, si].to(Kc.dtype)
                Vc[b, p + si] = v[b, si].to(Vc.dtype)
    attn = out.reshape(B * S, nq * d)
    if W_out is None:
        return attn, K_cache, V_cache
    if out_static is not None:
        ws, s_in = out_static
        o = static_fp8_linear(attn, W_out, torch.full((W_out.shape[1],), float(ws)), s_in, bias_out)
        return o, K_cache, V_cache
    o = attn @ W_out.float()
    if bias_out is not None:
        o = o + bias_out.float().reshape(1, -1)
    return o, K_cache, V_cache


# ---------------------------------------------------------------------------
# GPT-OSS decoder layer, stock-kernel flow (megakernels/gpt_oss/
# transformer_gpt_oss.py:239-522; HF semantics modeling_gpt_oss.py)
# ---------------------------------------------------------------------------
@dataclass
class GptOssShape:
    H: int = 2880            # actual hidden size (the kernel pads to 3072)
    nq: int = 64
    nkv: int = 8
    d: int = 64
    E: int = 32
    K: int = 4
    I: int = 2880
    eps: float = 1e-5
    alpha: float = 1.702
    limit: float = 7.0


@dataclass
class GptOssLayer:
    """HF-layout weights: q/k/v/o [out, in] with biases, sinks [nq], router [E, H] +
    bias, experts gate_up [E, H, 2I] with gate / up columns INTERLEAVED (HF
    modeling_gpt_oss.py:83), gate_up_b [E, 2I] interleaved, down [E, I, H], down_b [E, H]."""
    wq: torch.Tensor
    bq: torch.Tensor
    wk: torch.Tensor
    bk: torch.Tensor
    wv: torch.Tensor
    bv: torch.Tensor
    wo: torch.Tensor
    bo: torch.Tensor
    sinks: torch.Tensor
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    router_w: torch.Tensor
    router_b: torch.Tensor
    gate_up: torch.Tensor
    gate_up_b: torch.Tensor
    down: torch.Tensor
    down_b: torch.Tensor


def gpt_oss_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Contiguous-halves rotation (HF _apply_rotary_emb): cos/sin [B, d/2] (already
    carrying YaRN's attention scaling) broadcast over heads; x [B, heads, d]."""
    h = x.shape[-1] // 2
    c, s = cos[:, None, :], sin[:, None, :]
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def gpt_oss_decoder_layer(x_bf: torch.Tensor, lw: GptOssLayer, k_cache: torch.Tensor,
                          v_cache: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                          pos: torch.Tensor, window: int, shape: GptOssShape,
                          mx_experts: bool = False, emulate_bf16: bool = True,
                          force_idx: Optional[torch.Tensor] = None):
    """One decode token per sequence; residual in bf16 (transformer_gpt_oss.py:358-519).

    x [B, H] (bf16 values, unpadded H); caches [B, nkv, S, d] bf16, updated in
    place; cos/sin [B, d/2] fp32.  Full layers attend positions [0, pos) plus the
    new token; sliding layers (window W) hold a ring of W rows and attend its
    min(pos, W-1) filled rows plus the new token, the new row going to
    pos % (W-1) (gpt_oss_with_megakernel.py:669-671; masks :67-205).
    RMSNorm is rmsnorm_tkg's (x*g)*rsqrt(mean + eps) (rmsnorm_tkg.py:318-454),
    output bf16; q/k/v rounded to bf16 after RoPE (they are stored as bf16);
    softmax with the sink logit in the denominator (HF eager_attention_forward);
    router: biased logits, top-k, softmax over the top-k (router_topk.py:868-887;
    HF GptOssTopKRouter); experts: gate <= 7, up in [-7, 7], (up + 1) *
    gate * sigmoid(1.702 gate) -> bf16, down + bias, * routing weight, fp32 sum
    over k (HF GptOssExperts).  mx_experts: the expert weights given are
    dequantised MX and the activations go through MXFP8 before each projection
    (as moe_tkg_mx).  emulate_bf16=False drops every bf16 rounding point (the
    plain fp32 math the HF pin checks).  force_idx [B, K]: route to these
    experts (softmax over their logits) instead of the top-k.  Returns
    (x_out [B, H], aux).
    """
    bf = lambda t: _bf(t, emulate_bf16)
    B, H = x_bf.shape
    x = x_bf.float()
    h = bf(rmsnorm_tkg(x, lw.ln_in, shape.eps))
    q = (h @ lw.wq.float().t() + lw.bq.float()).reshape(B, shape.nq, shape.d)
    k = (h @ lw.wk.float().t() + lw.bk.float()).reshape(B, shape.nkv, shape.d)
    v = (h @ lw.wv.float().t() + lw.bv.float()).reshape(B, shape.nkv, shape.d)
    q = bf(gpt_oss_rope(q, cos, sin))
    k = bf(gpt_oss_rope(k, cos, sin))
    v = bf(v)
    gq = shape.nq // shape.nkv
    scale = shape.d ** -0.5
    attn = torch.zeros(B, shape.nq, shape.d)
    for b in range(B):
        p = int(pos[b])
        prior = min(p, window - 1) if window else p
        for g in range(shape.nkv):
            keys = torch.cat([k_cache[b, g, :prior].float(), k[b, g][None]], 0)
            vals = torch.cat([v_cache[b, g, :prior].float(), v[b, g][None]], 0)
            for j in range(gq):
                hq = g * gq + j
                sc = (keys @ q[b, hq]) * scale
                sink = lw.sinks[hq].float()
                m = torch.maximum(sc.max(), sink)
                e = torch.exp(sc - m)
                attn[b, hq] = (e / (e.sum() + torch.exp(sink - m))) @ vals
    for b in range(B):                                   # KV scatter after attention
        p = int(pos[b])
        row = p % (window - 1) if window else p
        k_cache[b, :, row] = k[b].to(k_cache.dtype)
        v_cache[b, :, row] = v[b].to(v_cache.dtype)
    o = bf(bf(attn.reshape(B, -1)) @ lw.wo.float().t() + lw.bo.float())
    r = bf(x + o)
    n = bf(rmsnorm_tkg(r, lw.ln_post, shape.eps))
    logits = n @ lw.router_w.float().t() + lw.router_b.float()
    if force_idx is not None:
        idx = force_idx.long()
        top = torch.gather(logits, -1, idx)
    else:
        top, idx = stable_topk(logits, shape.K)
    w = torch.softmax(top, -1)
    xin = mx_qdq(n) if mx_experts else n
    moe = torch.zeros(B, H)
    for b in range(B):
        for j in range(shape.K):
            e = int(idx[b, j])
            gu = xin[b] @ lw.gate_up[e].float() + lw.gate_up_b[e].float()
            gate = torch.clamp(gu[0::2], max=shape.limit)
            up = torch.clamp(gu[1::2], -shape.limit, shape.limit)
            hh = bf((up + 1) * (gate * torch.sigmoid(gate * shape.alpha)))
            if mx_experts:
                hh = mx_qdq(hh[None])[0]
            y = hh @ lw.down[e].float() + lw.down_b[e].float()
            moe[b] += w[b, j] * y
    out = bf(r + bf(moe))
    return out, {"h": h, "r": r, "n": n, "logits": logits, "idx": idx, "w": w, "moe": moe}
