"""attention_block_tkg operator (reference: nki_kernels/attention/attention_block_tkg.py:83-583)."""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib as L
from . import packing
from .common_types import QuantizationType

U32_MAX = 0xFFFFFFFF


def attention_block_tkg(
    X: torch.Tensor, X_hidden_dim_actual: Optional[int],
    rmsnorm_X_enabled: bool, rmsnorm_X_eps: Optional[float], rmsnorm_X_gamma: Optional[torch.Tensor],
    W_qkv: torch.Tensor, bias_qkv: Optional[torch.Tensor], quantization_type_qkv: QuantizationType,
    weight_dequant_scale_qkv: Optional[torch.Tensor], input_dequant_scale_qkv: Optional[torch.Tensor],
    rmsnorm_QK_pre_rope_enabled: bool, rmsnorm_QK_pre_rope_eps: float,
    rmsnorm_QK_pre_rope_W_Q: Optional[torch.Tensor], rmsnorm_QK_pre_rope_W_K: Optional[torch.Tensor],
    cos: Optional[torch.Tensor], sin: Optional[torch.Tensor], rope_contiguous_layout: bool,
    rmsnorm_QK_post_rope_enabled: bool, rmsnorm_QK_post_rope_eps: float,
    rmsnorm_QK_post_rope_W_Q: Optional[torch.Tensor], rmsnorm_QK_post_rope_W_K: Optional[torch.Tensor],
    K_cache_transposed: bool, active_blocks_table: Optional[torch.Tensor],
    K_cache: torch.Tensor, V_cache: torch.Tensor, attention_mask: torch.Tensor,
    sink: Optional[torch.Tensor], update_cache: bool, kv_cache_update_idx: Optional[torch.Tensor],
    W_out: Optional[torch.Tensor], bias_out: Optional[torch.Tensor],
    quantization_type_out: QuantizationType, weight_dequant_scale_out: Optional[torch.Tensor],
    input_dequant_scale_out: Optional[torch.Tensor], transposed_out: bool, out_in_sb: bool,
    softmax_scale: Optional[float] = None, enable_fa_s_prior_tiling: bool = True,
    k_scale: Optional[torch.Tensor] = None, v_scale: Optional[torch.Tensor] = None,
    sbm=None, skip_attention: bool = False, KVDP: int = 1, KVDP_replica_group=None,
):
    """Fused decode attention block; returns (out, K_cache, V_cache).

    Shapes follow the reference docstring (attention_block_tkg.py:140-289):
    X [B, S_tkg, H]; W_qkv [H, d*(q_heads + 2*kv_heads)] packed Q | K | V;
    cos/sin [d/2, B, S_tkg]; K_cache/V_cache [B, S_max, d] (one kv head, as in
    the reference) or [B, kv_heads, S_max, d] (this build's GQA
    generalisation); attention_mask [S_ctx, B, q_heads, S_tkg] with the active
    token in slot S_ctx - 1; kv_cache_update_idx [B, 1] (uint32 max = skip);
    W_out [q_heads*d, H].  out is [B*S_tkg, H] (or [B, q_heads, d, S_tkg]
    without W_out).  The caches are updated in place.

    Block (paged) KV cache (attention_block_tkg.py:199-206, 699-707,
    1473-1685): with active_blocks_table [B, num_active_blocks], K_cache /
    V_cache are [num_blocks, block_len, d] (or [num_blocks, block_len,
    kv_heads, d]); S_ctx = num_active_blocks * block_len, position t of
    sequence b is row t % block_len of block table[b, t // block_len], the
    active token is mask slot S_ctx - 1, and kv_cache_update_idx holds global
    rows block * block_len + row (uint32 max = skip).

    S_tkg <= 8 new tokens per sequence (attention_block_tkg.py:151): the window
    of sequence b is its first S_ctx - S_tkg cache positions followed by its
    S_tkg new tokens (mask slot S_ctx - S_tkg + i = new token i; the active keys
    close the window as in attention_tkg.py), and token s is written at
    kv_cache_update_idx[b] + s (attention_block_tkg.py:1365-1470; a global row of
    a block cache).  Pre- and post-RoPE per-head Q/K RMSNorm (attention_block_tkg.py:
    895-910; absent weights are ones).

    K_cache_transposed (attention_block_tkg.py:112, :197-202): the flat K cache
    is [B, d, S_max] (or [B, kv_heads, d, S_max]); V keeps [B, S_max, d]; not
    with a block table (ValueError, as the reference).

    FP8 KV cache (k_scale and v_scale both given, attention_block_tkg.py:133-134,
    :213-218, :749-754): K_cache / V_cache are float8 e4m3 (torch.float8_e4m3fn,
    or uint8 tensors of the codes); each scale is one value ((1, 1) or (PMAX, 1)
    replicated: element 0 is read, on the device); the new rows are stored as
    e4m3(clip(k * k_scale, +-240)) (_quantize_to_fp8, :1694-1737) and the
    attention uses the stored values as they are, the new tokens' own rows
    included -- the caller folds any dequantisation into softmax_scale / W_out.

    Static FP8 projections (quantization_type_qkv / _out = STATIC, :94-97, :124-127,
    :179-183, :225-229): W_qkv / W_out are float8 e4m3 ([H, I] / [q_heads*d, H]);
    the (normalised) input is quantised as e4m3(clip(x / input_scale, +-240)) and
    the product is dequantised by weight_scale * input_scale -- per Q / K / V
    segment for the QKV projection (weight_dequant_scale_qkv [1, 3] or [PMAX, 3],
    qkv_tkg.py:289-305, 946-986), one scale for the output projection
    (output_projection_tkg.py:185-200, 549-566) -- then the bias is added.

    ROW / MX projection quantisation (not offered by the reference's
    attention_block_tkg) and the remaining reference options raise
    NotImplementedError.  enable_fa_s_prior_tiling is a scheduling hint (the GPU
    path always tiles the KV length).
    """
    if KVDP != 1:
        raise NotImplementedError("KV data parallelism spans several devices; one GPU only")
    if K_cache_transposed and active_blocks_table is not None:
        raise ValueError("K_cache_transposed must be False for block KV cache")
    if transposed_out or out_in_sb or sbm is not None:
        raise NotImplementedError("transposed/SBUF outputs have no GPU equivalent")
    if skip_attention:
        raise NotImplementedError("skip_attention is a test hook of the reference")
    q_static = quantization_type_qkv == QuantizationType.STATIC
    o_static = quantization_type_out == QuantizationType.STATIC
    for nm, qt in (("quantization_type_qkv", quantization_type_qkv),
                   ("quantization_type_out", quantization_type_out)):
        if qt not in (None, QuantizationType.NONE, QuantizationType.STATIC):
            raise NotImplementedError(f"{nm} must be NONE or STATIC (attention_block_tkg.py:179, 225), got {qt}")
    if q_static and (weight_dequant_scale_qkv is None or input_dequant_scale_qkv is None):
        raise ValueError("STATIC QKV quantization needs weight_dequant_scale_qkv and input_dequant_scale_qkv")
    if o_static and (W_out is None or weight_dequant_scale_out is None or input_dequant_scale_out is None):
        raise ValueError("STATIC output quantization needs W_out, weight_dequant_scale_out and input_dequant_scale_out")
    # KV quantisation only when both scales are given (attention_block_tkg.py:749-754)
    kv_quant = k_scale is not None and v_scale is not None
    if not rope_contiguous_layout and cos is not None:
        raise NotImplementedError("interleaved RoPE layout is not supported")
    L.require_gpu(X, W_qkv, K_cache, V_cache, attention_mask)
    B, S_tkg, H = X.shape
    if not 1 <= S_tkg <= 8:
        raise ValueError(f"S_tkg must be in [1, 8] (attention_block_tkg.py:151), got {S_tkg}")
    if B * S_tkg > 128:
        raise ValueError(f"B * S_tkg = {B * S_tkg} must be <= 128")
    d = V_cache.shape[-1]
    if d % 2:
        raise ValueError(f"d_head must be even, got {d}")
    # a transposed K cache is compared in V's layout
    k_shape = tuple(K_cache.shape[:-2]) + (K_cache.shape[-1], K_cache.shape[-2]) \
        if K_cache_transposed else tuple(K_cache.shape)
    if K_cache_transposed and K_cache.dim() < 3:
        raise ValueError(f"transposed K_cache must be [B, d, S_max], got {tuple(K_cache.shape)}")
    if k_shape != tuple(V_cache.shape):
        raise ValueError(f"KV cache shape mismatch: K={tuple(K_cache.shape)} vs V={tuple(V_cache.shape)}"
                         + (" (K transposed)" if K_cache_transposed else ""))
    block = active_blocks_table is not None
    if block:
        if K_cache.dim() == 3:
            nkv = 1
        elif K_cache.dim() == 4:
            nkv = K_cache.shape[2]
        else:
            raise ValueError(f"block K_cache must be [num_blocks, block_len, (kv_heads,) d], got {tuple(K_cache.shape)}")
        num_blocks, blk_len = K_cache.shape[0], K_cache.shape[1]
        if active_blocks_table.dim() != 2 or active_blocks_table.shape[0] != B:
            raise ValueError(f"active_blocks_table must be [B={B}, num_active_blocks], got {tuple(active_blocks_table.shape)}")
        n_active = active_blocks_table.shape[1]
        S_max = n_active * blk_len
    else:   # V_cache [B, S_max, d] or [B, kv_heads, S_max, d] (K matches it, maybe transposed)
        if V_cache.dim() == 3:
            nkv = 1
            S_max = V_cache.shape[1]
        elif V_cache.dim() == 4:
            nkv = V_cache.shape[1]
            S_max = V_cache.shape[2]
        else:
            raise ValueError(f"K_cache must be 3-D or 4-D, got {tuple(K_cache.shape)}")
        if K_cache.shape[0] != B:
            raise ValueError(f"V_cache batch mismatch: expected {B}, got {K_cache.shape[0]}")
    I = W_qkv.shape[1]
    if I % d:
        raise ValueError(f"QKV weights must be packed as (q_heads + 2) * d_head, got I={I}, d_head={d}")
    nq = I // d - 2 * nkv
    S_ctx = attention_mask.shape[0]
    if block and S_ctx != S_max:
        raise ValueError(f"block KV: attention_mask covers S_ctx={S_ctx}, the table covers {S_max}")
    if tuple(attention_mask.shape) != (S_ctx, B, nq, S_tkg):
        raise ValueError(f"attention_mask shape mismatch: expected {(S_ctx, B, nq, S_tkg)}, got {tuple(attention_mask.shape)}")
    if S_ctx < S_tkg or S_ctx - S_tkg > S_max:
        raise ValueError(f"mask window S_ctx={S_ctx} must hold the {S_tkg} new tokens after at most "
                         f"{S_max} cache positions")
    if rmsnorm_X_enabled and rmsnorm_X_gamma is not None and tuple(rmsnorm_X_gamma.shape) not in ((1, H), (H,)):
        raise ValueError(f"rmsnorm_X_gamma must be (1, {H}), got {tuple(rmsnorm_X_gamma.shape)}")
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must be given together")
    if cos is not None and tuple(cos.shape) != (d // 2, B, S_tkg):
        raise ValueError(f"cos shape mismatch: expected ({d // 2}, {B}, {S_tkg}), got {tuple(cos.shape)}")
    if update_cache and kv_cache_update_idx is None:
        raise ValueError("update_cache=True needs kv_cache_update_idx")
    if X.dtype != torch.bfloat16:
        raise ValueError("X must be bfloat16")
    fp8_types = (torch.float8_e4m3fn, torch.uint8)
    if kv_quant:
        if K_cache.dtype not in fp8_types or V_cache.dtype not in fp8_types:
            raise ValueError(f"KV quantization requires float8_e4m3 K_cache / V_cache, got "
                             f"{K_cache.dtype} / {V_cache.dtype}")
        for nm, sc in (("k_scale", k_scale), ("v_scale", v_scale)):
            if sc.numel() < 1 or sc.dim() != 2 or sc.shape[1] != 1:
                raise ValueError(f"{nm} must be (1, 1) or (PMAX, 1), got {tuple(sc.shape)}")
            if sc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
                raise ValueError(f"{nm} dtype must be float32 / float16 / bfloat16, got {sc.dtype}")
    elif K_cache.dtype != torch.bfloat16 or V_cache.dtype != torch.bfloat16:
        raise ValueError("the KV caches must be bfloat16 (float8_e4m3 needs k_scale and v_scale)")

    dev = X.device
    wqkv = packing.packed_cached(W_qkv, packing.pack_fp8_in_out if q_static else packing.pack_in_out)
    wout = packing.packed_cached(W_out, packing.pack_fp8_in_out if o_static else packing.pack_in_out) \
        if W_out is not None else None

    def scale_row(t, n, nm):   # row 0 of a [1, n] / [PMAX, n] scale tensor, fp32 on the device
        if t.dim() != 2 or t.shape[1] != n:
            raise ValueError(f"{nm} must be [1, {n}] or [PMAX, {n}], got {tuple(t.shape)}")
        return t[0].float().contiguous()
    wsq = scale_row(weight_dequant_scale_qkv, 3, "weight_dequant_scale_qkv") if q_static else None
    isq = scale_row(input_dequant_scale_qkv, 1, "input_dequant_scale_qkv") if q_static else None
    wso = scale_row(weight_dequant_scale_out, 1, "weight_dequant_scale_out") if o_static else None
    iso = scale_row(input_dequant_scale_out, 1, "input_dequant_scale_out") if o_static else None
    H_out = W_out.shape[1] if W_out is not None else 0
    x = X.reshape(B * S_tkg, H).contiguous()
    gamma = rmsnorm_X_gamma.reshape(-1).to(torch.bfloat16).contiguous() \
        if (rmsnorm_X_enabled and rmsnorm_X_gamma is not None) else None
    qn = kn = None
    if rmsnorm_QK_pre_rope_enabled:
        qn = rmsnorm_QK_pre_rope_W_Q.reshape(-1).to(torch.bfloat16).contiguous() \
            if rmsnorm_QK_pre_rope_W_Q is not None else torch.ones(d, dtype=torch.bfloat16, device=dev)
        kn = rmsnorm_QK_pre_rope_W_K.reshape(-1).to(torch.bfloat16).contiguous() \
            if rmsnorm_QK_pre_rope_W_K is not None else torch.ones(d, dtype=torch.bfloat16, device=dev)
    qp = kp = None
    if rmsnorm_QK_post_rope_enabled:   # after RoPE (attention_block_tkg.py:906-910)
        qp = rmsnorm_QK_post_rope_W_Q.reshape(-1).to(torch.bfloat16).contiguous() \
            if rmsnorm_QK_post_rope_W_Q is not None else torch.ones(d, dtype=torch.bfloat16, device=dev)
        kp = rmsnorm_QK_post_rope_W_K.reshape(-1).to(torch.bfloat16).contiguous() \
            if rmsnorm_QK_post_rope_W_K is not None else torch.ones(d, dtype=torch.bfloat16, device=dev)
    cos_f = sin_f = None
    if cos is not None:
        # [d/2, B, S_tkg] -> [B * S_tkg, d] with the halves duplicated (row b * S_tkg + s)
        cos_f = torch.cat([cos, cos], 0).permute(1, 2, 0).reshape(B * S_tkg, d).float().contiguous()
        sin_f = torch.cat([sin, sin], 0).permute(1, 2, 0).reshape(B * S_tkg, d).float().contiguous()
    # [S_ctx, B, nq, S_tkg] 0/1 (with S_tkg = 1 the kernel reads it as [S_ctx, B, nq])
    mask_u8 = (attention_mask != 0).to(torch.uint8).contiguous()
    n_prior = torch.full((B,), S_ctx - S_tkg, dtype=torch.int32, device=dev)
    wpos = None
    if update_cache:
        idx = kv_cache_update_idx.reshape(-1).to(torch.int64)
        wpos = torch.where((idx == U32_MAX) | (idx < 0) | (idx > 0x7FFFFFFF),
                           torch.full_like(idx, -1), idx).to(torch.int32).contiguous()
    table = None
    if block:
        t64 = active_blocks_table.to(torch.int64)
        table = torch.where((t64 < 0) | (t64 >= num_blocks), torch.full_like(t64, -1), t64) \
            .to(torch.int32).contiguous()
    sink_f = sink.reshape(-1).float().contiguous() if sink is not None else None
    ks = vs = None
    if kv_quant:   # element 0 of each scale, as fp32 on the device (no host round trip)
        ks = k_scale.reshape(-1)[:1].float().contiguous()
        vs = v_scale.reshape(-1)[:1].float().contiguous()
    bqkv = bias_qkv.reshape(-1).to(torch.bfloat16).contiguous() if bias_qkv is not None else None
    bout = bias_out.reshape(-1).to(torch.bfloat16).contiguous() if bias_out is not None else None
    out = torch.empty(B * S_tkg, H_out if W_out is not None else nq * d, dtype=torch.bfloat16, device=dev)
    scale = float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(d)
    args = L.AttentionArgs(
        X=x.data_ptr(), rmsnorm_gamma=L.ptr(gamma),
        rmsnorm_eps=float(rmsnorm_X_eps if rmsnorm_X_eps is not None else 1e-3), rmsnorm_order=0,
        w_qkv_packed=wqkv.data_ptr(), bias_qkv=L.ptr(bqkv), q_norm=L.ptr(qn), k_norm=L.ptr(kn),
        qk_eps=float(rmsnorm_QK_pre_rope_eps), cos=L.ptr(cos_f), sin=L.ptr(sin_f),
        k_cache=K_cache.data_ptr(), v_cache=V_cache.data_ptr(), n_prior=n_prior.data_ptr(),
        mask=mask_u8.data_ptr(), mask_s_ctx=S_ctx, sink=L.ptr(sink_f), softmax_scale=scale,
        update_cache=int(bool(update_cache)), kv_cache_update_idx=L.ptr(wpos),
        w_out_packed=L.ptr(wout), bias_out=L.ptr(bout), residual=None, out=out.data_ptr(),
        B=B, H=H, H_out=H_out, nq=nq, nkv=nkv, d=d, S_max=S_max, round_qwen=0,
        active_blocks_table=L.ptr(table), blocks_per_seq=table.shape[1] if block else 0,
        block_len=blk_len if block else 0, num_blocks=num_blocks if block else 0, s_tkg=S_tkg,
        q_norm_post=L.ptr(qp), k_norm_post=L.ptr(kp),
        qk_post_eps=float(rmsnorm_QK_post_rope_eps) if rmsnorm_QK_post_rope_enabled else 0.0,
        kv_format=(L.KV_FP8 if kv_quant else 0) | (L.KV_K_TRANSPOSED if K_cache_transposed else 0),
        k_scale=L.ptr(ks), v_scale=L.ptr(vs),
        quant_qkv=1 if q_static else 0, quant_out=1 if o_static else 0,
        w_scale_qkv=L.ptr(wsq), in_scale_qkv=L.ptr(isq), w_scale_out=L.ptr(wso), in_scale_out=L.ptr(iso))
    lib = L.load()
    ws = torch.zeros(max(lib.mkd_attention_workspace_bytes_tkg(B, S_tkg, H, nq, nkv, d, S_max), 256),
                     dtype=torch.uint8, device=dev)
    rc = lib.mkd_attention_block_tkg(args, ws.data_ptr(), ws.numel(), L.stream_ptr(dev))
    L.check(rc, "attention_block_tkg")
    if W_out is None:   # [B, q_heads, d_head, S_tkg]
        out = out.reshape(B, S_tkg, nq, d).permute(0, 2, 3, 1).contiguous()
    return out, K_cache, V_cache
