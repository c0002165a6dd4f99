"""MX (OCP Microscaling v1.0) expert weights: layouts, quantisation, moe_tkg dispatch.

Reference: the MXFP4 / MXFP8 selective-expert path
(nki_kernels/moe/selective_expert_mx_impl.py:60-531,
down_projection_mx_shard_H.py:138-211) and the weight layouts documented at
moe_tkg.py:105-123.  The reference stores four 8-bit (or four 4-bit) elements
per "x4" item; here an x4 item is a trailing dimension of 4 bytes (E4M3) or
2 bytes (E2M1, two elements per byte, low nibble first):

    gate_up codes   [E, 128, 2, H/512, I, 4|2]   element (e, g, i, h) with
                    h = t*512 + 4*p + j at [e, p, g, t, i, j]
    gate_up scales  [E, 16, 2, H/512, I]          block h//32 = t*16 + p//8
    down codes      [E, I_p, ceil(I/512), H, 4|2] element (e, h, i) with
                    i = t*512 + 4*p + j at [e, p, t, h, j]   (I_p = I/4 if
                    I <= 512 else 128; positions past I are zero padding)
    down scales     [E, I_p/8, ceil(I/512), H]
    gate_up bias    [E, I_p, 2, ceil(I/512), 4]   (e, g, i) at [e, p, g, t, j]

Scale bytes are E8M0 (2^(byte-127)), one per 32 consecutive elements along
the contraction.  Activations are quantised to MXFP8 (E4M3) on the GPU before
each projection, as the reference does with nisa.quantize_mx
(selective_expert_mx_impl.py:143-149, down_projection_mx_shard_H.py:74-79).
The element dtype decides the format: torch.float8_e4m3fn (or uint8 with a
trailing 4) is MXFP8, torch.float4_e2m1fn_x2 (or uint8 with a trailing 2)
is MXFP4.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib as L
from . import packing
from .common_types import ActFnType, ExpertAffinityScaleMode

E4M3, E2M1 = 1, 2          # MKD_MX_E4M3 / MKD_MX_E2M1
_F4 = getattr(torch, "float4_e2m1fn_x2", None)
_F8 = getattr(torch, "float8_e4m3fn", None)
_E8 = getattr(torch, "float8_e8m0fnu", None)


def mx_format(w: torch.Tensor) -> int:
    """MX element format of a reference-layout code tensor (0 if not MX)."""
    if _F8 is not None and w.dtype == _F8:
        return E4M3
    if _F4 is not None and w.dtype == _F4:
        return E2M1
    if w.dtype == torch.uint8 and w.dim() in (5, 6) and w.shape[-1] in (2, 4):
        return E4M3 if w.shape[-1] == 4 else E2M1
    return 0


def is_mx_weight(w: torch.Tensor) -> bool:
    return mx_format(w) != 0


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def kpad(k: int) -> int:
    """Contraction padding of the packed MX layout (the library's mx_kpad)."""
    p = (k + 127) // 128 * 128
    for kw in (512, 384, 256, 128, 1024, 768, 1536, 2048):
        if p % kw == 0 and p // kw <= 8:
            return p
    return (k + 511) // 512 * 512


# ---------------------------------------------------------------- quantisation
def quantize_mx(x: torch.Tensor, fmt: int = E4M3, k_pad: Optional[int] = None):
    """Quantise the rows of a 2-D bf16/fp32 device tensor along its last dim.

    Returns (codes uint8 [rows, k_pad] (E4M3) or [rows, k_pad/2] (E2M1),
    scales uint8 [rows, k_pad/32]); k_pad defaults to k rounded up to 128.
    """
    L.require_gpu(x)
    if x.dim() != 2:
        raise ValueError(f"quantize_mx expects a 2-D tensor, got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    x = x.contiguous()
    rows, k = x.shape
    k_pad = k_pad or (k + 127) // 128 * 128
    codes = torch.empty(rows, k_pad if fmt == E4M3 else k_pad // 2, dtype=torch.uint8, device=x.device)
    scales = torch.empty(rows, k_pad // 32, dtype=torch.uint8, device=x.device)
    rc = L.load().mkd_quantize_mx(x.data_ptr(), L.DT_F32 if x.dtype == torch.float32 else L.DT_BF16,
                                  rows, k, k, fmt, codes.data_ptr(), scales.data_ptr(), k_pad,
                                  L.stream_ptr(x.device))
    L.check(rc, "quantize_mx")
    return codes, scales


# ---------------------------------------------------------------- layouts
def gate_up_to_logical(codes: torch.Tensor, scales: torch.Tensor):
    """Reference gate/up layout -> row-major codes [E, 2I, H (or H/2)], scales [E, 2I, H/32]."""
    c = _u8(codes)
    E, P, two, T, I, X = c.shape
    if P != 128 or two != 2:
        raise ValueError(f"gate_up codes {tuple(c.shape)} are not [E, 128, 2, H/512, I, x4]")
    lc = c.permute(0, 2, 4, 3, 1, 5).reshape(E, 2 * I, T * P * X)
    s = _u8(scales)
    if tuple(s.shape) != (E, 16, 2, T, I):
        raise ValueError(f"gate_up scales {tuple(s.shape)} != {(E, 16, 2, T, I)}")
    ls = s.permute(0, 2, 4, 3, 1).reshape(E, 2 * I, T * 16)
    return lc.contiguous(), ls.contiguous()


def down_to_logical(codes: torch.Tensor, scales: torch.Tensor, I: int):
    """Reference down layout -> row-major codes [E, H, I (or I/2)], scales [E, H, I/32]."""
    c = _u8(codes)
    E, Ip, T, H, X = c.shape
    lc = c.permute(0, 3, 2, 1, 4).reshape(E, H, T * Ip * X)[:, :, : I * X // 4]
    s = _u8(scales)
    if tuple(s.shape) != (E, Ip // 8, T, H):
        raise ValueError(f"down scales {tuple(s.shape)} != {(E, Ip // 8, T, H)}")
    ls = s.permute(0, 3, 2, 1).reshape(E, H, T * Ip // 8)[:, :, : I // 32]
    return lc.contiguous(), ls.contiguous()


def gate_up_bias_to_logical(b: torch.Tensor, I: int) -> torch.Tensor:
    """Reference MX gate/up bias [E, I_p, 2, ceil(I/512), 4] -> [E, 2, I]."""
    E, Ip, two, T, four = b.shape
    return b.permute(0, 2, 3, 1, 4).reshape(E, 2, T * Ip * four)[:, :, :I].contiguous()


def logical_to_gate_up(codes: torch.Tensor, scales: torch.Tensor, fmt: int):
    """Row-major codes [E, 2I, H(/2)] + scales [E, 2I, H/32] -> reference layout."""
    E, N2, Hb = codes.shape
    I = N2 // 2
    X = 4 if fmt == E4M3 else 2
    H = Hb if fmt == E4M3 else 2 * Hb
    if H % 512:
        raise ValueError(f"MX gate/up needs H % 512 == 0 (reference layout), got H={H}")
    T = H // 512
    c = codes.reshape(E, 2, I, T, 128, X).permute(0, 4, 1, 3, 2, 5).contiguous()
    s = scales.reshape(E, 2, I, T, 16).permute(0, 4, 1, 3, 2).contiguous()
    return c, s


def logical_to_down(codes: torch.Tensor, scales: torch.Tensor, fmt: int, I: int):
    """Row-major codes [E, H, I(/2)] + scales [E, H, I/32] -> reference layout."""
    E, H, _ = codes.shape
    X = 4 if fmt == E4M3 else 2
    Ip = I // 4 if I <= 512 else 128
    T = (I + 511) // 512
    n = T * Ip * X
    ib = I * X // 4                                   # code bytes of one row
    c = torch.zeros(E, H, n, dtype=torch.uint8, device=codes.device)
    c[:, :, :ib] = codes[:, :, :ib]
    c = c.reshape(E, H, T, Ip, X).permute(0, 3, 2, 1, 4).contiguous()
    s = torch.zeros(E, H, T * Ip // 8, dtype=torch.uint8, device=codes.device)
    s[:, :, : I // 32] = scales[:, :, : I // 32]
    s = s.reshape(E, H, T, Ip // 8).permute(0, 3, 2, 1).contiguous()
    return c, s


def quantize_experts_mx(gate_up: torch.Tensor, down: torch.Tensor, fmt: int = E4M3):
    """bf16 expert weights (reference bf16 layouts [E, H, 2, I] and [E, I, H]) ->
    MX weights in the reference MX layouts: (gu_codes, gu_scales, dn_codes, dn_scales)."""
    E, H, two, I = gate_up.shape
    rows = gate_up.permute(0, 2, 3, 1).reshape(E * 2 * I, H)          # [E, 2, I, H]
    gc, gs = quantize_mx(rows, fmt, H)
    gc, gs = logical_to_gate_up(gc.reshape(E, 2 * I, -1), gs.reshape(E, 2 * I, -1), fmt)
    drows = down.permute(0, 2, 1).reshape(E * H, I)                    # [E, H, I]
    dc, ds = quantize_mx(drows, fmt, (I + 127) // 128 * 128)
    dc, ds = logical_to_down(dc.reshape(E, H, -1), ds.reshape(E, H, -1), fmt, I)
    return gc, gs, dc, ds


# ---------------------------------------------------------------- packing
def pack_mx(codes: torch.Tensor, scales: torch.Tensor, fmt: int, k: int, interleave_half: int = 0):
    """Row-major [G, N, k(/2)] codes + [G, N, k/32] scales -> (packed codes, packed scales)."""
    L.require_gpu(codes, scales)
    G, N, _ = codes.shape
    lib = L.load()
    dst = torch.empty(lib.mkd_packed_mx_bytes(G, N, k, fmt), dtype=torch.uint8, device=codes.device)
    dsc = torch.empty(lib.mkd_packed_mx_scale_bytes(G, N, k), dtype=torch.uint8, device=codes.device)
    rc = lib.mkd_pack_mx_weights(codes.data_ptr(), scales.data_ptr(), dst.data_ptr(), dsc.data_ptr(),
                                 G, N, k, codes.stride(0), codes.stride(1), scales.stride(0),
                                 scales.stride(1), fmt, interleave_half, L.stream_ptr(codes.device))
    L.check(rc, "pack_mx_weights")
    return dst, dsc


def _pack_gate_up(codes, scales, fmt):
    lc, ls = gate_up_to_logical(codes, scales)
    E, N2, _ = lc.shape
    H = ls.shape[2] * 32
    return pack_mx(lc, ls, fmt, H, N2 // 2)


def _pack_down(codes, scales, fmt, I):
    lc, ls = down_to_logical(codes, scales, I)
    return pack_mx(lc, ls, fmt, I)


# ---------------------------------------------------------------- moe_tkg (MX)
def moe_tkg_mx(hidden_input, expert_gate_up_weights, expert_down_weights, expert_affinities,
               expert_index, expert_gate_up_bias, expert_down_bias, expert_gate_up_weights_scale,
               expert_down_weights_scale, expert_affinities_scaling_mode, activation_fn,
               output_dtype, gate_clamp_upper_limit, gate_clamp_lower_limit, up_clamp_upper_limit,
               up_clamp_lower_limit):
    """MX selective-expert moe_tkg (selective_expert_mx_impl.py:60-531).

    Flow: hidden (bf16) -> MXFP8; gate/up = scaled MFMA against MX weights (+
    bias), clamps, act(gate) * up in fp32 -> bf16 intermediate -> MXFP8; down =
    scaled MFMA (+ bias); POST_SCALE by the affinity; fp32 sum over k -> bf16.
    """
    fmt = mx_format(expert_gate_up_weights)
    if mx_format(expert_down_weights) != fmt:
        raise ValueError("gate_up and down MX weights must share one element format")
    if expert_gate_up_weights_scale is None or expert_down_weights_scale is None:
        raise ValueError("MX weights need expert_gate_up_weights_scale and expert_down_weights_scale")
    L.require_gpu(hidden_input, expert_gate_up_weights, expert_down_weights, expert_index,
                  expert_gate_up_weights_scale, expert_down_weights_scale)
    T, H = hidden_input.shape
    gcodes = _u8(expert_gate_up_weights)
    E, _, _, Tt, I, _ = gcodes.shape
    if Tt * 512 != H:
        raise ValueError(f"gate_up weights cover H={Tt * 512}, hidden has H={H}")
    if T > 128:
        raise ValueError("Currently only batch size * seq len <= 128 is supported (except for all-expert mode)")
    if I % 32:
        raise ValueError(f"I={I} must be a multiple of 32")
    dcodes = _u8(expert_down_weights)
    if dcodes.shape[0] != E or dcodes.shape[3] != H:
        raise ValueError(f"down weights {tuple(dcodes.shape)} do not match E={E}, H={H}")
    K = expert_index.shape[-1]
    act = {ActFnType.SiLU: L.ACT_SILU, ActFnType.Swish: L.ACT_SWISH, ActFnType.GELU: L.ACT_GELU,
           ActFnType.GELU_Tanh_Approx: L.ACT_GELU_TANH}.get(activation_fn)
    if act is None:
        raise NotImplementedError(f"activation {activation_fn} is not supported")

    # packed once per code tensor (the cache key is the code tensor and its
    # version; its scale tensor is expected to change only together with it)
    gu, gus = packing.packed_cached(
        expert_gate_up_weights, lambda w: _pack_gate_up(w, expert_gate_up_weights_scale, fmt))
    dn, dns = packing.packed_cached(
        expert_down_weights, lambda w: _pack_down(w, expert_down_weights_scale, fmt, I))
    dev = hidden_input.device
    out_dtype = output_dtype if output_dtype is not None else hidden_input.dtype
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    out32 = torch.empty(T, H, dtype=torch.float32, device=dev) if out_dtype == torch.float32 else None
    idx = expert_index.to(torch.int32).contiguous()
    post = expert_affinities_scaling_mode == ExpertAffinityScaleMode.POST_SCALE
    aff = expert_affinities.float().contiguous() if (post and expert_affinities is not None) else None
    gub = None
    if expert_gate_up_bias is not None:
        b = expert_gate_up_bias
        gub = (gate_up_bias_to_logical(b, I) if b.dim() == 5 else b).to(torch.bfloat16).contiguous()
    dnb = expert_down_bias.to(torch.bfloat16).contiguous() if expert_down_bias is not None else None
    inf = math.inf
    hid = hidden_input.to(torch.bfloat16).contiguous()
    args = L.MoeArgs(
        hidden=hid.data_ptr(), gate_up_packed=gu.data_ptr(), down_packed=dn.data_ptr(),
        expert_affinities=L.ptr(aff), slot_weights=None, expert_index=idx.data_ptr(),
        gate_up_bias=L.ptr(gub), down_bias=L.ptr(dnb), residual=None, output=out.data_ptr(),
        output_f32=L.ptr(out32), T=T, H=H, E=E, I=I, K=K,
        scaling_mode=L.SCALE_POST if post else L.SCALE_NONE, activation=act, alpha=1.702,
        gate_hi=gate_clamp_upper_limit if gate_clamp_upper_limit is not None else inf,
        gate_lo=gate_clamp_lower_limit if gate_clamp_lower_limit is not None else -inf,
        up_hi=up_clamp_upper_limit if up_clamp_upper_limit is not None else inf,
        up_lo=up_clamp_lower_limit if up_clamp_lower_limit is not None else -inf,
        round_qwen=0, weight_format=fmt, gate_up_scales=gus.data_ptr(), down_scales=dns.data_ptr())
    lib = L.load()
    ws = torch.empty(lib.mkd_moe_workspace_bytes(T, H, E, I, K), dtype=torch.uint8, device=dev)
    rc = lib.mkd_moe_tkg(args, ws.data_ptr(), ws.numel(), L.stream_ptr(dev))
    L.check(rc, "moe_tkg (mx)")
    if out32 is not None:
        return out32
    return out if out_dtype == torch.bfloat16 else out.to(out_dtype)
