"""ctypes binding of libmkd.so (C ABI in include/mkd.h).

The library is loaded from this package directory.  There is no fallback: if
the HIP build is missing, every operator raises ``MkdLibraryMissing``.
``torch`` is imported first so that the HIP runtime torch ships with is the one
libmkd binds to (both carry the SONAME libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes as C
import os

import torch  # noqa: F401  (must precede the CDLL load, see module doc)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmkd.so")

MKD_OK = 0
MKD_ERR_INVALID = -1
MKD_ERR_NULL = -2
MKD_ERR_UNSUPPORTED = -3
MKD_ERR_WORKSPACE = -4
MKD_ERR_HIP = -5
DT_BF16, DT_F32 = 0, 1

ROUTER_SIGMOID, ROUTER_PRE_NORM, ROUTER_NORM_TOPK, ROUTER_QWEN = 1, 2, 4, 8
ACT_SILU, ACT_SWISH, ACT_GELU, ACT_GELU_TANH = 0, 1, 2, 3
SCALE_NONE, SCALE_POST = 0, 1
FP8_E4M3 = 3          # MKD_FP8_E4M3: mkd_moe_args::weight_format of e4m3 experts


class MkdLibraryMissing(RuntimeError):
    pass


class MkdError(RuntimeError):
    pass


vp = C.c_void_p
i32 = C.c_int
f32 = C.c_float
i64 = C.c_longlong
sz = C.c_size_t


class MoeArgs(C.Structure):
    _fields_ = [
        ("hidden", vp), ("gate_up_packed", vp), ("down_packed", vp),
        ("expert_affinities", vp), ("slot_weights", vp), ("expert_index", vp),
        ("gate_up_bias", vp), ("down_bias", vp), ("residual", vp), ("output", vp),
        ("output_f32", vp),
        ("T", i32), ("H", i32), ("E", i32), ("I", i32), ("K", i32),
        ("scaling_mode", i32), ("activation", i32), ("alpha", f32),
        ("gate_hi", f32), ("gate_lo", f32), ("up_hi", f32), ("up_lo", f32),
        ("round_qwen", i32),
        ("weight_format", i32), ("gate_up_scales", vp), ("down_scales", vp),
    ]


class AttentionArgs(C.Structure):
    _fields_ = [
        ("X", vp), ("rmsnorm_gamma", vp), ("rmsnorm_eps", f32), ("rmsnorm_order", i32),
        ("w_qkv_packed", vp), ("bias_qkv", vp), ("q_norm", vp), ("k_norm", vp),
        ("qk_eps", f32), ("cos", vp), ("sin", vp), ("k_cache", vp), ("v_cache", vp),
        ("n_prior", vp), ("mask", vp), ("mask_s_ctx", i32), ("sink", vp),
        ("softmax_scale", f32), ("update_cache", i32), ("kv_cache_update_idx", vp),
        ("w_out_packed", vp), ("bias_out", vp), ("residual", vp), ("out", vp),
        ("B", i32), ("H", i32), ("H_out", i32), ("nq", i32), ("nkv", i32), ("d", i32),
        ("S_max", i32), ("round_qwen", i32),
        ("active_blocks_table", vp), ("blocks_per_seq", i32), ("block_len", i32), ("num_blocks", i32),
        ("hidden_actual", i32), ("window", i32), ("s_tkg", i32),
        ("q_norm_post", vp), ("k_norm_post", vp), ("qk_post_eps", f32),
        ("kv_format", i32), ("k_scale", vp), ("v_scale", vp),
        ("quant_qkv", i32), ("quant_out", i32), ("w_scale_qkv", vp), ("in_scale_qkv", vp),
        ("w_scale_out", vp), ("in_scale_out", vp),
    ]


KV_FP8 = 1            # MKD_KV_FP8
KV_K_TRANSPOSED = 2   # MKD_KV_K_TRANSPOSED


class Qwen3Model(C.Structure):
    _fields_ = [
        ("num_layers", i32), ("H", i32), ("nq", i32), ("nkv", i32), ("d", i32), ("E", i32),
        ("K", i32), ("I", i32), ("S_max", i32), ("eps", f32),
        ("w_qkv", C.POINTER(vp)), ("w_o", C.POINTER(vp)), ("q_norm", C.POINTER(vp)),
        ("k_norm", C.POINTER(vp)), ("ln_in", C.POINTER(vp)), ("ln_post", C.POINTER(vp)),
        ("router", C.POINTER(vp)), ("gate_up", C.POINTER(vp)), ("down", C.POINTER(vp)),
        ("k_cache", C.POINTER(vp)), ("v_cache", C.POINTER(vp)), ("inv_freq", vp),
        ("expert_format", i32), ("gate_up_scales", C.POINTER(vp)), ("down_scales", C.POINTER(vp)),
        ("block_table", vp), ("blocks_per_seq", i32), ("block_len", i32), ("num_blocks", i32),
        ("variant", i32), ("H_actual", i32), ("b_qkv", C.POINTER(vp)), ("b_o", C.POINTER(vp)),
        ("sinks", C.POINTER(vp)), ("router_bias", C.POINTER(vp)), ("gate_up_bias", C.POINTER(vp)),
        ("down_bias", C.POINTER(vp)), ("window", C.POINTER(i32)), ("layer_s_max", C.POINTER(i32)),
        ("act_alpha", f32), ("gate_hi", f32), ("gate_lo", f32), ("up_hi", f32), ("up_lo", f32),
        ("layer_table", vp), ("route_log", vp), ("route_log_bytes", sz),
    ]


# name: (restype, argtypes)
_SIGS = {
    "mkd_version": (i32, []),
    "mkd_last_error": (C.c_char_p, []),
    "mkd_rmsnorm_tkg": (i32, [vp, i32, vp, vp, i32, i32, i32, i32, f32, vp]),
    "mkd_packed_bytes": (sz, [i32, i32, i32]),
    "mkd_pack_weights": (i32, [vp, vp, i32, i32, i32, i64, i64, i64, i32, vp]),
    "mkd_linear": (i32, [vp, i32, i32, i32, vp, i32, i32, vp, vp, i32, i32, vp, vp]),
    "mkd_router_workspace_bytes": (sz, [i32, i32, i32]),
    "mkd_router_topk": (i32, [vp, i32, i32, i32, vp, i32, vp, vp, vp, vp, vp, i32, i32, vp, sz, vp]),
    "mkd_router_topk_static": (i32, [vp, i32, i32, i32, vp, i32, vp, vp, vp, vp, vp, i32, i32, vp]),
    "mkd_quantize_mx": (i32, [vp, i32, i32, i32, i32, i32, vp, vp, i32, vp]),
    "mkd_packed_mx_bytes": (sz, [i32, i32, i32, i32]),
    "mkd_packed_mx_scale_bytes": (sz, [i32, i32, i32]),
    "mkd_pack_mx_weights": (i32, [vp, vp, vp, vp, i32, i32, i32, i64, i64, i64, i64, i32, i32, vp]),
    "mkd_moe_workspace_bytes": (sz, [i32, i32, i32, i32, i32]),
    "mkd_moe_tkg": (i32, [C.POINTER(MoeArgs), vp, sz, vp]),
    "mkd_moe_prefill": (i32, [C.POINTER(MoeArgs), vp, sz, vp]),
    "mkd_attention_workspace_bytes": (sz, [i32, i32, i32, i32, i32, i32]),
    "mkd_attention_workspace_bytes_tkg": (sz, [i32, i32, i32, i32, i32, i32, i32]),
    "mkd_attention_block_tkg": (i32, [C.POINTER(AttentionArgs), vp, sz, vp]),
    "mkd_packed_fp8_bytes": (sz, [i32, i32, i32]),
    "mkd_pack_fp8_weights": (i32, [vp, vp, i32, i32, i32, vp]),
    "mkd_qwen3_workspace_bytes": (sz, [C.POINTER(Qwen3Model), i32]),
    "mkd_qwen3_route_log_bytes": (sz, [C.POINTER(Qwen3Model), i32]),
    "mkd_qwen3_route_log_layout": (i32, [C.POINTER(Qwen3Model), i32, C.POINTER(sz)]),
    "mkd_qwen3_decode_layers": (i32, [C.POINTER(Qwen3Model), i32, vp, vp, vp, vp, vp, sz, vp]),
    "mkd_qwen3_prefill_layers": (i32, [C.POINTER(Qwen3Model), i32, i32, vp, vp, vp, vp, vp, sz, vp]),
    "mkd_embed": (i32, [vp, vp, vp, i32, i32, i32, vp]),
    "mkd_lm_head_workspace_bytes": (sz, [i32, i32, i32]),
    "mkd_lm_head_greedy": (i32, [vp, vp, f32, vp, i32, i32, i32, i32, i32, vp, vp, vp, sz, vp]),
    "mkd_decode_advance": (i32, [vp, vp, vp, i32, vp]),
    "mkd_profile_events": (i32, [i32, C.POINTER(vp), C.POINTER(vp), i32]),
    "mkd_profile_count": (i32, []),
    "mkd_set_decode_path": (i32, [i32]),
    "mkd_qwen3_layer_table_bytes": (sz, [C.POINTER(Qwen3Model)]),
    "mkd_qwen3_write_layer_table": (i32, [C.POINTER(Qwen3Model), vp, sz]),
    "mkd_qwen3_decode_plan": (i32, [C.POINTER(Qwen3Model), i32, C.POINTER(i32)]),
    "mkd_selfcheck_bf16_round": (i32, [vp, vp]),
    "mkd_qwen3_layer_kernel_status": (i32, [C.POINTER(Qwen3Model), i32, vp, sz, C.POINTER(i32),
                                            C.POINTER(i32)]),
}
KCLASS = {"moe_gate_up": 1, "moe_down": 2, "qkv": 3, "oproj": 4, "attn": 5, "lm_head": 6,
          "router": 7, "layer": 8}

EXPORTED = tuple(_SIGS)

_lib = None


def load(path: str = LIB_PATH):
    """Load libmkd.so once; raise MkdLibraryMissing if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise MkdLibraryMissing(
            f"{path} not found: build it with `python nki-moe-megakernel_amd/build.py` "
            "(there is no CPU fallback)")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str):
    if rc == MKD_OK:
        return
    msg = load().mkd_last_error().decode(errors="replace")
    if rc in (MKD_ERR_INVALID, MKD_ERR_NULL, MKD_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    if rc == MKD_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise MkdError(f"{what}: {msg} (rc={rc})")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("mkd operators take device (HIP) tensors; got a CPU tensor")
