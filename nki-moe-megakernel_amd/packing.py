"""Weight repacking into the library's MFMA fragment layout (device-side).

The reference's converters turn HF checkpoints into the NKI kernels' layouts
(convert_qwen3_moe_hf_to_neuron_state_dict, megakernels/qwen3_moe/
qwen_with_megakernel.py:171-271).  Here every weight matrix becomes the frag
layout documented in csrc/gemm.hip: for a logical [n, k] matrix (n output
features, k contraction), 16-row x 32-k MFMA A-fragments stored as contiguous
1 KiB blocks.  The repack runs on the GPU through mkd_pack_weights.

Operator-level calls receive the reference layouts ([in, out] for W_qkv, W_out,
router w, [E, H, 2, I] / [E, I, H] for experts); `packed_cached` memoises the
repack per source tensor object (weakly keyed, invalidated by in-place
modification through the tensor version counter).
"""
from __future__ import annotations

import weakref

import torch

from . import _lib as L

# id(source tensor) -> (weakref to it, key, packed); an entry is dropped when its
# source tensor is collected.  (A WeakKeyDictionary would compare tensor keys
# with ==, which is elementwise for tensors.)
_cache: "dict[int, tuple]" = {}


def pack(src: torch.Tensor, groups: int, n: int, k: int, g_stride: int, row_stride: int,
         col_stride: int, interleave_half: int = 0) -> torch.Tensor:
    """Repack a bf16 device tensor viewed as [groups][n][k] with the given element strides."""
    L.require_gpu(src)
    if src.dtype != torch.bfloat16:
        raise ValueError(f"weights must be bfloat16, got {src.dtype}")
    lib = L.load()
    out = torch.empty(lib.mkd_packed_bytes(groups, n, k) // 2, dtype=torch.bfloat16, device=src.device)
    rc = lib.mkd_pack_weights(src.data_ptr(), out.data_ptr(), groups, n, k, g_stride, row_stride,
                              col_stride, interleave_half, L.stream_ptr(src.device))
    L.check(rc, "pack_weights")
    return out


def pack_fp8_in_out(w: torch.Tensor) -> torch.Tensor:
    """float8 e4m3 weights in the reference layout [k_in, n_out] (or G such
    matrices [G, k_in, n_out]; torch.float8_e4m3fn, or uint8 codes) -> the
    frag-packed e4m3 layout of the FP8 projections and experts."""
    L.require_gpu(w)
    if w.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise ValueError(f"FP8 weights must be float8_e4m3, got {w.dtype}")
    k, n = w.shape[-2], w.shape[-1]
    g = w.numel() // (k * n)
    src = w.contiguous().view(torch.uint8)
    lib = L.load()
    out = torch.empty(lib.mkd_packed_fp8_bytes(g, n, k), dtype=torch.uint8, device=w.device)
    rc = lib.mkd_pack_fp8_weights(src.data_ptr(), out.data_ptr(), g, n, k, L.stream_ptr(w.device))
    L.check(rc, "pack_fp8_weights")
    return out


def pack_fp8_experts_gate_up(w: torch.Tensor) -> torch.Tensor:
    """FP8 experts' gate/up [E, H, 2, I] e4m3 -> E x packed [H, 2I] (gate columns first)."""
    E, H, two, I = w.shape
    assert two == 2
    return pack_fp8_in_out(w.reshape(E, H, 2 * I))


def pack_out_in(w: torch.Tensor) -> torch.Tensor:
    """HF / nn.Linear layout [n_out, k_in] -> packed."""
    n, k = w.shape
    return pack(w, 1, n, k, 0, w.stride(0), w.stride(1))


def pack_in_out(w: torch.Tensor) -> torch.Tensor:
    """Reference layout [k_in, n_out] (x @ W) -> packed."""
    k, n = w.shape
    return pack(w, 1, n, k, 0, w.stride(1), w.stride(0))


def pack_in_out_exact(w: torch.Tensor) -> torch.Tensor:
    """[k_in, n_out] -> packed, accepting fp32 weights whose values are bf16-representable
    (the Qwen router keeps bf16 weights in fp32 registers, moe_fused_nki.py:189-205)."""
    if w.dtype == torch.float32:
        wb = w.to(torch.bfloat16)
        if not torch.equal(wb.float(), w):
            raise NotImplementedError("fp32 weights must hold bf16-representable values")
        w = wb
    return pack_in_out(w)


def pack_experts_gate_up_ref(w: torch.Tensor) -> torch.Tensor:
    """Reference [E, H, 2, I] -> E x packed [2I, H] with gate/up row blocks interleaved."""
    E, H, two, I = w.shape
    assert two == 2
    # logical row n in [0, 2I): n < I -> gate column n, else up column n - I
    # element (e, n, h) at e*sE + (n // I)*s2 + (n % I)*sI + h*sH; since the
    # (2, I) pair is contiguous as 2*I when w is contiguous, row stride = sI.
    if not (w.stride(2) == I * w.stride(3)):
        w = w.contiguous()
    return pack(w, E, 2 * I, H, w.stride(0), w.stride(3), w.stride(1), interleave_half=I)


def pack_experts_down_ref(w: torch.Tensor) -> torch.Tensor:
    """Reference [E, I, H] -> E x packed [H, I]."""
    E, I, H = w.shape
    return pack(w, E, H, I, w.stride(0), w.stride(2), w.stride(1))


def pack_experts_gate_up_hf(w: torch.Tensor) -> torch.Tensor:
    """HF fused [E, 2I, H] (gate rows then up rows) -> E x packed, interleaved."""
    E, I2, H = w.shape
    return pack(w, E, I2, H, w.stride(0), w.stride(1), w.stride(2), interleave_half=I2 // 2)


def pack_experts_down_hf(w: torch.Tensor) -> torch.Tensor:
    """HF [E, H, I] -> E x packed [H, I]."""
    E, H, I = w.shape
    return pack(w, E, H, I, w.stride(0), w.stride(1), w.stride(2))


def packed_cached(src: torch.Tensor, fn) -> torch.Tensor:
    """Memoise fn(src) per tensor object and version."""
    ident = id(src)
    key = (fn.__name__, src._version, src.data_ptr(), tuple(src.shape), tuple(src.stride()))
    ent = _cache.get(ident)
    same = ent is not None and ent[0]() is src
    if same and ent[1] == key:
        return ent[2]
    out = fn(src)
    if not same:
        weakref.finalize(src, _cache.pop, ident, None)
    _cache[ident] = (weakref.ref(src), key, out)
    return out
