"""rmsnorm_tkg operator (reference: nki_kernels/norm/rmsnorm_tkg.py:49-147)."""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib as L


def rmsnorm_tkg(input: torch.Tensor, gamma: torch.Tensor, output: torch.Tensor,
                eps: float = 1e-6, hidden_actual: Optional[int] = None,
                hidden_dim_tp: bool = False, single_core_forced: bool = False,
                shard_on_h: bool = False, use_heap_memory: bool = False, sbm=None):
    """RMSNorm for decode: output = (input * gamma) * rsqrt(sum(input^2)/H_actual + eps).

    input [B, S, H] (or [T, H]) bf16/fp32 on the GPU; gamma [1, H] or [H] bf16;
    output has input's shape (bf16 or fp32) and is written in place and
    returned, as in the reference.  The reference's SBUF/LNC scheduling flags
    (single_core_forced, shard_on_h, use_heap_memory) have no meaning on one
    GPU and are accepted; their invalid combinations raise as in the
    reference (rmsnorm_tkg.py:118-121).  hidden_dim_tp selects an SBUF
    partition order only and is not supported for HBM tensors.
    """
    if shard_on_h:
        if hidden_dim_tp:
            raise ValueError("hidden_dim_tp is not supported in shard on H implementation")
        if single_core_forced:
            raise ValueError("single_core_forced is not supported in shard on H implementation")
    if hidden_dim_tp:
        raise NotImplementedError("hidden_dim_tp describes an SBUF layout; HBM tensors only")
    if sbm is not None:
        raise NotImplementedError("sbm (SBUF manager) has no GPU equivalent; pass None")
    L.require_gpu(input, gamma, output)
    H = input.shape[-1]
    if output.shape != input.shape:
        raise ValueError(f"output shape {tuple(output.shape)} != input shape {tuple(input.shape)}")
    if gamma.numel() != H:
        raise ValueError(f"gamma must have {H} elements, got {tuple(gamma.shape)}")
    if H % 128 != 0:
        raise ValueError(f"H ({H}) must be divisible by 128")
    dt = {torch.bfloat16: L.DT_BF16, torch.float32: L.DT_F32}
    if input.dtype not in dt or output.dtype not in dt:
        raise ValueError("input/output must be bfloat16 or float32")
    if gamma.dtype != torch.bfloat16:
        gamma = gamma.to(torch.bfloat16)
    x = input.contiguous()
    out = output if output.is_contiguous() else torch.empty_like(output)
    rows = x.numel() // H
    rc = L.load().mkd_rmsnorm_tkg(x.data_ptr(), dt[x.dtype], gamma.contiguous().data_ptr(),
                                  out.data_ptr(), dt[out.dtype], rows, H,
                                  int(hidden_actual) if hidden_actual else 0, float(eps),
                                  L.stream_ptr(x.device))
    L.check(rc, "rmsnorm_tkg")
    if out is not output:
        output.copy_(out)
    return output
