"""MX (microscaling) expert path -- placeholder until the MXFP8 kernels land."""
from __future__ import annotations

import torch

MX_DTYPES = tuple(d for d in (getattr(torch, "float8_e4m3fn", None),) if d is not None)


def is_mx_weight(w: torch.Tensor) -> bool:
    return w.dtype in MX_DTYPES


def moe_tkg_mx(*args, **kwargs):
    raise NotImplementedError("MX expert weights are not implemented yet")
