"""MI355X-native decode hot path of a Mixture-of-Experts transformer.

Operator surface (same names, argument order and defaults as the reference):
  rmsnorm_tkg           nki_kernels/norm/rmsnorm_tkg.py:49
  attention_block_tkg   nki_kernels/attention/attention_block_tkg.py:83
  router_topk           nki_kernels/moe/router_topk.py:69
  moe_tkg               nki_kernels/moe/moe_tkg.py:56
  moe_prefill           moe_tkg for prefill-shaped batches (T > 128; no
                        reference counterpart), LDS-tiled MFMA GEMMs
Model surface:
  qwen_with_megakernel  megakernels/qwen3_moe/qwen_with_megakernel.py
  gpt_oss_with_megakernel  megakernels/gpt_oss/gpt_oss_with_megakernel.py
  checkpoint            HF safetensors directories -> packed decode models
                        (the converters at qwen_with_megakernel.py:171-271,
                        gpt_oss_with_megakernel.py:290-327)

All compute runs in libmkd.so (hand-written HIP for gfx950, C ABI in
include/mkd.h).  The package directory name contains dashes, so it is
imported through ``__graft_entry__.load_package()`` (registered as
``nki_moe_megakernel_amd``).
"""
from . import _lib
from .attention import attention_block_tkg
from .common_types import (ActFnType, ExpertAffinityScaleMode, QuantizationType,
                           RouterActFnType)
from .moe import moe_prefill, moe_tkg, router_topk
from .norm import rmsnorm_tkg

__all__ = ["rmsnorm_tkg", "attention_block_tkg", "router_topk", "moe_tkg", "moe_prefill", "ActFnType",
           "ExpertAffinityScaleMode", "QuantizationType", "RouterActFnType"]
