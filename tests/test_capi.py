"""CPU checks of the C ABI: libmkd.so loads and exports every symbol include/*.h declares,
and the ctypes binding covers exactly those symbols.  No compute calls (no GPU here)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "nki-moe-megakernel_amd", "libmkd.so")


def declared_symbols():
    syms = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b(mkd_[a-z0-9_]+)\s*\(", src):
            syms.add(m.group(1))
    return syms


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ["mkd_rmsnorm_tkg", "mkd_router_topk", "mkd_moe_tkg", "mkd_attention_block_tkg",
              "mkd_qwen3_decode_layers", "mkd_last_error"]:
        assert s in syms


@pytest.mark.skipif(not os.path.exists(LIB), reason="libmkd.so not built")
def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (same HIP runtime the package binds to)
    lib = ctypes.CDLL(LIB)
    missing = [s for s in sorted(declared_symbols()) if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_matches_header():
    import __graft_entry__ as ge
    from importlib import import_module
    ge.load_package()
    L = import_module("nki_moe_megakernel_amd._lib")
    assert set(L.EXPORTED) == declared_symbols()


def test_operators_fail_loudly_without_gpu_tensors():
    import torch
    import __graft_entry__ as ge
    mk = ge.load_package()
    x = torch.zeros(1, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        mk.rmsnorm_tkg(x, torch.ones(128, dtype=torch.bfloat16), torch.empty_like(x))


def test_packed_cache_is_per_tensor_and_version(mk):
    """The repack memo hits for the same tensor object, misses after an in-place
    change or for another tensor, and drops the entry when the tensor dies."""
    import gc
    import torch
    from nki_moe_megakernel_amd import packing
    calls = []

    def fake_pack(t):
        calls.append(1)
        return t.clone()

    a = torch.randn(4, 8)
    b = torch.randn(4, 8)
    pa = packing.packed_cached(a, fake_pack)
    assert packing.packed_cached(a, fake_pack) is pa and len(calls) == 1
    packing.packed_cached(b, fake_pack)
    assert len(calls) == 2
    a.add_(1.0)                      # bumps the version counter
    assert packing.packed_cached(a, fake_pack) is not pa and len(calls) == 3
    ident = id(b)
    del b
    gc.collect()
    assert ident not in packing._cache


def test_router_static_scratch_covers_every_accepted_shape():
    """mkd_router_topk_static's scratch (2 MiB + 256 B) holds the split-K partial
    logits of every shape mkd_router_topk accepts (T <= 128, E <= 512)."""
    from nki_moe_megakernel_amd import _lib as L
    lib = L.load()
    cap = (1 << 21) + 256
    worst = 0
    for E in range(1, 513):
        for H in (32, 64, 96, 512, 1024, 2048, 2880, 3072, 4096, 8192):
            worst = max(worst, lib.mkd_router_workspace_bytes(128, H, E))
    assert worst <= cap, worst
