"""mkd_router_topk_static (router top-k with its scratch in a library device
array, for callers that cannot allocate) against mkd_router_topk (the same
kernels on a caller workspace), through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller input, and a clear error past the
scratch's maximum."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(L, dev, T, H, E, k, mode, x_f32, seed, static):
    from nki_moe_megakernel_amd import packing
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    x = (x if x_f32 else x.to(torch.bfloat16)).to(dev)
    w = (0.02 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(dev)
    wp = packing.pack_out_in(w)
    logits = torch.full((T, E), float("nan"), device=dev)
    aff = torch.full((T, E), float("nan"), device=dev)
    idx = torch.full((T, k), -7, dtype=torch.int32, device=dev)
    topk = torch.full((T, k), float("nan"), device=dev)
    lib = L.load()
    dt = L.DT_F32 if x_f32 else L.DT_BF16
    args = (x.data_ptr(), dt, T, H, wp.data_ptr(), E, None, logits.data_ptr(), aff.data_ptr(),
            idx.data_ptr(), topk.data_ptr(), k, mode)
    if static:
        rc = lib.mkd_router_topk_static(*args, L.stream_ptr(dev))
    else:
        ws = torch.empty(lib.mkd_router_workspace_bytes(T, H, E), dtype=torch.uint8, device=dev)
        rc = lib.mkd_router_topk(*args, ws.data_ptr(), ws.numel(), L.stream_ptr(dev))
    L.check(rc, "router_topk_static" if static else "router_topk")
    torch.cuda.synchronize()
    return logits.cpu(), aff.cpu(), idx.cpu(), topk.cpu()


def test_router_topk_static_matches_workspace_entry(mk, dev):
    from nki_moe_megakernel_amd import _lib as L
    qwen = L.ROUTER_QWEN | L.ROUTER_PRE_NORM | L.ROUTER_NORM_TOPK
    cases = [   # second call smaller than the first: stale scratch must not matter
        (128, 2048, 240, 8, qwen, True, 11),       # the scratch's largest use: 16 K-slices x 240
        (128, 2048, 512, 8, qwen, True, 15),
        (5, 1024, 64, 4, L.ROUTER_PRE_NORM, False, 12),
        (64, 2048, 128, 8, qwen, True, 13),
        (1, 2048, 128, 8, qwen, True, 14),
    ]
    for T, H, E, k, mode, xf, seed in cases:
        a = _case(L, dev, T, H, E, k, mode, xf, seed, static=True)
        b = _case(L, dev, T, H, E, k, mode, xf, seed, static=False)
        for u, v in zip(a, b):
            assert torch.equal(u, v), (T, H, E)
        assert bool((a[2] >= 0).all() and (a[2] < E).all())


def test_router_topk_static_rejects_out_of_range(mk, dev):
    from nki_moe_megakernel_amd import _lib as L
    lib = L.load()
    z = torch.zeros(16, dtype=torch.float32, device=dev)
    rc = lib.mkd_router_topk_static(z.data_ptr(), L.DT_F32, 129, 2048, z.data_ptr(), 128, None,
                                    z.data_ptr(), z.data_ptr(), z.data_ptr(), None, 8, 0,
                                    L.stream_ptr(dev))
    assert rc == L.MKD_ERR_INVALID
    assert b"T 129" in lib.mkd_last_error()
