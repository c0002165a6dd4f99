"""GPU parity of the MX (OCP Microscaling) path against the CPU oracle.

Quantisation (codes and E8M0 scale bytes) must be bit-exact with oracle/mx.py.
moe_tkg with MX weights is compared with the fp32 oracle on the dequantised
weights, oracle/ref.py:moe_tkg_mx, at max-abs-rel <= 5e-2.  The reference MX
layouts are built here from their index formulas (moe_tkg.py:105-123), not
with the package's own layout helpers.
"""
import numpy as np
import pytest
import torch

from conftest import max_abs_rel
from oracle import mx as omx
from oracle import ref

pytestmark = pytest.mark.gpu

TOL_MX = 5e-2
FMT = {"e4m3": 1, "e2m1": 2}


def pack_nibbles(codes):
    """[..., 2m] one code per element -> [..., m] bytes, low nibble first."""
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


@pytest.mark.parametrize("rows,K,dtype,fmt", [
    (7, 96, torch.bfloat16, "e4m3"), (33, 2048, torch.bfloat16, "e4m3"),
    (5, 256, torch.float32, "e4m3"), (9, 160, torch.bfloat16, "e2m1"), (4, 512, torch.float32, "e2m1"),
])
def test_quantize_mx_bit_exact(mk, dev, rows, K, dtype, fmt):
    from nki_moe_megakernel_amd import mx
    g = torch.Generator().manual_seed(rows * K)
    x = torch.randn(rows, K, generator=g) * torch.exp2(torch.randint(-20, 20, (rows, 1), generator=g).float())
    x[0] = 0.0                                              # all-zero blocks
    x[1, :32] = torch.linspace(-500, 500, 32)               # saturating block
    x[-1, -32:] = 1e-30                                     # tiny block
    x = x.to(dtype)
    k_pad = (K + 127) // 128 * 128
    codes, scales = mx.quantize_mx(x.to(dev), FMT[fmt], k_pad)
    oc, os_ = omx.quantize_mx(x.float().numpy(), fmt)
    want_c = np.zeros((rows, k_pad), np.uint8)
    want_c[:, :K] = oc
    if fmt == "e2m1":
        want_c = pack_nibbles(want_c)
    want_s = np.zeros((rows, k_pad // 32), np.uint8)
    want_s[:, : K // 32] = os_
    np.testing.assert_array_equal(scales.cpu().numpy(), want_s)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_c)


def reference_gate_up_layout(codes_l, scales_l, I, fmt):
    """Logical [E, 2I, H] codes (one per element) + [E, 2I, H/32] scales -> the
    reference [E, 128, 2, H/512, I, x4] codes and [E, 16, 2, H/512, I] scales:
    element (e, g, i, h = t*512 + 4p + j) sits at [e, p, g, t, i, j]."""
    E, _, H = codes_l.shape
    T = H // 512
    e, p, gg, t, i, j = np.indices((E, 128, 2, T, I, 4), sparse=True)
    c = codes_l[e, gg * I + i, t * 512 + 4 * p + j]
    if fmt == "e2m1":
        c = pack_nibbles(c)
    e, pb, gg, t, i = np.indices((E, 16, 2, T, I), sparse=True)
    s = scales_l[e, gg * I + i, t * 16 + pb]
    return np.ascontiguousarray(c), np.ascontiguousarray(s)


def reference_down_layout(codes_l, scales_l, I, fmt):
    """Logical [E, H, I] codes + [E, H, I/32] scales -> [E, I_p, ceil(I/512), H, x4]
    codes and [E, I_p/8, ceil(I/512), H] scales; element (e, h, i = t*512 + 4p + j)
    at [e, p, t, h, j], zero past I."""
    E, H, _ = codes_l.shape
    Ip = I // 4 if I <= 512 else 128
    T = (I + 511) // 512
    e, p, t, h, j = np.indices((E, Ip, T, H, 4), sparse=True)
    ii = t * 512 + 4 * p + j
    c = np.where(ii < I, codes_l[e, h, np.minimum(ii, I - 1)], 0).astype(np.uint8)
    if fmt == "e2m1":
        c = pack_nibbles(c)
    e, pb, t, h = np.indices((E, Ip // 8, T, H), sparse=True)
    bi = t * 16 + pb
    s = np.where(bi < I // 32, scales_l[e, h, np.minimum(bi, I // 32 - 1)], 0).astype(np.uint8)
    return np.ascontiguousarray(c), np.ascontiguousarray(s)


def reference_gate_up_bias(b, I):
    """[E, 2, I] -> [E, I_p, 2, ceil(I/512), 4]: (e, g, i = t*512 + 4p + j) at [e, p, g, t, j]."""
    E = b.shape[0]
    Ip = I // 4 if I <= 512 else 128
    T = (I + 511) // 512
    e, p, gg, t, j = np.indices((E, Ip, 2, T, 4), sparse=True)
    ii = t * 512 + 4 * p + j
    return np.where(ii < I, b[e, gg, np.minimum(ii, I - 1)], 0).astype(np.float32)


@pytest.mark.parametrize("T,E,K,H,I,fmt,act,clamp,bias", [
    (1, 8, 2, 512, 256, "e4m3", "silu", False, False),
    (5, 16, 4, 1024, 768, "e4m3", "silu", False, False),
    (40, 8, 2, 512, 128, "e4m3", "silu", False, True),
    (32, 32, 4, 512, 192, "e2m1", "swish", True, True),
    (3, 4, 2, 512, 2880, "e2m1", "swish", True, True),
])
def test_moe_tkg_mx(mk, dev, T, E, K, H, I, fmt, act, clamp, bias):
    from nki_moe_megakernel_amd import mx
    from nki_moe_megakernel_amd.common_types import ActFnType, ExpertAffinityScaleMode
    g = torch.Generator().manual_seed(T * 7 + I)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gu_l = (0.05 * torch.randn(E, 2 * I, H, generator=g)).to(torch.bfloat16).float()
    dn_l = (0.05 * torch.randn(E, H, I, generator=g)).to(torch.bfloat16).float()
    gc, gs = omx.quantize_mx(gu_l.numpy(), fmt)
    dc, ds = omx.quantize_mx(dn_l.numpy(), fmt)
    gu_deq = torch.from_numpy(omx.dequantize_mx(gc, gs, fmt))
    dn_deq = torch.from_numpy(omx.dequantize_mx(dc, ds, fmt))
    rgc, rgs = reference_gate_up_layout(gc, gs, I, fmt)
    rdc, rds = reference_down_layout(dc, ds, I, fmt)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    aff = torch.zeros(T, E).scatter_(1, idx.long(), torch.rand(T, K, generator=g))
    gub = (0.1 * torch.randn(E, 2, I, generator=g)).to(torch.bfloat16) if bias else None
    dnb = (0.1 * torch.randn(E, H, generator=g)).to(torch.bfloat16) if bias else None
    kw = dict(gate_clamp_upper_limit=7.0, up_clamp_upper_limit=8.0, up_clamp_lower_limit=-6.0) if clamp else {}
    t = lambda a: torch.from_numpy(a).to(dev)
    out = mk.moe_tkg(
        x.to(dev), t(rgc), t(rdc), aff.to(dev), idx.to(dev), False,
        expert_gate_up_bias=torch.from_numpy(reference_gate_up_bias(gub.float().numpy(), I)).to(torch.bfloat16).to(dev) if bias else None,
        expert_down_bias=dnb.to(dev) if bias else None,
        expert_gate_up_weights_scale=t(rgs), expert_down_weights_scale=t(rds),
        expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE,
        activation_fn=ActFnType.Swish if act == "swish" else ActFnType.SiLU, **kw)
    y_ref = ref.moe_tkg_mx(x, gu_deq, dn_deq, aff, idx.long(), gub, dnb, "post", act,
                           gate_clamp_upper=7.0 if clamp else None,
                           up_clamp_upper=8.0 if clamp else None, up_clamp_lower=-6.0 if clamp else None)
    assert out.shape == (T, H)
    err = max_abs_rel(out, y_ref)
    assert err < TOL_MX, err

    # the package's bf16 -> MX converter yields exactly these reference tensors
    gu_ref_bf = gu_l.reshape(E, 2, I, H).permute(0, 3, 1, 2).to(torch.bfloat16)     # [E, H, 2, I]
    dn_ref_bf = dn_l.permute(0, 2, 1).to(torch.bfloat16)                            # [E, I, H]
    qgc, qgs, qdc, qds = mx.quantize_experts_mx(gu_ref_bf.to(dev), dn_ref_bf.to(dev), FMT[fmt])
    np.testing.assert_array_equal(qgc.cpu().numpy(), rgc)
    np.testing.assert_array_equal(qgs.cpu().numpy(), rgs)
    np.testing.assert_array_equal(qdc.cpu().numpy(), rdc)
    np.testing.assert_array_equal(qds.cpu().numpy(), rds)


def test_moe_tkg_mx_rejects_bad_inputs(mk, dev):
    from nki_moe_megakernel_amd import mx
    E, H, I, T, K = 4, 512, 64, 2, 2
    gc = torch.zeros(E, 128, 2, H // 512, I, 4, dtype=torch.uint8, device=dev)
    dc = torch.zeros(E, I // 4, 1, H, 4, dtype=torch.uint8, device=dev)
    idx = torch.zeros(T, K, dtype=torch.int32, device=dev)
    x = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):          # scales missing
        mk.moe_tkg(x, gc, dc, torch.zeros(T, E, device=dev), idx, False)
    with pytest.raises(ValueError):          # formats differ
        mk.moe_tkg(x, gc, dc[..., :2].contiguous(), torch.zeros(T, E, device=dev), idx, False,
                   expert_gate_up_weights_scale=torch.zeros(E, 16, 2, 1, I, dtype=torch.uint8, device=dev),
                   expert_down_weights_scale=torch.zeros(E, 2, 1, H, dtype=torch.uint8, device=dev))
    with pytest.raises(ValueError):          # k not a multiple of 32
        mx.quantize_mx(torch.zeros(2, 48, device=dev), 1, 128)
