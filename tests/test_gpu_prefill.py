"""moe_prefill (LDS-tiled grouped MFMA GEMMs) against the fp32 oracle.

The prefill-shaped entry runs moe_tkg's selective-expert computation
(moe_tkg.py:151-170 pseudocode; oracle.ref.moe_tkg) for batches with many
tokens per expert.  Tolerance as for the decode path: max-abs error relative
to the reference's max-abs, 2e-2.
"""
import pytest
import torch

from conftest import max_abs_rel
from oracle import ref

pytestmark = pytest.mark.gpu
TOL = 2e-2


def bf(t):
    return t.to(torch.bfloat16)


def _case(T, E, K, H, I, bias, seed, skew=False):
    g = torch.Generator().manual_seed(seed)
    x = bf(torch.randn(T, H, generator=g))
    gu = bf(0.03 * torch.randn(E, H, 2, I, generator=g))
    dn = bf(0.03 * torch.randn(E, I, H, generator=g))
    if skew:   # every token routes to expert 0 first: one group holds all T tokens
        rest = torch.stack([torch.randperm(E - 1, generator=g)[:K - 1] + 1 for _ in range(T)])
        idx = torch.cat([torch.zeros(T, 1, dtype=torch.long), rest], 1).to(torch.int32)
    else:
        idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    w = torch.rand(T, K, generator=g)
    aff = torch.zeros(T, E).scatter_(1, idx.long(), w)
    gub = bf(0.1 * torch.randn(E, 2, I, generator=g)) if bias else None
    dnb = bf(0.1 * torch.randn(E, H, generator=g)) if bias else None
    return x, gu, dn, idx, aff, gub, dnb


@pytest.mark.parametrize("T,E,K,H,I,act,clamp,bias,skew", [
    (512, 8, 2, 512, 256, "silu", False, False, False),     # ~128 tokens per expert
    (1536, 4, 2, 448, 192, "swish", True, True, False),     # ~768 per expert; partial row tiles
    (300, 16, 4, 256, 64, "silu", False, True, True),       # one group of all 300 tokens
    (2048, 32, 4, 1024, 384, "silu", False, False, False),  # 256 per expert, deeper K
])
def test_moe_prefill_matches_oracle(mk, dev, T, E, K, H, I, act, clamp, bias, skew):
    from nki_moe_megakernel_amd.common_types import ActFnType, ExpertAffinityScaleMode
    print(f"moe_prefill T={T} E={E} K={K} H={H} I={I} act={act} clamp={clamp} bias={bias} skew={skew}",
          flush=True)
    x, gu, dn, idx, aff, gub, dnb = _case(T, E, K, H, I, bias, seed=T * 7 + E, skew=skew)
    kw = dict(gate_clamp_upper_limit=7.0, up_clamp_upper_limit=7.0, up_clamp_lower_limit=-7.0) if clamp else {}
    out = mk.moe_prefill(x.to(dev), gu.to(dev), dn.to(dev), aff.to(dev), idx.to(dev),
                         expert_gate_up_bias=gub.to(dev) if bias else None,
                         expert_down_bias=dnb.to(dev) if bias else None,
                         expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE,
                         activation_fn=ActFnType.Swish if act == "swish" else ActFnType.SiLU, **kw)
    torch.cuda.synchronize()
    y_ref = ref.moe_tkg(x, gu, dn, aff, idx.long(), gub, dnb, "post", act,
                        gate_clamp_upper=7.0 if clamp else None,
                        up_clamp_upper=7.0 if clamp else None, up_clamp_lower=-7.0 if clamp else None)
    assert out.shape == (T, H)
    assert torch.isfinite(out.float()).all()
    assert max_abs_rel(out, y_ref) < TOL


def test_moe_prefill_agrees_with_decode_path(mk, dev):
    """At T = 128 both entries apply: same result to the decode tolerance, and
    the tiled path is deterministic run to run."""
    from nki_moe_megakernel_amd.common_types import ExpertAffinityScaleMode
    x, gu, dn, idx, aff, _, _ = _case(128, 8, 2, 512, 128, False, seed=11)
    args = (x.to(dev), gu.to(dev), dn.to(dev), aff.to(dev), idx.to(dev))
    post = ExpertAffinityScaleMode.POST_SCALE
    a = mk.moe_prefill(*args, expert_affinities_scaling_mode=post)
    b = mk.moe_prefill(*args, expert_affinities_scaling_mode=post)
    c = mk.moe_tkg(*args, False, expert_affinities_scaling_mode=post)
    torch.cuda.synchronize()
    torch.testing.assert_close(a, b, rtol=0, atol=0)
    assert max_abs_rel(a, c.float()) < TOL


def test_moe_prefill_rejects_unsupported(mk, dev):
    x = torch.zeros(4, 80, dtype=torch.bfloat16, device=dev)          # H = 80: not a multiple of 32
    gu = torch.zeros(2, 80, 2, 64, dtype=torch.bfloat16, device=dev)
    dn = torch.zeros(2, 64, 80, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        mk.moe_prefill(x, gu, dn, torch.zeros(4, 2, device=dev),
                       torch.zeros(4, 1, dtype=torch.int32, device=dev))
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=dev)
    gu8 = torch.zeros(2, 128, 2, 64, dtype=torch.float8_e4m3fn, device=dev)   # MX codes
    with pytest.raises(NotImplementedError):
        mk.moe_prefill(x, gu8, gu8, torch.zeros(4, 2, device=dev),
                       torch.zeros(4, 1, dtype=torch.int32, device=dev))
