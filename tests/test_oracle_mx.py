"""CPU pins of the MX (OCP Microscaling v1.0) oracle, oracle/mx.py.

The reference quantises with the Neuron instruction nisa.quantize_mx
(selective_expert_mx_impl.py:143-149), whose rounding is not in its sources, so
the oracle follows the OCP MX v1.0 rules; these tests pin it against an
independent implementation of the element formats (torch's float8_e4m3fn and
float8_e8m0fnu casts), brute force over the E2M1 value set, and known answers.
"""
import numpy as np
import pytest
import torch

from oracle import mx

E2M1_VALUES = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_e4m3_decode_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    finite = (codes & 0x7F) != 0x7F                      # 0x7f / 0xff are NaN
    ours = mx.decode_elements(codes[finite], "e4m3")
    theirs = torch.from_numpy(codes[finite].copy()).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(ours, theirs.astype(np.float64))


def test_e4m3_rounding_matches_torch_rne_with_saturation():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(20000) * 100,                  # normals, some saturating
        rng.uniform(-2 ** -6, 2 ** -6, 5000),              # subnormal range
        np.array([0.0, -0.0, 448.0, 464.0, 470.0, -1000.0, 2 ** -10, 3 * 2 ** -11]),
    ]).astype(np.float32)
    ours = mx.quantize_elements(v, "e4m3")
    theirs = torch.from_numpy(np.clip(v, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_e2m1_rounding_is_nearest_even_by_brute_force():
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.uniform(-8, 8, 5000), np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, -5.0])])
    codes = mx.quantize_elements(v, "e2m1")
    mags = np.array(E2M1_VALUES)
    for x, c in zip(v, codes):
        a = min(abs(x), 6.0)
        d = np.abs(mags - a)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:                                  # tie: even mantissa (code bit 0 clear)
            best = [b for b in best if b % 2 == 0]
        assert (c & 7) == best[0], (x, c)
        if (c & 7) != 0:
            assert (c >> 3) == (1 if x < 0 else 0)


def test_scale_known_answers():
    blk = np.zeros((1, 32), np.float32)
    _, s = mx.quantize_mx(blk, "e4m3")
    assert s[0, 0] == 0                                    # all-zero block
    for amax, want8, want4 in [(1.0, 127 - 8, 127 - 2), (448.0, 127, 127 + 6), (0.75, 126 - 8, 126 - 2),
                               (2.0 ** -20, 107 - 8, 107 - 2)]:
        blk = np.zeros((1, 32), np.float32)
        blk[0, 5] = -amax
        assert mx.quantize_mx(blk, "e4m3")[1][0, 0] == want8
        assert mx.quantize_mx(blk, "e2m1")[1][0, 0] == want4


def test_scale_bytes_decode_like_torch_e8m0():
    b = np.arange(0, 255, dtype=np.uint8)
    theirs = torch.from_numpy(b.copy()).view(torch.float8_e8m0fnu).float().numpy().astype(np.float64)
    np.testing.assert_array_equal(np.ldexp(1.0, b.astype(np.int64) - 127), theirs)


@pytest.mark.parametrize("fmt", ["e4m3", "e2m1"])
def test_representable_blocks_round_trip_exactly(fmt):
    rng = np.random.default_rng(2)
    vals = mx.decode_elements(np.arange(256 if fmt == "e4m3" else 16, dtype=np.uint8), fmt)
    vals = vals[np.isfinite(vals)]
    x = rng.choice(vals, size=(8, 128)).astype(np.float32)
    x[:, ::32] = vals.max()                                # block max fixes the scale at 2^0
    x *= 2.0 ** rng.integers(-6, 6, size=(8, 1))
    codes, scales = mx.quantize_mx(x, fmt)
    np.testing.assert_array_equal(mx.dequantize_mx(codes, scales, fmt), x)


@pytest.mark.parametrize("fmt,rel,emax,vmax", [("e4m3", 2 ** -4, 8, 448.0), ("e2m1", 0.25, 2, 6.0)])
def test_quantisation_error_bound(fmt, rel, emax, vmax):
    """|x - deq(q(x))| <= half a quantum of the block's top binade, or the
    saturation loss amax - vmax*X when amax/X exceeds the largest element."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    codes, scales = mx.quantize_mx(x, fmt)
    y = mx.dequantize_mx(codes, scales, fmt)
    amax = np.abs(x.reshape(16, 8, 32)).max(-1, keepdims=True).astype(np.float64)
    X = np.ldexp(1.0, np.floor(np.log2(amax)).astype(np.int64) - emax)
    np.testing.assert_array_equal(np.ldexp(1.0, scales.astype(np.int64) - 127), X[..., 0])
    bound = np.maximum(rel * amax, amax - vmax * X)
    err = np.abs((y - x).reshape(16, 8, 32))
    assert (err <= bound + 1e-12).all()
    assert (np.abs(y) <= vmax * X.repeat(32, -1).reshape(y.shape)).all()


def _moe_case(seed, T=3, E=4, K=2, H=256, I=64):
    from oracle import ref
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gu = torch.from_numpy(mx.dequantize_mx(*mx.quantize_mx((0.05 * torch.randn(E, 2 * I, H, generator=g)).numpy(), "e4m3"), "e4m3"))
    dn = torch.from_numpy(mx.dequantize_mx(*mx.quantize_mx((0.05 * torch.randn(E, H, I, generator=g)).numpy(), "e4m3"), "e4m3"))
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    aff = torch.zeros(T, E).scatter_(1, idx, torch.rand(T, K, generator=g))
    return ref, x, gu, dn, idx, aff


def test_moe_mx_oracle_matches_bf16_oracle_within_activation_quantisation():
    """Same dequantised weights: the MX flow differs from the (HF-pinned) bf16 moe_tkg
    only by the MXFP8 rounding of the two activations."""
    ref, x, gu, dn, idx, aff = _moe_case(0)
    I = gu.shape[1] // 2
    y_mx = ref.moe_tkg_mx(x, gu, dn, aff, idx, scaling_mode="post")
    # bf16 oracle layouts: gate_up [E, H, 2, I], down [E, I, H]
    gu_ref = torch.stack([gu[:, :I], gu[:, I:]], 1).permute(0, 3, 1, 2)
    y_bf = ref.moe_tkg(x, gu_ref, dn.transpose(1, 2), aff, idx, scaling_mode="post")
    rel = ((y_mx - y_bf).abs().max() / y_bf.abs().max()).item()
    assert 1e-4 < rel < 5e-2, rel


def test_moe_mx_oracle_exact_for_representable_activations():
    """One expert, identity-like down projection and MX-representable x: the only
    remaining rounding is the intermediate's, which the check reproduces by hand."""
    from oracle import ref
    H = I = 64
    x = torch.zeros(1, H)
    # E4M3 values whose block maximum (1.75 * 2^2) keeps every element unsaturated
    codes = np.minimum(np.arange(0x30, 0x50, dtype=np.uint8), 0x4E)
    x[0, :32] = torch.tensor(mx.decode_elements(codes, "e4m3"), dtype=torch.float32)
    x[0, 32:] = -x[0, :32]
    gu = torch.zeros(1, 2 * I, H)
    gu[0, :I] = torch.eye(H)                     # g = x
    gu[0, I:] = torch.eye(H)                     # u = x
    dn = torch.eye(H)[None]                      # y = h
    c0, s0 = mx.quantize_mx(x.numpy(), "e4m3")
    np.testing.assert_array_equal(mx.dequantize_mx(c0, s0, "e4m3"), x.numpy())   # x representable
    y = ref.moe_tkg_mx(x.to(torch.bfloat16), gu, dn, torch.ones(1, 1), torch.zeros(1, 1, dtype=torch.long))
    h = (x[0] * torch.sigmoid(x[0]) * x[0]).to(torch.bfloat16).float()
    c, s = mx.quantize_mx(h[None].numpy(), "e4m3")
    np.testing.assert_array_equal(y[0].numpy(), mx.dequantize_mx(c, s, "e4m3")[0])
