"""numpy restatement of OCP Microscaling (MX v1.0) quantisation (TEST INFRASTRUCTURE ONLY).

The reference quantises activations with the Neuron ISA instruction
``nisa.quantize_mx`` (nki_kernels/moe/selective_expert_mx_impl.py:143-149,
down_projection_mx_shard_H.py:74-79) whose rounding and scale choice are not
in the reference sources, so this module follows the published OCP MX v1.0
rules instead (parity unpinned against the Neuron instruction; pinned against
the spec's known answers in tests/test_oracle_mx.py):

* blocks of 32 consecutive elements along the contraction dim share one E8M0
  scale X = 2^(floor(log2(max|v|)) - emax_elem), emax_elem = 8 for E4M3
  (largest normal 448 = 1.75 * 2^8) and 2 for E2M1 (largest 6 = 1.5 * 2^2);
  the scale byte is that exponent + 127, clamped to [0, 254]; an all-zero
  block gets byte 0;
* each element is v / X rounded to nearest-even in the element format and
  saturated to the largest finite magnitude.

Codes are returned as uint8 (E4M3: s eeee mmm, bias 7; E2M1: low nibble
s ee m, bias 1).
"""
from __future__ import annotations

import numpy as np

BLOCK = 32
FORMATS = {
    # name: (exp_bits, man_bits, bias, emax_elem, max_finite)
    "e4m3": (4, 3, 7, 8, 448.0),
    "e2m1": (2, 1, 1, 2, 6.0),
}


def _floor_log2(a: np.ndarray) -> np.ndarray:
    """Exact floor(log2(a)) for a > 0 (float64 input)."""
    m, e = np.frexp(a)          # a = m * 2^e, m in [0.5, 1)
    return (e - 1).astype(np.int64)


def quantize_elements(v: np.ndarray, fmt: str) -> np.ndarray:
    """Round fp values (already divided by the block scale) to element codes."""
    eb, mb, bias, _, vmax = FORMATS[fmt]
    v = np.asarray(v, dtype=np.float64)
    sign = (np.signbit(v)).astype(np.uint8)
    a = np.abs(v)
    emin = 1 - bias                                     # smallest normal exponent
    e = np.where(a > 0, _floor_log2(np.where(a > 0, a, 1.0)), emin)
    e = np.maximum(e, emin)
    quantum = np.ldexp(1.0, (e - mb).astype(np.int64))
    q = np.round(a / quantum) * quantum                 # np.round is half-to-even
    q = np.minimum(q, vmax)
    # encode q (exactly representable now)
    qe = np.where(q > 0, _floor_log2(np.where(q > 0, q, 1.0)), emin)
    normal = q >= np.ldexp(1.0, emin)
    exp_field = np.where(normal, qe + bias, 0).astype(np.int64)
    man_field = np.where(
        normal,
        np.round((q / np.ldexp(1.0, qe) - 1.0) * (1 << mb)),
        np.round(q / np.ldexp(1.0, emin - mb)),
    ).astype(np.int64)
    code = (sign.astype(np.int64) << (eb + mb)) | (exp_field << mb) | man_field
    return code.astype(np.uint8)


def decode_elements(code: np.ndarray, fmt: str) -> np.ndarray:
    """Element codes -> float64 values (scale not applied)."""
    eb, mb, bias, _, _ = FORMATS[fmt]
    c = np.asarray(code).astype(np.int64)
    sign = (c >> (eb + mb)) & 1
    ef = (c >> mb) & ((1 << eb) - 1)
    mf = c & ((1 << mb) - 1)
    normal = ef > 0
    val = np.where(normal,
                   np.ldexp(1.0 + mf / (1 << mb), (ef - bias)),
                   np.ldexp(mf.astype(np.float64), (1 - bias - mb)))
    val = np.where(sign == 1, -val, val)
    if fmt == "e4m3":                                   # E4M3 "fn": s 1111 111 is NaN, no inf
        val = np.where((ef == 15) & (mf == 7), np.nan, val)
    return val


def quantize_mx(x: np.ndarray, fmt: str = "e4m3"):
    """Quantise along the last axis in blocks of 32.

    Returns (codes uint8 [..., K], scales uint8 [..., K/32]).
    """
    _, _, _, emax, _ = FORMATS[fmt]
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    K = x.shape[-1]
    assert K % BLOCK == 0, "K must be a multiple of 32"
    xb = x.reshape(*x.shape[:-1], K // BLOCK, BLOCK)
    amax = np.abs(xb).max(-1)
    e = np.where(amax > 0, _floor_log2(np.where(amax > 0, amax, 1.0)) - emax, -127)
    sbyte = np.clip(e + 127, 0, 254).astype(np.int64)
    scale = np.ldexp(1.0, sbyte - 127)
    codes = quantize_elements(xb / scale[..., None], fmt)
    return codes.reshape(x.shape), sbyte.astype(np.uint8)


def dequantize_mx(codes: np.ndarray, scales: np.ndarray, fmt: str = "e4m3") -> np.ndarray:
    K = codes.shape[-1]
    v = decode_elements(codes, fmt).reshape(*codes.shape[:-1], K // BLOCK, BLOCK)
    s = np.ldexp(1.0, scales.astype(np.int64) - 127)
    return (v * s[..., None]).reshape(codes.shape).astype(np.float32)
