// float8 e4m3 element codes: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no
// infinities, 0x7f / 0xff NaN (the OCP e4m3 layout, torch.float8_e4m3fn).  The
// reference's float8_e4m3 keeps the top exponent for infinities (largest
// finite 240); every value its quantisers produce (clipped to +-240) has the
// same code in both layouts.  Every e4m3 value is exactly a bf16 value.
#pragma once
#include "common.h"

namespace mkd {

constexpr float kFp8Max = 240.0f;   // largest finite value of the reference's float8_e4m3

// floor(log2(a)) for finite a > 0, fp32 subnormals included
MKD_DEV int fp8_floor_log2(float a) {
  const uint32_t b = __float_as_uint(a);
  const int e = (int)((b >> 23) & 0xffu);
  if (e) return e - 127;
  return (31 - __clz(b & 0x7fffffu)) - 149;
}

// e4m3 code of v, round to nearest even, saturating at 448 (callers clip to
// +-240 first): the quantum at |v| is 2^(max(floor(log2|v|), -6) - 3).
MKD_DEV uint32_t e4m3_encode(float v) {
  const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  if (!(a > 0.f)) return sign;
  const int e = max(fp8_floor_log2(a), -6);
  const float q = fminf(ldexpf(rintf(ldexpf(a, 3 - e)), e - 3), 448.0f);
  if (q == 0.f) return sign;
  const int qe = fp8_floor_log2(q);
  const uint32_t mag = qe >= -6 ? (((uint32_t)(qe + 7) << 3) | ((__float_as_uint(q) >> 20) & 7u))
                                : (uint32_t)ldexpf(q, 9);   // subnormal: q / 2^-9
  return sign | mag;
}

MKD_DEV float e4m3_decode(uint32_t c) {
  const uint32_t e = (c >> 3) & 15u, m = c & 7u;
  if ((c & 0x7fu) == 0x7fu) return __uint_as_float(0x7fc00000u);
  const float mag = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
  return (c & 0x80u) ? -mag : mag;
}

// the bf16 bits of code c (exact)
MKD_DEV uint32_t e4m3_to_bf16(uint32_t c) { return __float_as_uint(e4m3_decode(c)) >> 16; }

// e4m3(clip(x * s, +-240)) -- the reference's fp8 quantisers (attention_block_tkg.py:
// 1694-1737 for the KV cache; qkv_tkg.py:849-862 and output_projection_tkg.py:549-566
// with s = 1 / input scale for static activations)
MKD_DEV uint32_t fp8_quant(float x, float s) {
  return e4m3_encode(fminf(fmaxf(x * s, -kFp8Max), kFp8Max));
}

}  // namespace mkd
