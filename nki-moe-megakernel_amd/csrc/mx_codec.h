// MX (OCP Microscaling v1.0) element and scale encoding, shared by the
// quantisation kernel (mx.hip) and the norm that quantises its own output
// rows (norm.hip): blocks of 32 elements share one E8M0 scale X =
// 2^(floor(log2 amax) - emax_elem) (byte = exponent + 127, clamped to
// [0, 254]; an all-zero block gets byte 0); each element is v / X rounded to
// nearest-even in the element format and saturated to its largest finite
// magnitude (E4M3 448, E2M1 6).
#pragma once
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

template <int FMT>
struct MxSpec;
template <>
struct MxSpec<MX_E4M3> {
  static constexpr int MB = 3, EB = 4, BIAS = 7, EMIN = -6, EMAX = 8, BPL = 32, HW = 0;
  static constexpr float VMAX = 448.0f;
};
template <>
struct MxSpec<MX_E2M1> {
  static constexpr int MB = 1, EB = 2, BIAS = 1, EMIN = 0, EMAX = 2, BPL = 16, HW = 4;
  static constexpr float VMAX = 6.0f;
};

// floor(log2(a)) for finite a > 0, fp32 subnormals included.
MKD_DEV int floor_log2_pos(float a) {
  const uint32_t b = __float_as_uint(a);
  const int e = (int)((b >> 23) & 0xffu);
  if (e) return e - 127;
  return (31 - __clz(b & 0x7fffffu)) - 149;
}

// Element code of v (already divided by the block scale): RNE, saturating.
template <int FMT>
MKD_DEV uint32_t mx_encode(float v) {
  using S = MxSpec<FMT>;
  const uint32_t sign = __float_as_uint(v) >> 31;
  const float a = fabsf(v);
  const int e = a > 0.f ? max(floor_log2_pos(a), S::EMIN) : S::EMIN;
  float q = ldexpf(rintf(ldexpf(a, S::MB - e)), e - S::MB);  // exact scalings, RNE
  q = fminf(q, S::VMAX);
  uint32_t mag = 0;
  if (q > 0.f) {
    const int qe = floor_log2_pos(q);
    if (qe >= S::EMIN)
      mag = ((uint32_t)(qe + S::BIAS) << S::MB) |
            ((__float_as_uint(q) >> (23 - S::MB)) & ((1u << S::MB) - 1u));
    else
      mag = (uint32_t)ldexpf(q, S::MB - S::EMIN);            // subnormal: q / 2^(EMIN-MB)
  }
  return (sign << (S::EB + S::MB)) | mag;
}

template <int FMT>
MKD_DEV uint32_t mx_scale_byte(float amax) {
  if (!(amax > 0.f)) return 0u;
  const int e = floor_log2_pos(amax) - MxSpec<FMT>::EMAX + 127;
  return (uint32_t)min(max(e, 0), 254);
}

}  // namespace mkd
