// Shared device helpers for the gfx950 decode kernels.
//
// bf16 is handled as raw uint16 bit patterns: conversion to fp32 is a shift,
// conversion from fp32 is round-to-nearest-even (NaN -> a quiet NaN), which is
// the rounding torch's bfloat16 cast uses, so every place the reference rounds
// through bf16 gives the identical bit pattern here.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MKD_DEV __device__ __forceinline__

typedef uint16_t bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8_t;

constexpr int kWave = 64;

MKD_DEV float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
MKD_DEV float bf_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
MKD_DEV float bf_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

// fp32 -> bf16 by gfx950's v_cvt_pk_bf16_f32 (round to nearest even; checked
// bit-identical to the integer form u + 0x7fff + ((u >> 16) & 1) >> 16 for every
// non-NaN fp32 pattern; a NaN stays a NaN), one instruction per pair instead of
// six per value.
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
MKD_DEV uint32_t f2bf(float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f); }
// Round fp32 through bf16 and back.
MKD_DEV float rbf(float f) { return (float)(__bf16)f; }
MKD_DEV uint32_t pack2bf(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// Wave reductions without LDS traffic: DPP moves inside each row of 16 lanes
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: the
// gfx9 encodings 0xB1, 0x4E, 0x141, 0x140), after which every lane of a row
// holds the row's value, then the four row values are read out with readlane
// and combined in a fixed order.  The wave must be fully active.  Every lane
// gets the bit-identical result (each step combines a pair of identical
// partial results in both lanes, and the final combine is uniform).
template <int CTRL>
MKD_DEV float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
MKD_DEV float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
MKD_DEV float row_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}
MKD_DEV float row_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}
MKD_DEV float wave_sum(float v) {
  v = row_sum(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
MKD_DEV float wave_max(float v) {
  v = row_max(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024).  `red` needs 16 floats.
MKD_DEV float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < nw; ++i) s += red[i];  // fixed order -> deterministic
  return s;
}

// One 1 KiB fragment into LDS: lane l's 16 bytes from byte offset voff of the
// buffer land at dst + 16 l (buffer_load_dwordx4 ... lds; dst is wave-uniform;
// tracked by vmcnt alone).  A plain function so that the builtin stays out of
// template instantiation.
MKD_DEV void copy_frag_lds(__amdgpu_buffer_rsrc_t src, u32x4_t* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, voff,
                                           0, 0, 0);
}
MKD_DEV u32x4_t ld16(const void* p) { return *reinterpret_cast<const u32x4_t*>(p); }
MKD_DEV void st16(void* p, u32x4_t v) { *reinterpret_cast<u32x4_t*>(p) = v; }

MKD_DEV bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// 16x16x32 bf16 MFMA: A lane l holds row l%16, 8 k-values; B lane l holds
// column l%16, the same 8 k-values; D lane l holds rows 4*(l/16)+i, column l%16.
MKD_DEV f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

MKD_DEV float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// Make this wave's LDS writes visible to its own later LDS reads by other lanes.
// A wave's LDS operations complete in issue order, so no hardware wait is needed
// (an s_waitcnt 0 here would also drain every outstanding global access); the
// wavefront-scope fence only keeps the compiler from moving accesses across.
MKD_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}
