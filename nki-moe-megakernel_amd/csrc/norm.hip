// Decode RMSNorm (one row per block), optionally fused with the bf16 residual add
// that precedes it in the decoder layer.
//
//   x_eff = bf16(x + delta)            (if delta; x_eff written to resid_out)
//   rinv  = 1 / sqrt(sum(x_eff^2) / hidden_actual + eps)      fp32
//   order 0: y = (x_eff * gamma) * rinv        rmsnorm_tkg order
//   order 1: y = (x_eff * rinv) * gamma        Qwen fused pre-attention order
//   order 2: y = gamma * bf16(x_eff * rinv)    HF RMSNorm order (final norm)
//
// y is written as bf16 and/or fp32.  The row is held in registers (H <= 8192,
// H % 8 == 0); all global traffic is 16-byte vectors.
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

constexpr int kNormThreads = 256;
constexpr int kNormMaxVec = 4;  // 4 x 8 elements x 256 threads = 8192

__global__ void __launch_bounds__(kNormThreads)
rmsnorm_kernel(const void* __restrict__ x, int x_f32, const uint16_t* __restrict__ delta,
               uint16_t* __restrict__ resid_out, const uint16_t* __restrict__ gamma,
               uint16_t* __restrict__ out_bf16, float* __restrict__ out_f32, int H, int ld_in,
               float inv_h, float eps, int order) {
  __shared__ float red[16];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  float v[kNormMaxVec][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormMaxVec; ++c) {
    const int i = (c * kNormThreads + tid) * 8;
    if (i < H) {
      if (x_f32) {
        const float* xp = reinterpret_cast<const float*>(x) + (long long)row * ld_in + i;
        f32x4_t a = *reinterpret_cast<const f32x4_t*>(xp);
        f32x4_t b = *reinterpret_cast<const f32x4_t*>(xp + 4);
        v[c][0] = a[0]; v[c][1] = a[1]; v[c][2] = a[2]; v[c][3] = a[3];
        v[c][4] = b[0]; v[c][5] = b[1]; v[c][6] = b[2]; v[c][7] = b[3];
      } else {
        u32x4_t p = ld16(reinterpret_cast<const uint16_t*>(x) + (long long)row * ld_in + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[c][2 * j] = bf_lo(p[j]); v[c][2 * j + 1] = bf_hi(p[j]); }
      }
      if (delta) {
        u32x4_t p = ld16(delta + (long long)row * H + i);
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[c][2 * j] = rbf(v[c][2 * j] + bf_lo(p[j]));
          v[c][2 * j + 1] = rbf(v[c][2 * j + 1] + bf_hi(p[j]));
          o[j] = pack2bf(v[c][2 * j], v[c][2 * j + 1]);
        }
        if (resid_out) st16(resid_out + (long long)row * H + i, o);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[c][j] * v[c][j];
    }
  }
  ss = block_sum(ss, red);
  const float rinv = 1.0f / sqrtf(ss * inv_h + eps);
#pragma unroll
  for (int c = 0; c < kNormMaxVec; ++c) {
    const int i = (c * kNormThreads + tid) * 8;
    if (i < H) {
      u32x4_t gp = ld16(gamma + i);
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g = (j & 1) ? bf_hi(gp[j >> 1]) : bf_lo(gp[j >> 1]);
        if (order == 0) y[j] = (v[c][j] * g) * rinv;
        else if (order == 1) y[j] = (v[c][j] * rinv) * g;
        else y[j] = g * rbf(v[c][j] * rinv);
      }
      if (out_bf16) {
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack2bf(y[2 * j], y[2 * j + 1]);
        st16(out_bf16 + (long long)row * H + i, o);
      }
      if (out_f32) {
        float* op = out_f32 + (long long)row * H + i;
        *reinterpret_cast<f32x4_t*>(op) = f32x4_t{y[0], y[1], y[2], y[3]};
        *reinterpret_cast<f32x4_t*>(op + 4) = f32x4_t{y[4], y[5], y[6], y[7]};
      }
    }
  }
}

hipError_t rmsnorm_launch(const void* x, int x_f32, const uint16_t* delta, uint16_t* resid_out,
                          const uint16_t* gamma, uint16_t* out_bf16, float* out_f32, int rows,
                          int H, int ld_in, int hidden_actual, float eps, int order,
                          hipStream_t s) {
  if (H % 8 != 0 || H > kNormThreads * 8 * kNormMaxVec || rows <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, s, x, x_f32, delta,
                     resid_out, gamma, out_bf16, out_f32, H, ld_in, 1.0f / (float)hidden_actual,
                     eps, order);
  return hipGetLastError();
}

}  // namespace mkd
