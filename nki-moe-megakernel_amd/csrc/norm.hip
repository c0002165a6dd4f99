// Decode RMSNorm (one row per block), optionally fused with the residual update
// that precedes it in the decoder layer.
//
//   if dsum:  x_eff = bf16(x + bf16(sum_k dsum[row, k, :]))   fp32 sum in k order,
//             written to resid_out (the new residual stream)
//   else:     x_eff = x
//   rinv  = 1 / sqrt(sum(x_eff^2) / hidden_actual + eps)      fp32
//   order 0: y = (x_eff * gamma) * rinv        rmsnorm_tkg order
//   order 1: y = (x_eff * rinv) * gamma        Qwen fused pre-attention order
//   order 2: y = gamma * bf16(x_eff * rinv)    HF RMSNorm order (final norm)
//
// The fp32 partial rows are either the K expert outputs of a token (MoE
// finalize: bf16 residual + bf16 sum) or the split-K partials of a projection
// (o_proj -> residual add).  y is written as bf16 and/or fp32, and optionally
// as MXFP8 codes + E8M0 scales of the bf16 values (a 32-element block is four
// threads' 8 elements); gamma == null skips the normalisation.  The row is held in registers (H <= 8192,
// H % 8 == 0); all global traffic is 16-byte vectors.
#include "common.h"
#include "mkd_internal.h"
#include "mx_codec.h"

namespace mkd {

constexpr int kNormThreads = 256;
constexpr int kNormMaxVec = 4;  // 4 x 8 elements x 256 threads = 8192
constexpr int kNormMaxDK = 8;   // partial rows summed per element (experts / split-K)

// VEC slices of 2048 elements per row (1, 2 or 4: the row's span, H or the MX
// padding past it); one slice keeps the kernel near 60 VGPRs, so a prefill
// pass's one-block-per-row grid is resident in one round
template <int VEC>
__global__ void __launch_bounds__(kNormThreads) rmsnorm_kernel(NormArgs a) {
  __shared__ float red[16];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int H = a.H;
  float v[VEC][8];
  u32x4_t gp[VEC];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const int i = (c * kNormThreads + tid) * 8;
    if (i < H) {
      if (a.gamma) gp[c] = ld16(a.gamma + i);
      // every load of this slice first (gamma, the partial rows, x) so their
      // latencies overlap; the partials are then summed in k order
      f32x4_t dp[kNormMaxDK][2];
      if (a.dsum) {
#pragma unroll
        for (int k = 0; k < kNormMaxDK; ++k)
          if (k < a.dK) {
            const float* p = a.dsum + row * a.ds_row + k * a.ds_k + i;
            dp[k][0] = *reinterpret_cast<const f32x4_t*>(p);
            dp[k][1] = *reinterpret_cast<const f32x4_t*>(p + 4);
          }
      }
      if (a.x_f32) {
        const float* xp = reinterpret_cast<const float*>(a.x) + (long long)row * a.ld_in + i;
        f32x4_t p = *reinterpret_cast<const f32x4_t*>(xp);
        f32x4_t q = *reinterpret_cast<const f32x4_t*>(xp + 4);
        v[c][0] = p[0]; v[c][1] = p[1]; v[c][2] = p[2]; v[c][3] = p[3];
        v[c][4] = q[0]; v[c][5] = q[1]; v[c][6] = q[2]; v[c][7] = q[3];
      } else {
        u32x4_t p = ld16(reinterpret_cast<const uint16_t*>(a.x) + (long long)row * a.ld_in + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[c][2 * j] = bf_lo(p[j]); v[c][2 * j + 1] = bf_hi(p[j]); }
      }
      if (a.dsum) {
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < kNormMaxDK; ++k)
          if (k < a.dK) {
            const f32x4_t p = dp[k][0], q = dp[k][1];
            s[0] += p[0]; s[1] += p[1]; s[2] += p[2]; s[3] += p[3];
            s[4] += q[0]; s[5] += q[1]; s[6] += q[2]; s[7] += q[3];
          }
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[c][2 * j] = rbf(v[c][2 * j] + rbf(s[2 * j]));
          v[c][2 * j + 1] = rbf(v[c][2 * j + 1] + rbf(s[2 * j + 1]));
          o[j] = pack2bf(v[c][2 * j], v[c][2 * j + 1]);
        }
        if (a.resid_out) st16(a.resid_out + (long long)row * H + i, o);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[c][j] * v[c][j];
    }
  }
  if (!a.gamma) return;                  // finalize only (uniform per block)
  ss = block_sum(ss, red);
  const float rinv = 1.0f / sqrtf(ss * a.inv_h + a.eps);
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const int i = (c * kNormThreads + tid) * 8;
    if (i < H) {
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g = (j & 1) ? bf_hi(gp[c][j >> 1]) : bf_lo(gp[c][j >> 1]);
        if (a.order == 0) y[j] = (v[c][j] * g) * rinv;
        else if (a.order == 1) y[j] = (v[c][j] * rinv) * g;
        else y[j] = g * rbf(v[c][j] * rinv);
      }
      if (a.out_bf16) {
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack2bf(y[2 * j], y[2 * j + 1]);
        st16(a.out_bf16 + (long long)row * H + i, o);
      }
      if (a.out_f32) {
        float* op = a.out_f32 + (long long)row * H + i;
        *reinterpret_cast<f32x4_t*>(op) = f32x4_t{y[0], y[1], y[2], y[3]};
        *reinterpret_cast<f32x4_t*>(op + 4) = f32x4_t{y[4], y[5], y[6], y[7]};
      }
      if (a.mx_codes) {
        // the block's amax over the four threads tid & ~3 .. +3 (H % 32 == 0:
        // all four are in range together)
        float q[8], amax = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          q[j] = rbf(y[j]);
          amax = fmaxf(amax, fabsf(q[j]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        const uint32_t sb = mx_scale_byte<MX_E4M3>(amax);
        const int sh = 127 - (int)sb;
        uint2 c = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          (j < 4 ? c.x : c.y) |= mx_encode<MX_E4M3>(ldexpf(q[j], sh)) << (8 * (j & 3));
        *reinterpret_cast<uint2*>(a.mx_codes + (long long)row * a.mx_kpad + i) = c;
        if ((tid & 3) == 0) a.mx_scales[(long long)row * (a.mx_kpad / 32) + i / 32] = (uint8_t)sb;
      }
    } else if (a.mx_codes && i < a.mx_kpad) {   // the padding blocks past H: zero codes and scales
      *reinterpret_cast<uint2*>(a.mx_codes + (long long)row * a.mx_kpad + i) = uint2{0u, 0u};
      if ((tid & 3) == 0) a.mx_scales[(long long)row * (a.mx_kpad / 32) + i / 32] = 0;
    }
  }
}

hipError_t norm_launch(NormArgs a, hipStream_t s) {
  if (a.H % 8 != 0 || a.H > kNormThreads * 8 * kNormMaxVec || a.rows <= 0 || a.hidden_actual <= 0 ||
      (a.dsum && (a.dK < 1 || a.dK > kNormMaxDK)))
    return hipErrorInvalidValue;
  if (a.mx_codes && (!a.mx_scales || !a.gamma || a.H % 32 || a.mx_kpad % 32 || a.mx_kpad < a.H ||
                     a.mx_kpad > kNormThreads * 8 * kNormMaxVec))
    return hipErrorInvalidValue;
  a.inv_h = 1.0f / (float)a.hidden_actual;
  const int span = a.mx_codes && a.mx_kpad > a.H ? a.mx_kpad : a.H;
  constexpr int kSlice = kNormThreads * 8;
  if (span <= kSlice) hipLaunchKernelGGL(rmsnorm_kernel<1>, dim3(a.rows), dim3(kNormThreads), 0, s, a);
  else if (span <= 2 * kSlice) hipLaunchKernelGGL(rmsnorm_kernel<2>, dim3(a.rows), dim3(kNormThreads), 0, s, a);
  else hipLaunchKernelGGL(rmsnorm_kernel<kNormMaxVec>, dim3(a.rows), dim3(kNormThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t rmsnorm_launch(const void* x, int x_f32, const uint16_t* gamma, uint16_t* out_bf16,
                          float* out_f32, int rows, int H, int ld_in, int hidden_actual,
                          float eps, int order, hipStream_t s) {
  NormArgs a = {};
  a.x = x; a.x_f32 = x_f32; a.ld_in = ld_in;
  a.gamma = gamma; a.out_bf16 = out_bf16; a.out_f32 = out_f32;
  a.rows = rows; a.H = H; a.hidden_actual = hidden_actual; a.eps = eps; a.order = order;
  return norm_launch(a, s);
}

}  // namespace mkd
