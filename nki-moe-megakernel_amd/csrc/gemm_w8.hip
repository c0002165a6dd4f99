// Dense projections with float8 e4m3 weights and static activation
// quantisation: the STATIC paths of the QKV projection (qkv_tkg.py:289-305,
// :849-862, :946-986, :1094-1098) and the output projection
// (output_projection_tkg.py:185-200, :549-566), as attention_block_tkg passes
// them through (quantization_type_qkv / _out, attention_block_tkg.py:94-97,
// :124-127, :179-183, :225-229).
//
//   x_q[t, k] = e4m3(clip(x[t, k] * (1 / s_in), +-240))
//   y[t, n]   = (sum_k x_q[t, k] W[n, k]) * (s_w[seg(n)] * s_in) + bias[n]
//
// seg(n) picks the Q / K / V weight scale of the QKV projection (columns below
// seg0, below seg1, the rest); the output projection has one segment.
//
// The weights stay e4m3 in HBM (half the bytes of bf16), frag-packed: fragment
// (rb, kb) is 64 lanes x 8 bytes, lane l holding row 16 rb + l%16 at
// k = 32 kb + 8 (l/16) .. +8 -- one v_mfma_f32_16x16x32_bf16 A operand once each
// byte is widened to its bf16 value (exact: every e4m3 value is a bf16 value).
// The activations are quantised once into bf16-valued e4m3 numbers by
// w8_quant_kernel, so the MFMA multiplies two e4m3 values exactly and
// accumulates in fp32 -- the arithmetic of an fp8 x fp8 matrix multiply.
//
// gemm_w8_kernel: block = 4 waves on one 16-row block, each wave a quarter of K
// (its weight fragments all in flight before the MFMAs), every token tile of
// the T <= 128 tokens per fragment; the wave partials are summed in LDS in wave
// order and the epilogue applies the scale and bias.
#include "common.h"
#include "fp8.h"
#include "mkd_internal.h"
#include "gemm_epi.h"

namespace mkd {

namespace {
constexpr int kW8MaxF = 8;   // weight fragments in flight per wave per batch
}

// x [T, K] bf16 -> x_q [T, K] bf16 bits of e4m3(clip(x / s_in, +-240)); 8 per thread
__global__ void __launch_bounds__(256) w8_quant_kernel(const uint16_t* __restrict__ x, int ldx, int T,
                                                       int K, const float* __restrict__ in_scale,
                                                       uint16_t* __restrict__ xq) {
  const long long i = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i >= (long long)T * K) return;
  const int t = (int)(i / K), k = (int)(i % K);
  const float inv = 1.0f / in_scale[0];
  const u32x4_t v = ld16(x + (long long)t * ldx + k);
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t lo = e4m3_to_bf16(fp8_quant(bf2f(v[e] & 0xffffu), inv));
    const uint32_t hi = e4m3_to_bf16(fp8_quant(bf2f(v[e] >> 16), inv));
    o[e] = lo | (hi << 16);
  }
  st16(xq + i, o);
}

// G x W [K, N] e4m3 codes (row-major, the reference's [in, out] layout) ->
// frag packed [G][N/16][K/32][64][8]; one thread per lane-fragment (8 bytes).
__global__ void __launch_bounds__(256) w8_pack_kernel(const uint8_t* __restrict__ src, int G, int N,
                                                      int K, uint8_t* __restrict__ dst) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  const int KB = K / 32;
  const long long per = (long long)(N / 16) * KB * 64;
  if (i >= per * G) return;
  const long long gi = i / per, li = i % per;
  const int l = (int)(li % 64);
  const long long fk = li / 64;
  const int kb = (int)(fk % KB), rb = (int)(fk / KB);
  src += gi * (long long)K * N;
  const int n = rb * 16 + (l & 15), k0 = kb * 32 + (l >> 4) * 8;
  uint32_t w0 = 0, w1 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w0 |= (uint32_t)src[(long long)(k0 + j) * N + n] << (8 * j);
    w1 |= (uint32_t)src[(long long)(k0 + 4 + j) * N + n] << (8 * j);
  }
  *reinterpret_cast<uint2*>(dst + i * 8) = uint2{w0, w1};
}

// 8 e4m3 codes -> the A operand (8 bf16)
MKD_DEV u32x4_t w8_widen(uint2 c) {
  u32x4_t o;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t v = e ? c.y : c.x;
    o[2 * e] = e4m3_to_bf16(v & 0xffu) | (e4m3_to_bf16((v >> 8) & 0xffu) << 16);
    o[2 * e + 1] = e4m3_to_bf16((v >> 16) & 0xffu) | (e4m3_to_bf16(v >> 24) << 16);
  }
  return o;
}

template <int TT>
__global__ void __launch_bounds__(256) gemm_w8_kernel(W8Args a) {
  __shared__ f32x4_t red[4][TT][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int rb = blockIdx.x, KB = a.K / 32;
  const int kb0 = w * KB / 4, kb1 = (w + 1) * KB / 4;
  const uint8_t* wp = a.w + ((long long)rb * KB) * 512 + lane * 8;
  const int c = lane & 15;
  f32x4_t acc[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) acc[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int f0 = kb0; f0 < kb1; f0 += kW8MaxF) {
    uint2 wf[kW8MaxF];
#pragma unroll
    for (int u = 0; u < kW8MaxF; ++u)
      wf[u] = *reinterpret_cast<const uint2*>(wp + (long long)min(f0 + u, kb1 - 1) * 512);
#pragma unroll
    for (int u = 0; u < kW8MaxF; ++u) {
      if (f0 + u >= kb1) break;
      const u32x4_t av = w8_widen(wf[u]);
      const int k = (f0 + u) * 32 + (lane >> 4) * 8;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int t = tt * 16 + c;
        const u32x4_t xv = t < a.T ? ld16(a.x + (long long)t * a.ldx + k) : u32x4_t{0u, 0u, 0u, 0u};
        acc[tt] = mfma16x16x32(av, xv, acc[tt]);
      }
    }
  }
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) red[w][tt][lane] = acc[tt];
  __syncthreads();
  // wave q sums token tiles q, q + 4, ..; D lane l: rows 4 (l/16) + i of token l%16
  for (int tt = w; tt < TT; tt += 4) {
    const f32x4_t v = ((red[0][tt][lane] + red[1][tt][lane]) + red[2][tt][lane]) + red[3][tt][lane];
    const int t = tt * 16 + c;
    if (t >= a.T) continue;
    const float sin_ = a.in_scale[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = rb * 16 + (lane >> 4) * 4 + i;
      if (n >= a.N) continue;
      const int seg = n < a.seg0 ? 0 : (n < a.seg1 ? 1 : 2);
      float o = v[i] * (a.w_scale[seg] * sin_);
      if (a.bias) o += bf2f(a.bias[n]);
      if (a.y_f32) a.y_f32[(long long)t * a.ldy + n] = o;
      else a.y_bf16[(long long)t * a.ldy + n] = (uint16_t)f2bf(o);
    }
  }
}

hipError_t w8_pack_launch(const uint8_t* src, int G, int N, int K, uint8_t* dst, hipStream_t s) {
  if (N % 16 || K % 32 || N <= 0 || K <= 0 || G <= 0) return hipErrorInvalidValue;
  const long long n = (long long)G * (N / 16) * (K / 32) * 64;
  hipLaunchKernelGGL(w8_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, G, N, K, dst);
  return hipGetLastError();
}

hipError_t gemm_w8_launch(const W8Args& a, uint16_t* xq, hipStream_t s) {
  if (a.N % 16 || a.K % 32 || a.T <= 0 || a.T > 128 || a.ldx % 8 || !a.x_bf16 || !a.w ||
      !a.w_scale || !a.in_scale || !xq || (!a.y_f32 == !a.y_bf16))
    return hipErrorInvalidValue;
  const long long nx = (long long)a.T * a.K;
  hipLaunchKernelGGL(w8_quant_kernel, dim3((unsigned)((nx / 8 + 255) / 256)), dim3(256), 0, s, a.x_bf16,
                     a.ldx, a.T, a.K, a.in_scale, xq);
  if (hipError_t e = hipGetLastError()) return e;
  W8Args b = a;
  b.x = xq;
  b.ldx = a.K;
  const dim3 grid(a.N / 16);
  const int tt = (a.T + 15) / 16;
  if (tt == 1) hipLaunchKernelGGL((gemm_w8_kernel<1>), grid, dim3(256), 0, s, b);
  else if (tt == 2) hipLaunchKernelGGL((gemm_w8_kernel<2>), grid, dim3(256), 0, s, b);
  else if (tt <= 4) hipLaunchKernelGGL((gemm_w8_kernel<4>), grid, dim3(256), 0, s, b);
  else hipLaunchKernelGGL((gemm_w8_kernel<8>), grid, dim3(256), 0, s, b);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Routed experts with e4m3 weights (moe_tkg's FP8 ROW and STATIC modes,
// moe_tkg.py:119-131, 296-328; mlp_tkg_gate_up_projection.py:188-275, 847-900;
// mlp_tkg_down_projection.py:418-560): bf16 activations times e4m3 weights,
// fp32 accumulation, each output column dequantised by its weight scale
// (col_scale [E][N]: the per-column ROW scales, or a STATIC expert's scalar per
// gate / up half) before the bias.  The reference's input scales of these
// modes select the mode only; its expert kernels do not quantise the
// activations.
//
// Block (i-block ib, routed group g), 4 waves over K quarters, token tiles of
// 16 of the group in turn.  Gate / up (W8_SWIGLU): the block owns gate rows
// 16 ib .. +16 and the matching up rows I + 16 ib .., so one lane holds the
// gate and up values of an (i, token) pair; h = act(gate) * up (bf16) goes to
// the pair's slot row.  Down (W8_SCALE): rows 16 ib .. +16 of H, times the
// pair's affinity, fp32 into the slot row (moe_finalize sums the K slots).
template <int EPI>
__global__ void __launch_bounds__(256) gemm_w8_grouped_kernel(W8GroupArgs a) {
  constexpr int RB = EPI == W8_SWIGLU ? 2 : 1;
  __shared__ f32x4_t red[4][RB][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ib = blockIdx.x, g = blockIdx.y;
  if (g >= *a.g.n_groups) return;
  const int e = a.g.grp_expert[g], count = a.g.grp_count[g], base = a.g.grp_offset[g];
  const int KB = a.K / 32, kb0 = w * KB / 4, kb1 = (w + 1) * KB / 4;
  const int rbs[2] = {ib, EPI == W8_SWIGLU ? ib + a.N / 32 : ib};   // gate / up row blocks
  const uint8_t* we = a.w + (long long)e * a.w_group_stride;
  const int c = lane & 15;
  for (int t0 = 0; t0 < count; t0 += 16) {
    if (t0) __syncthreads();               // the previous tile's reduction buffer is free
    const int p = t0 + c < count ? base + t0 + c : -1;
    const int xr = p >= 0 ? a.x_row[p] : 0;
    const uint16_t* xp = a.x + (long long)xr * a.ldx + (lane >> 4) * 8;
    f32x4_t acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int f0 = kb0; f0 < kb1; f0 += kW8MaxF) {
      uint2 wf[RB][kW8MaxF];
      u32x4_t xv[kW8MaxF];
#pragma unroll
      for (int u = 0; u < kW8MaxF; ++u) {
        const int kb = min(f0 + u, kb1 - 1);
#pragma unroll
        for (int r = 0; r < RB; ++r)
          wf[r][u] = *reinterpret_cast<const uint2*>(we + ((long long)rbs[r] * KB + kb) * 512 + lane * 8);
        xv[u] = ld16(xp + kb * 32);
      }
#pragma unroll
      for (int u = 0; u < kW8MaxF; ++u) {
        if (f0 + u >= kb1) break;
        const u32x4_t xu = p >= 0 ? xv[u] : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r] = mfma16x16x32(w8_widen(wf[r][u]), xu, acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) red[w][r][lane] = acc[r];
    __syncthreads();
    if (w == 0 && p >= 0) {
      const int slot = a.out_row[p];
      f32x4_t v[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) v[r] = ((red[0][r][lane] + red[1][r][lane]) + red[2][r][lane]) + red[3][r][lane];
      const float* cs = a.col_scale + (long long)e * a.N;
      const uint16_t* bp = a.bias ? a.bias + (long long)e * a.N : nullptr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = ib * 16 + (lane >> 4) * 4 + i;   // gate / down row (up: n + N / 2)
        if constexpr (EPI == W8_SWIGLU) {
          const int I = a.N / 2;
          const float gv = v[0][i] * cs[n] + (bp ? bf2f(bp[n]) : 0.f);
          const float uv = v[1][i] * cs[I + n] + (bp ? bf2f(bp[I + n]) : 0.f);
          a.h[(long long)slot * a.ldy + n] = (uint16_t)f2bf(swiglu_value(a.act, gv, uv));
        } else {
          const float sc = a.pair_scale ? a.pair_scale[slot] : 1.0f;
          a.y[(long long)slot * a.ldy + n] = (v[0][i] * cs[n] + (bp ? bf2f(bp[n]) : 0.f)) * sc;
        }
      }
    }
  }
}

hipError_t gemm_w8_grouped_launch(const W8GroupArgs& a, int epi, int groups_max, hipStream_t s) {
  if (a.K % 32 || a.N % 16 || (epi == W8_SWIGLU && a.N % 32) || groups_max <= 0 || !a.w ||
      !a.x || !a.col_scale || !a.g.n_groups || !a.x_row || !a.out_row || (a.ldx & 7))
    return hipErrorInvalidValue;
  if (epi == W8_SWIGLU) {
    if (!a.h) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_w8_grouped_kernel<W8_SWIGLU>, dim3(a.N / 32, groups_max), dim3(256), 0, s, a);
  } else {
    if (!a.y) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_w8_grouped_kernel<W8_SCALE>, dim3(a.N / 16, groups_max), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace mkd
