// QKV projection with the MoE finalize and the pre-attention RMSNorm folded in,
// for T tokens with T * K <= 4096 (the decode step at batch 1-2 of a 2048-wide model):
//
//   x    = bf16(r + bf16(sum_k dsum[t, k, :]))   (x = r when there are no partials)
//   rinv = 1 / sqrt(sum(x^2) / H_actual + eps)
//   hn   = bf16((x * rinv) * gamma)               (the Qwen fused pre-attention order,
//                                                  rmsnorm_tkg.py:318-454 / norm.hip order 1)
//   y[t][n] = sum_k hn[t][k] * W[n][k]             fp32 (qkv_tkg.py:71-363)
//
// Grid: one block per 16 output rows; 8 waves, wave w takes the contraction
// slice [w K/8, (w+1) K/8).  Every block forms x, rinv and hn for the T whole
// rows itself (the residual and the partial rows: a few tens of KB, shared
// through L2) while its weight fragments are already in flight, which removes
// the separate finalize / norm launch between the MoE of one layer and the
// QKV projection of the next; block 0 also writes x, the new residual stream.
#include "common.h"
#include "mkd_internal.h"
#include "launch_rules.h"
#include "coherent.h"

namespace mkd {

namespace {
constexpr int kQnThreads = 512;
constexpr int kQnWaves = kQnThreads / 64;
constexpr int kQnMaxDK = 8;      // partial rows per token
}  // namespace

// NF weight fragments per wave (K / 32 / 8); one 8-element row chunk per
// thread (T * K <= 4096: measured at 3-4 tokens of 2048, the partial rows of a
// second chunk cost more than the separate norm launch saves).  Two blocks per
// CU (4 waves per SIMD, <= 128 VGPRs) up to NF = 8: the grid (N / 16 blocks)
// exceeds the CU count, and a second round of blocks would double the launch's
// latency.  NF = 16 (K = 4096) keeps one block per CU, where the cap would spill.
//
// XQ: more 16-row tiles than CUs (N = 5120: 320 tiles on 256 CUs) -- one block
// per CU owns tile blockIdx.x, and two more waves take a K quarter of one of the
// remaining tiles (tile nmain + blockIdx.x / 4, quarter blockIdx.x % 4), written
// as partial quarter of those rows at y + quarter * part_stride; the head
// preparation adds the quarters in order.  Every CU then streams the same bytes,
// where a second block on a quarter of the CUs (the plain grid) made the launch
// wait for those CUs (9.1 against 6.7 us with the extra tiles left out).
template <int NF, bool XQ>
__global__ void __launch_bounds__(kQnThreads + (XQ ? 128 : 0), XQ ? 1 : (NF <= 8 ? 4 : 2))
qkv_norm_gemm_kernel(QkvNormArgs a) {
  constexpr int NWV = kQnWaves + (XQ ? 2 : 0);
  extern __shared__ __attribute__((aligned(16))) uint16_t hs[];    // [T][K] x, then hn
  __shared__ float ssr[NWV * kQkvNormMaxT];
  __shared__ __attribute__((aligned(16))) f32x4_t red[NWV][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = a.K, T = a.T, KB = K / 32;
  // the wave's tile and K slice (of eight)
  const bool xw = XQ && w >= kQnWaves;
  const int xq = blockIdx.x & 3;                              // extra waves: K quarter
  const bool xlive = xw && (int)blockIdx.x / 4 < a.n_extra;
  const int rb = xw ? a.n_main + min((int)blockIdx.x / 4, a.n_extra - 1) : (int)blockIdx.x;
  const int ks = xw ? xq * 2 + (w - kQnWaves) : w;

  // ---- 1. the row loads (residual, partial rows) go out first, then the
  // wave's weight fragments: a wave's loads complete in issue order, so the
  // norm runs while the weights stream ----
  constexpr int NC = 1;
  u32x4_t rv[NC], gm[NC];
  f32x4_t dp[kQnMaxDK][2];
  auto load_chunk = [&](int c) {
    const int i = min((c * kQnThreads + (int)threadIdx.x) * 8, T * K - 8);
    const int t = i / K, h = i - t * K;
    rv[c] = ld16(a.r + (long long)t * a.ld_r + h);
    if (a.dsum) {
#pragma unroll
      for (int k = 0; k < kQnMaxDK; ++k) {
        const float* p = a.dsum + t * a.ds_row + (long long)min(k, a.dK - 1) * a.ds_k + h;
        dp[k][0] = *reinterpret_cast<const f32x4_t*>(p);
        dp[k][1] = *reinterpret_cast<const f32x4_t*>(p + 4);
      }
    }
  };
  float ss[kQkvNormMaxT] = {0.f, 0.f, 0.f, 0.f};
  // x = bf16(r + bf16(sum of the partial rows)) of chunk c into rv[c]; sums of squares
  auto form_chunk = [&](int c) {
    const int i = (c * kQnThreads + (int)threadIdx.x) * 8;
    if (i >= T * K) return;
    const int t = i / K, h = i - t * K;
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = bf_lo(rv[c][j]);
      x[2 * j + 1] = bf_hi(rv[c][j]);
    }
    if (a.dsum) {
      float sm[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < kQnMaxDK; ++k)
        if (k < a.dK) {
          sm[0] += dp[k][0][0]; sm[1] += dp[k][0][1]; sm[2] += dp[k][0][2]; sm[3] += dp[k][0][3];
          sm[4] += dp[k][1][0]; sm[5] += dp[k][1][1]; sm[6] += dp[k][1][2]; sm[7] += dp[k][1][3];
        }
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = rbf(x[j] + rbf(sm[j]));
    }
    u32x4_t xb;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xb[j] = pack2bf(x[2 * j], x[2 * j + 1]);
      q += x[2 * j] * x[2 * j] + x[2 * j + 1] * x[2 * j + 1];
    }
    rv[c] = xb;
    if (blockIdx.x == 0 && a.resid_out) st16(a.resid_out + (long long)t * a.ld_r + h, xb);
#pragma unroll
    for (int tt = 0; tt < kQkvNormMaxT; ++tt)
      if (tt == t) ss[tt] += q;
  };
  load_chunk(0);
  // gamma before the weights too: a wave's loads complete in issue order, so
  // the norm (which needs gamma) then runs while the weight fragments stream
#pragma unroll
  for (int c = 0; c < NC; ++c)
    gm[c] = ld16(a.gamma + (min((c * kQnThreads + (int)threadIdx.x) * 8, T * K - 8) % K));
  u32x4_t wf[NF];
  const uint16_t* wp = a.w + ((long long)rb * KB + ks * NF) * 512 + lane * 8;
#pragma unroll
  for (int u = 0; u < NF; ++u)
    wf[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + u * 512));
  form_chunk(0);
  // per-token sums over the block (fixed order)
#pragma unroll
  for (int t = 0; t < kQkvNormMaxT; ++t) {
    const float v = wave_sum(ss[t]);
    if (lane == 0) ssr[w * kQkvNormMaxT + t] = v;
  }
  // (the block barriers here order LDS only -- ssr, hs, red -- so they wait for
  // LDS, not for the weight loads still in flight as __syncthreads' fence would)
  lds_barrier();
  float rinv[kQkvNormMaxT];
#pragma unroll
  for (int t = 0; t < kQkvNormMaxT; ++t) {
    float s = 0.f;
    for (int q = 0; q < kQnWaves; ++q) s += ssr[q * kQkvNormMaxT + t];
    rinv[t] = 1.0f / sqrtf(s * a.inv_h + a.eps);
  }
  // ---- 3. hn = bf16((x * rinv) * gamma) into LDS ----
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int i = (c * kQnThreads + (int)threadIdx.x) * 8;
    if (i >= T * K) break;
    const int t = i / K, h = i - t * K;
    float ri = rinv[0];
#pragma unroll
    for (int tt = 1; tt < kQkvNormMaxT; ++tt)
      if (tt == t) ri = rinv[tt];
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = pack2bf((bf_lo(rv[c][j]) * ri) * bf_lo(gm[c][j]), (bf_hi(rv[c][j]) * ri) * bf_hi(gm[c][j]));
    *reinterpret_cast<u32x4_t*>(hs + t * K + h) = o;
  }
  lds_barrier();

  // ---- 4. the wave's MFMAs (B operand: token l%16, k 8*(l/16)..+8 of the slice) ----
  const int col = lane & 15;
  const uint16_t* xrow = hs + (col < T ? col : 0) * K + ks * NF * 32 + (lane >> 4) * 8;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NF; ++u) {
    const u32x4_t xf = col < T ? *reinterpret_cast<const u32x4_t*>(xrow + u * 32) : u32x4_t{0, 0, 0, 0};
    acc = mfma16x16x32(wf[u], xf, acc);
  }
  red[w][lane] = acc;
  lds_barrier();
  // ---- 5. the 8 waves' tiles in wave order; rows 4*(l/16).. of token l%16 ----
  if (w == 0 && col < T) {
    f32x4_t s = red[0][lane];
#pragma unroll
    for (int q = 1; q < kQnWaves; ++q) s += red[q][lane];
    const int n0 = rb * 16 + (lane >> 4) * 4;
    float* y = a.y + (long long)col * a.ldy + n0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n0 + i < a.N) y[i] = s[i];
  }
  if (XQ && w == kQnWaves && xlive && col < T) {   // the extra tile's K quarter xq
    const f32x4_t s = red[kQnWaves][lane] + red[kQnWaves + 1][lane];
    const int n0 = rb * 16 + (lane >> 4) * 4;
    float* y = a.y + (long long)xq * a.part_stride + (long long)col * a.ldy + n0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (n0 + i < a.N) y[i] = s[i];
  }
}

bool qkv_norm_supported(int T, int N, int K) {
  const int nf = K / 32 / kQnWaves;
  return T >= 1 && T <= kQkvNormMaxT && N % 16 == 0 && K % (32 * kQnWaves) == 0 &&
         (nf == 1 || nf == 2 || nf == 4 || nf == 8 || nf == 16) &&
         T * K <= kQnThreads * 8;
}

int qkv_norm_extra_tiles(int N, int K, int d) { return qkv_extra_tiles_rule(N, K, d, device_cus()); }

hipError_t qkv_norm_launch(const QkvNormArgs& ain, hipStream_t s) {
  QkvNormArgs a = ain;
  if (!qkv_norm_supported(a.T, a.N, a.K) || (a.dsum && (a.dK < 1 || a.dK > kQnMaxDK)))
    return hipErrorInvalidValue;
  a.n_extra = qkv_norm_extra_tiles(a.N, a.K, a.d);
  a.n_main = a.N / 16 - a.n_extra;
  if (a.n_extra && a.part_stride < (long long)a.T * a.ldy) return hipErrorInvalidValue;
  const dim3 grid(a.n_main), block(kQnThreads + (a.n_extra ? 128 : 0));
  const size_t lds = (size_t)a.T * a.K * 2;
#define MKD_QN(NF_)                                                                          \
  case NF_:                                                                                  \
    return a.n_extra ? timed_launch(qkv_norm_gemm_kernel<NF_, true>, grid, block, lds, s, a)  \
                     : timed_launch(qkv_norm_gemm_kernel<NF_, false>, grid, block, lds, s, a);
  switch (a.K / 32 / kQnWaves) {
    MKD_QN(1) MKD_QN(2) MKD_QN(4) MKD_QN(8)
    case 16: return timed_launch(qkv_norm_gemm_kernel<16, false>, grid, block, lds, s, a);
    default: return hipErrorInvalidValue;
  }
#undef MKD_QN
}

}  // namespace mkd
