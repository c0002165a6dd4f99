// Dense decode projection for 17..128 tokens (QKV and output projections at
// batch 17-128): Y[t, n] = sum_k X[t, k] * W[n, k] in fp32 split-K partials
// (qkv_tkg.py:71-363, output_projection_tkg.py:66-265 -- the same contraction as
// the weight-streaming GEMM in gemm.hip, shaped for a wider token dimension).
//
// At these token counts the weight-streaming GEMM (one 16-row block per launch
// block, waves splitting K) reads the activation tile of every token for every
// weight fragment: at 64 tokens that is 4 bytes of activations per weight byte,
// all through the issuing CU's vector L1 (64 B/clk).  Here a block of 4 waves
// owns a K slice of KS and 4 * RBW row blocks: the slice's activations
// X[0:T, k0:k0+KS] are copied to LDS once (in MFMA B-operand order, 16 bytes per
// lane per fragment) and every wave reads them from there while streaming only
// its own row blocks' weight fragments (frag layout, one 1 KiB
// v_mfma_f32_16x16x32_bf16 A operand per fragment).  Waves own disjoint rows,
// so there is no cross-wave reduction; block (row group, kb) writes partial kb
// of the K split to y + kb * part_stride (bias in partial 0), which the
// consumer (attention head preparation, post-attention norm) adds in order.
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

namespace {
constexpr int kMidWaves = 4;
// the largest divisor of n that is <= cap (the staging batch)
constexpr int batch_of(int n, int cap) {
  int b = n < cap ? n : cap;
  while (n % b) --b;
  return b;
}
}

// TT token tiles of 16; RBW row blocks per wave; NF = KS / 32 weight fragments
// per row block (all issued before the first MFMA).  XF32: fp32 activations (the
// router's normalised rows) carried as a bf16 hi + lo pair, two LDS slices and
// two MFMAs per fragment (~2^-16 relative, as the weight-streaming GEMM).
template <int TT, int RBW, int NF, bool XF32>
__global__ void __launch_bounds__(256) gemm_mid_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4_t xs[];    // [hi/lo][TT][NF][64]
  // grid z: chunks of 128 tokens (more than 128 tokens), each a call of its own
  // on rows z * 128 .. of x and of every partial
  if (gridDim.z > 1) {
    const int t0 = (int)blockIdx.z * 128;
    a.x = static_cast<const char*>(a.x) + (long long)t0 * a.ldx * (XF32 ? 4 : 2);
    a.y = static_cast<char*>(a.y) + (long long)t0 * a.ldy * 4;
    a.T = min(a.T - t0, 128);
  }
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KB = a.K / 32;
  const int kb = blockIdx.y;                      // K slice
  const int kf0 = kb * NF;                        // first 32-wide k block of the slice
  const int NRB = (a.N + 15) / 16;

  // ---- weights of the wave's row blocks: every fragment in flight at once ----
  u32x4_t wf[RBW][NF];
#pragma unroll
  for (int r = 0; r < RBW; ++r) {
    const int rb = min((blockIdx.x * kMidWaves * RBW) + r * kMidWaves + w, NRB - 1);
    const uint16_t* wp = a.w + ((long long)rb * KB + kf0) * 512 + lane * 8;
#pragma unroll
    for (int f = 0; f < NF; ++f)
      wf[r][f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp + f * 512));
  }

  // ---- the activation slice into LDS in B-operand order: chunk c = (tile tt,
  // fragment f, lane l) holds token tt*16 + l%16, k = (kf0 + f)*32 + (l/16)*8 .. +8 ----
  // A thread's chunks are c = tid + 256 j; each batch of BJ chunks has all its
  // loads in flight before the first LDS store (absent tokens read row 0 and
  // store zeros).
  constexpr int NCH = TT * NF * 64;
  constexpr int PJ = NCH / 256;                    // chunks per thread
  constexpr int BJ = batch_of(PJ, XF32 ? 8 : 16);
  static_assert(NCH % 256 == 0 && PJ % BJ == 0, "chunk split");
#pragma unroll
  for (int j0 = 0; j0 < PJ; j0 += BJ) {
    u32x4_t v[BJ][XF32 ? 2 : 1];
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int c = threadIdx.x + (j0 + j) * 256;
      const int l = c & 63, f = (c >> 6) % NF, tt = c / (64 * NF);
      const int t = tt * 16 + (l & 15);
      const long long off = (long long)(t < a.T ? t : 0) * a.ldx + (long long)(kf0 + f) * 32 + (l >> 4) * 8;
      if constexpr (XF32) {
        const float* xp = static_cast<const float*>(a.x) + off;
        v[j][0] = ld16(xp);
        v[j][1] = ld16(xp + 4);
      } else {
        v[j][0] = ld16(static_cast<const uint16_t*>(a.x) + off);
      }
    }
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
      const int c = threadIdx.x + (j0 + j) * 256;
      const bool live = (c / (64 * NF)) * 16 + (c & 15) < a.T;
      if constexpr (XF32) {
        const float x8[8] = {__uint_as_float(v[j][0][0]), __uint_as_float(v[j][0][1]),
                             __uint_as_float(v[j][0][2]), __uint_as_float(v[j][0][3]),
                             __uint_as_float(v[j][1][0]), __uint_as_float(v[j][1][1]),
                             __uint_as_float(v[j][1][2]), __uint_as_float(v[j][1][3])};
        u32x4_t hi, lo;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t h0 = f2bf(x8[2 * q]), h1 = f2bf(x8[2 * q + 1]);
          hi[q] = h0 | (h1 << 16);
          lo[q] = f2bf(x8[2 * q] - bf2f(h0)) | (f2bf(x8[2 * q + 1] - bf2f(h1)) << 16);
        }
        xs[c] = live ? hi : u32x4_t{0u, 0u, 0u, 0u};
        xs[NCH + c] = live ? lo : u32x4_t{0u, 0u, 0u, 0u};
      } else {
        xs[c] = live ? v[j][0] : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  }
  __syncthreads();

  // ---- MFMAs: acc[r][tt] = rows of row block r x tokens of tile tt ----
  f32x4_t acc[RBW][TT];
#pragma unroll
  for (int r = 0; r < RBW; ++r)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[r][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    u32x4_t xf[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) xf[tt] = xs[(tt * NF + f) * 64 + lane];
#pragma unroll
    for (int r = 0; r < RBW; ++r)
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) acc[r][tt] = mfma16x16x32(wf[r][f], xf[tt], acc[r][tt]);
    if constexpr (XF32) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) xf[tt] = xs[NCH + (tt * NF + f) * 64 + lane];
#pragma unroll
      for (int r = 0; r < RBW; ++r)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) acc[r][tt] = mfma16x16x32(wf[r][f], xf[tt], acc[r][tt]);
    }
  }

  // ---- partial kb: lane l holds rows 4*(l/16)+i of its row block, token l%16 ----
  float* yb = static_cast<float*>(a.y) + (long long)kb * a.part_stride;
#pragma unroll
  for (int r = 0; r < RBW; ++r) {
    const int rb = (blockIdx.x * kMidWaves * RBW) + r * kMidWaves + w;
    if (rb >= NRB) continue;
    const int n0 = rb * 16 + (lane >> 4) * 4;
    float bb[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias && kb == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) bb[i] = (n0 + i < a.N) ? bf2f(a.bias[n0 + i]) : 0.f;
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = tt * 16 + (lane & 15);
      if (t >= a.T) continue;
      float* y = yb + (long long)t * a.ldy + n0;
      if (n0 + 3 < a.N && (a.ldy & 3) == 0) {
        *reinterpret_cast<f32x4_t*>(y) = f32x4_t{acc[r][tt][0] + bb[0], acc[r][tt][1] + bb[1],
                                                 acc[r][tt][2] + bb[2], acc[r][tt][3] + bb[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n0 + i < a.N) y[i] = acc[r][tt][i] + bb[i];
      }
    }
  }
}

// Fragments per K slice with a kernel instantiation.
static bool mid_nf_ok(int nf) { return nf == 4 || nf == 6 || nf == 8 || nf == 12 || nf == 16; }

// Row blocks per wave: 2 for narrow outputs (the router: 128 rows make one
// block of 4 waves), else 1.
static int mid_rbw(int N) { return N <= 256 ? 2 : 1; }

// K split for N output rows, K contraction and T tokens: among the slice counts
// (a power of two <= max_parts cutting K / 32 into NF whole fragments, NF
// instantiated), the one with the least work on the busiest CU -- rounds of
// blocks over the 256 CUs times the work of a block, ceil(blocks / 256) / kg --
// the fewest slices on a tie; 0 when no split fits.  (A grid of 320 blocks left
// a quarter of the CUs with two blocks and the launch waiting for them.)
int gemm_mid_kgrid(int N, int K, int T, int max_parts) {
  if (T < 17 || T > 128 || K % 32 || N <= 0) return 0;
  constexpr int kCUs = 256;
  const int rbw = mid_rbw(N);
  const int KB = K / 32, groups = ((N + 15) / 16 + kMidWaves * rbw - 1) / (kMidWaves * rbw);
  int best = 0;
  double best_load = 1e30;
  for (int kg = 1; kg <= max_parts && kg <= 16 && KB % kg == 0; kg *= 2) {
    if (!mid_nf_ok(KB / kg)) continue;
    const double load = (double)((groups * kg + kCUs - 1) / kCUs) / kg;
    if (load < best_load - 1e-9) {
      best_load = load;
      best = kg;
    }
  }
  return best;
}

// The same contraction for very tall outputs (the vocabulary projection at
// 17..128 tokens): each block owns 4 * RBW row blocks over the WHOLE K range,
// looping over K slices of NF fragments -- the slice's activations staged in
// LDS, the wave's weight fragments streamed -- and writes finished fp32 rows
// (bias added), so there are no K-split partials to write and read back.  One
// 16-row block per launch block instead (the weight-streaming GEMM) reads the
// activations of every token for every weight fragment through the CU:
// 4 bytes per weight byte at 64 tokens.
template <int TT, int RBW, int NF>
__global__ void __launch_bounds__(256) gemm_kloop_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4_t xs[];    // [TT][NF][64]
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KB = a.K / 32, NRB = (a.N + 15) / 16, nsl = KB / NF;
  constexpr int NCH = TT * NF * 64;
  constexpr int PJ = NCH / 256;                    // staging chunks per thread
  static_assert(NCH % 256 == 0, "chunk split");
  f32x4_t acc[RBW][TT];
#pragma unroll
  for (int r = 0; r < RBW; ++r)
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[r][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* wp[RBW];
#pragma unroll
  for (int r = 0; r < RBW; ++r) {
    const int rb = min(blockIdx.x * kMidWaves * RBW + r * kMidWaves + w, NRB - 1);
    wp[r] = a.w + (long long)rb * KB * 512 + lane * 8;
  }
  for (int sl = 0; sl < nsl; ++sl) {
    const int kf0 = sl * NF;
    // the slice's weight fragments, then its activation chunks (L2-resident)
    u32x4_t wf[RBW][NF];
#pragma unroll
    for (int r = 0; r < RBW; ++r)
#pragma unroll
      for (int f = 0; f < NF; ++f)
        wf[r][f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp[r] + (kf0 + f) * 512));
    u32x4_t v[PJ];
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int c = threadIdx.x + j * 256;
      const int l = c & 63, f = (c >> 6) % NF, tt = c / (64 * NF);
      const int t = tt * 16 + (l & 15);
      v[j] = ld16(static_cast<const uint16_t*>(a.x) + (long long)(t < a.T ? t : 0) * a.ldx +
                  (long long)(kf0 + f) * 32 + (l >> 4) * 8);
    }
    __syncthreads();                               // the previous slice's reads of xs are done
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int c = threadIdx.x + j * 256;
      const bool live = (c / (64 * NF)) * 16 + (c & 15) < a.T;
      xs[c] = live ? v[j] : u32x4_t{0u, 0u, 0u, 0u};
    }
    __syncthreads();
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      u32x4_t xf[TT];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) xf[tt] = xs[(tt * NF + f) * 64 + lane];
#pragma unroll
      for (int r = 0; r < RBW; ++r)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) acc[r][tt] = mfma16x16x32(wf[r][f], xf[tt], acc[r][tt]);
    }
  }
  float* yb = static_cast<float*>(a.y);
#pragma unroll
  for (int r = 0; r < RBW; ++r) {
    const int rb = blockIdx.x * kMidWaves * RBW + r * kMidWaves + w;
    if (rb >= NRB) continue;
    const int n0 = rb * 16 + (lane >> 4) * 4;
    float bb[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias) {
#pragma unroll
      for (int i = 0; i < 4; ++i) bb[i] = (n0 + i < a.N) ? bf2f(a.bias[n0 + i]) : 0.f;
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int t = tt * 16 + (lane & 15);
      if (t >= a.T) continue;
      float* y = yb + (long long)t * a.ldy + n0;
      if (n0 + 3 < a.N && (a.ldy & 3) == 0) {
        *reinterpret_cast<f32x4_t*>(y) = f32x4_t{acc[r][tt][0] + bb[0], acc[r][tt][1] + bb[1],
                                                 acc[r][tt][2] + bb[2], acc[r][tt][3] + bb[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n0 + i < a.N) y[i] = acc[r][tt][i] + bb[i];
      }
    }
  }
}

constexpr int kKloopRBW = 2, kKloopNF = 8;

bool gemm_kloop_supported(int N, int K, int T) {
  return T >= 17 && T <= 128 && K % (32 * kKloopNF) == 0 && N > 0 &&
         (long long)((N + 15) / 16 + kMidWaves * kKloopRBW - 1) / (kMidWaves * kKloopRBW) >= 1024;
}

hipError_t gemm_kloop_launch(const GemmArgs& a, hipStream_t s) {
  if (!gemm_kloop_supported(a.N, a.K, a.T) || a.grp_expert || a.kgrid > 1) return hipErrorInvalidValue;
  const int TT = (a.T + 15) / 16;
  const int tt = TT <= 2 ? 2 : (TT <= 4 ? 4 : 8);
  const dim3 grid(((a.N + 15) / 16 + kMidWaves * kKloopRBW - 1) / (kMidWaves * kKloopRBW));
  const size_t lds = (size_t)tt * kKloopNF * 64 * 16;
  if (tt == 2) return timed_launch(gemm_kloop_kernel<2, kKloopRBW, kKloopNF>, grid, dim3(256), lds, s, a);
  if (tt == 4) return timed_launch(gemm_kloop_kernel<4, kKloopRBW, kKloopNF>, grid, dim3(256), lds, s, a);
  return timed_launch(gemm_kloop_kernel<8, kKloopRBW, kKloopNF>, grid, dim3(256), lds, s, a);
}

template <int TT, int RBW, int NF, bool XF32>
static hipError_t mid_go(const GemmArgs& a, dim3 grid, size_t lds, hipStream_t s) {
  if (lds > 65536)   // above the default dynamic LDS limit: raise the kernel's
    if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_mid_kernel<TT, RBW, NF, XF32>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds))
      return e;
  return timed_launch(gemm_mid_kernel<TT, RBW, NF, XF32>, grid, dim3(256), lds, s, a);
}

bool gemm_mid_chunked_ok(int K, int kgrid) {
  return K > 0 && K % 32 == 0 && kgrid >= 1 && (K / 32) % kgrid == 0 && mid_nf_ok(K / 32 / kgrid);
}

hipError_t gemm_mid_launch(GemmArgs a, int kgrid, bool xf32, hipStream_t s) {
  const int KB = a.K / 32;
  if (kgrid < 1 || KB % kgrid || !mid_nf_ok(KB / kgrid) || a.T < 1 || a.grp_expert)
    return hipErrorInvalidValue;
  const int chunks = (a.T + 127) / 128;     // > 1: token chunks of 128 over grid z
  if (chunks > 65535) return hipErrorInvalidValue;
  const int nf = KB / kgrid, rbw = mid_rbw(a.N);
  const int TT = chunks > 1 ? 8 : (a.T + 15) / 16;
  const int groups = ((a.N + 15) / 16 + kMidWaves * rbw - 1) / (kMidWaves * rbw);
  const dim3 grid(groups, kgrid, chunks);
  // token tiles rounded up to 2 / 4 / 8 (fewer instantiations); the activation
  // slice takes tt * nf KiB of LDS (twice that for fp32 activations)
  const int tt = TT <= 2 ? 2 : (TT <= 4 ? 4 : 8);
  const size_t lds = (size_t)tt * nf * 64 * 16 * (xf32 ? 2 : 1);
#define MKD_MID(TT_, NF_)                                                           \
  if (tt == TT_ && nf == NF_) {                                                      \
    if (xf32) return rbw == 2 ? mid_go<TT_, 2, NF_, true>(a, grid, lds, s)          \
                              : mid_go<TT_, 1, NF_, true>(a, grid, lds, s);         \
    return rbw == 2 ? mid_go<TT_, 2, NF_, false>(a, grid, lds, s)                   \
                    : mid_go<TT_, 1, NF_, false>(a, grid, lds, s);                  \
  }
  MKD_MID(2, 4) MKD_MID(2, 6) MKD_MID(2, 8) MKD_MID(2, 12) MKD_MID(2, 16)
  MKD_MID(4, 4) MKD_MID(4, 6) MKD_MID(4, 8) MKD_MID(4, 12) MKD_MID(4, 16)
  MKD_MID(8, 4) MKD_MID(8, 6) MKD_MID(8, 8) MKD_MID(8, 12) MKD_MID(8, 16)
#undef MKD_MID
  return hipErrorInvalidValue;
}

}  // namespace mkd
