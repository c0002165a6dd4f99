// LDS-tiled grouped GEMM for the MFMA-bound regime: many tokens per expert
// (a prefill-shaped batch), the same frag-packed bf16 weights as the decode
// GEMMs.
//
//   Y[t, n] = sum_k X[row(t), k] * W_e[n, k]   for the tokens t of expert e
//
// Block tile 256 weight rows (16 row blocks of the frag layout) x 256 tokens,
// K in stages of 32 (one fragment).  8 waves in a 2 x 4 grid, each owning 128
// rows x 64 tokens = 8 x 4 v_mfma_f32_16x16x32_bf16 tiles (128 fp32
// accumulators per lane, so two waves share a SIMD and hide each other's LDS
// and barrier waits).  A stage is 16 A fragments (each a contiguous 1 KiB
// run of the packed weights) and 16 B fragments (16 tokens x 32 k, gathered
// through the routing table), copied global -> LDS directly in MFMA operand
// order (global_load_lds_dwordx4), three stages ahead in a ring of four LDS
// buffers (128 KiB); one barrier per stage.  Per stage a wave issues 32 MFMAs
// against 12 contiguous 1 KiB LDS reads.
//
// Epilogues: EPI_SWIGLU_BF16 (gate / up row blocks interleaved in the packing,
// so both halves of a pair sit in the same wave) and EPI_SCALE_F32 (affinity
// scaled fp32 rows), with the same element math as the decode GEMMs.
#include "common.h"
#include "gemm_epi.h"
#include "mkd_internal.h"

namespace mkd {

namespace {

constexpr int kTileRows = 256;           // packed weight rows per block
constexpr int kTileTok = 256;            // tokens per block
constexpr int kStageK = 32;              // k per stage (one fragment)
constexpr int kStages = 4;               // LDS stage buffers (3 in flight)
constexpr int kRB = kTileRows / 16;      // row blocks per block (16)
constexpr int kTT = kTileTok / 16;       // token tiles per block (16)
constexpr int kStageFrags = kRB + kTT;   // 1 KiB fragments per stage (32)
constexpr int kLdsBytes = kStages * kStageFrags * 1024;

// s_waitcnt with only vmcnt = n (expcnt / lgkmcnt left at their maxima); gfx9
// encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14.
template <int N>
MKD_DEV void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int EPI>
__global__ void __launch_bounds__(512) gemm_tile_kernel(GemmArgs a) {
  extern __shared__ u32x4_t lds[];       // [kStages][kStageFrags][64 lanes]: A tiles 0..15, B 16..31
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1;     // wave: 128 rows (wm) x 64 tokens (wn)
  // XCD-aware tile order: blocks are dealt round-robin to the 8 XCDs by linear
  // id, so linear id L runs logical tile (L % 8) * per + L / 8 -- each XCD
  // walks a contiguous run of (n tile, token tile, group), and the blocks that
  // share an expert's weight and token tiles run together on one XCD's L2.
  const int gx = gridDim.x, gy = gridDim.y;
  const int total = gx * gy * gridDim.z;
  const int per = (total + 7) / 8;
  const int L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int lt = (L % 8) * per + L / 8;
  if (lt >= total) return;
  const int nb0 = (lt % gx) * kRB;
  const int t0 = ((lt / gx) % gy) * kTileTok;
  const int group = lt / (gx * gy);

  int count, base;
  const uint16_t* wp = a.w;
  if (a.grp_expert) {
    const int ng = *a.n_groups;
    count = a.grp_count[group];
    base = a.grp_offset[group];
    const int ex = a.grp_expert[group];
    asm volatile("" ::"s"(ng), "s"(count), "s"(base), "s"(ex));
    if (group >= ng) return;
    wp += (long long)ex * a.w_group_stride;
  } else {
    count = a.T;
    base = 0;
  }
  if (t0 >= count) return;

  const int KB = a.K / 32;
  const int NB = (a.N + 15) / 16;
  const int S = KB;                      // one 32-wide fragment per stage

  // ---- loads: wave w moves fragments f = w + 8j (j < 4) of each stage, one
  // 1 KiB fragment per global_load_lds_dwordx4 (lane l's 16 bytes land at
  // l * 16 of the fragment's LDS slot).  f < 16: A row block f (the packed
  // weights are already in operand order).  f >= 16: B token tile f - 16, lane
  // l = token l%16, k (l/16)*8 .. +8 of its routed row.
  const uint16_t* src[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int f = w + 8 * j;
    if (f < kRB) {
      const int nb = min(nb0 + f, NB - 1);         // rows past N: any valid block
      src[j] = wp + (long long)nb * KB * 512 + lane * 8;
    } else {
      const int c = min(t0 + (f - kRB) * 16 + (lane & 15), count - 1);   // absent: any valid row
      const int row = a.pair_row ? a.pair_row[base + c] : base + c;
      src[j] = static_cast<const uint16_t*>(a.x) + (long long)row * a.ldx + (lane >> 4) * 8;
    }
  }
  auto issue = [&](int s) {
    u32x4_t* dst = lds + (s % kStages) * kStageFrags * 64;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int f = w + 8 * j;
      const long long step = f < kRB ? (long long)s * 512 : (long long)s * 32;
      __builtin_amdgcn_global_load_lds(src[j] + step, dst + f * 64, 16, 0, 0);
    }
  };

  f32x4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < kStages - 1 && s < S; ++s) issue(s);
  for (int s = 0; s < S; ++s) {
    // this thread's loads of stage s have landed once at most the later issued
    // stages (4 loads each) are outstanding; the barrier then makes every
    // wave's stage s visible and frees the buffer of stage s - 1
    const int later = min(kStages - 2, S - 1 - s);
    if (later >= 2) wait_vmcnt<8>();
    else if (later == 1) wait_vmcnt<4>();
    else wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    if (s + kStages - 1 < S) issue(s + kStages - 1);
    const u32x4_t* st = lds + (s % kStages) * kStageFrags * 64;
    u32x4_t af[8], bf[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) af[i] = st[(wm * 8 + i) * 64 + lane];
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = st[(kRB + wn * 4 + j) * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);     // all 12 operand reads in flight together
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
  }

  // ---- epilogue: lane holds rows 4*(lane/16)+e of each row block, token lane%16 ----
  const int q4 = (lane >> 4) * 4;
  if (EPI == EPI_SWIGLU_BF16) {
    const int I = a.N / 2;
    const uint16_t* bp = a.bias ? a.bias + (a.grp_expert ? (long long)a.grp_expert[group] * a.bias_group_stride : 0)
                                : nullptr;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int nbg = nb0 + wm * 8 + 2 * p;           // gate row block (even), up = nbg + 1
      if (nbg + 1 >= NB) continue;
      const int n = (nbg >> 1) * 16 + q4;             // logical intermediate index
      float gb[4] = {0.f, 0.f, 0.f, 0.f}, ub[4] = {0.f, 0.f, 0.f, 0.f};
      if (bp) {
#pragma unroll
        for (int e = 0; e < 4; ++e) { gb[e] = bf2f(bp[n + e]); ub[e] = bf2f(bp[I + n + e]); }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tc = t0 + (wn * 4 + j) * 16 + (lane & 15);
        if (tc >= count) continue;
        const int orow = a.pair_out_row ? a.pair_out_row[base + tc] : base + tc;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = swiglu_value(a, acc[2 * p][j][e] + gb[e], acc[2 * p + 1][j][e] + ub[e]);
        uint16_t* y = static_cast<uint16_t*>(a.y) + (long long)orow * a.ldy + n;
        *reinterpret_cast<uint2*>(y) = uint2{pack2bf(o[0], o[1]), pack2bf(o[2], o[3])};
      }
    }
  } else {   // EPI_SCALE_F32
    const uint16_t* bp = a.bias ? a.bias + (a.grp_expert ? (long long)a.grp_expert[group] * a.bias_group_stride : 0)
                                : nullptr;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int nb = nb0 + wm * 8 + i;
      if (nb >= NB) continue;
      const int n = nb * 16 + q4;
      float bb[4] = {0.f, 0.f, 0.f, 0.f};
      if (bp) {
#pragma unroll
        for (int e = 0; e < 4; ++e) bb[e] = (n + e < a.N) ? bf2f(bp[n + e]) : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tc = t0 + (wn * 4 + j) * 16 + (lane & 15);
        if (tc >= count) continue;
        const int orow = a.pair_out_row ? a.pair_out_row[base + tc] : base + tc;
        const float sc = a.pair_scale ? a.pair_scale[orow] : 1.0f;
        float* y = static_cast<float*>(a.y) + (long long)orow * a.ldy + n;
        if (n + 3 < a.N) {
          *reinterpret_cast<f32x4_t*>(y) = f32x4_t{(acc[i][j][0] + bb[0]) * sc, (acc[i][j][1] + bb[1]) * sc,
                                                   (acc[i][j][2] + bb[2]) * sc, (acc[i][j][3] + bb[3]) * sc};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < a.N) y[e] = (acc[i][j][e] + bb[e]) * sc;
        }
      }
    }
  }
}

}  // namespace

int gemm_tile_lds_bytes() { return kLdsBytes; }

bool gemm_tile_supported(int N, int K, int epi) {
  if (K % kStageK != 0 || K <= 0 || N <= 0) return false;
  if (epi == EPI_SWIGLU_BF16) return N % 32 == 0;
  return epi == EPI_SCALE_F32;
}

hipError_t gemm_tile_launch(const GemmArgs& a, int epi, int groups_max, int max_tokens_per_group,
                            hipStream_t s) {
  if (!gemm_tile_supported(a.N, a.K, epi) || groups_max <= 0 || max_tokens_per_group <= 0)
    return hipErrorInvalidValue;
  const dim3 grid((a.N + kTileRows - 1) / kTileRows, (max_tokens_per_group + kTileTok - 1) / kTileTok,
                  a.grp_expert ? groups_max : 1);
  const void* fn = epi == EPI_SWIGLU_BF16 ? reinterpret_cast<const void*>(gemm_tile_kernel<EPI_SWIGLU_BF16>)
                                          : reinterpret_cast<const void*>(gemm_tile_kernel<EPI_SCALE_F32>);
  // 128 KiB of dynamic LDS is above the default launch limit (set per kernel)
  if (hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes)) return e;
  if (epi == EPI_SWIGLU_BF16)
    return timed_launch(gemm_tile_kernel<EPI_SWIGLU_BF16>, grid, dim3(512), kLdsBytes, s, a);
  return timed_launch(gemm_tile_kernel<EPI_SCALE_F32>, grid, dim3(512), kLdsBytes, s, a);
}

}  // namespace mkd
