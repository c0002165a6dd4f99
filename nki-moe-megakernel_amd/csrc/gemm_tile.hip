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
// order (buffer_load_dwordx4 ... lds), three stages ahead in a ring of four LDS
// buffers (128 KiB).  Per stage a wave issues 32 MFMAs against 12 contiguous
// 1 KiB LDS reads; the two halves of the block's waves run half a stage apart
// (two barriers per stage), one group reading while the other multiplies.
//
// Epilogues: EPI_SWIGLU_BF16 (gate / up row blocks interleaved in the packing,
// so both halves of a pair sit in the same wave) and EPI_SCALE_F32 (affinity
// scaled fp32 rows), with the same element math as the decode GEMMs.
#include "common.h"
#include "gemm_epi.h"
#include "mkd_internal.h"
#include "launch_rules.h"

namespace mkd {

namespace {

constexpr int kTileRows = 256;           // packed weight rows per block
constexpr int kTileTok = 256;            // tokens per block
constexpr int kStageK = 32;              // k per stage (one fragment)
#ifndef MKD_TILE_STAGES
#define MKD_TILE_STAGES 4
#endif
constexpr int kStages = MKD_TILE_STAGES;  // LDS stage buffers (kStages - 1 in flight)
constexpr int kRB = kTileRows / 16;      // row blocks per block (16)
constexpr int kTT = kTileTok / 16;       // token tiles per block (16)
constexpr int kStageFrags = kRB + kTT;   // 1 KiB fragments per stage (32)
constexpr int kRingBytes = kStages * kStageFrags * 1024;
// the fp32 epilogue stages half of the output tile in LDS, [256 tokens][128 + 4
// rows] (the 4 floats of padding spread a lane group's 16 rows over the banks),
// then the block's output row indices
constexpr int kStgLd = 132;
constexpr int kStgBytes = kTileTok * kStgLd * 4 + kTileTok * 4;
// the SwiGLU epilogue stages the whole h tile, [256 tokens][128 + 8 columns]
// bf16 (the padding shifts each token row by 4 banks), then the row indices
constexpr int kHsLd = 136;
static_assert(kTileTok * kHsLd * 2 + kTileTok * 4 <= kStgBytes, "h staging fits the fp32 staging area");
constexpr int kLdsBytes = kRingBytes > kStgBytes ? kRingBytes : kStgBytes;

// s_waitcnt with only vmcnt = n (expcnt / lgkmcnt left at their maxima); gfx9
// encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14.

template <int N>
MKD_DEV void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}


}  // namespace

template <int EPI>
__global__ void __launch_bounds__(512) gemm_tile_kernel(GemmArgs a) {
  constexpr int NW = 8;                  // waves: 2 (rows) x 4 (tokens)
  constexpr int WT = 4;                  // token tiles per wave
  constexpr int FPW = kStageFrags / NW;  // fragments copied per wave per stage
  extern __shared__ u32x4_t lds[];       // [kStages][kStageFrags][64 lanes]: A tiles 0..15, B 16..31
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform in an SGPR
  const int wm = w & 1, wn = w >> 1;     // wave: 128 rows (wm) x 16*WT tokens (wn)
  // Grid (n tile, work item).  Work items are the token tiles of all groups in
  // group order (group g owns ceil(count_g / 256) consecutive items); the grid
  // holds an upper bound (ceil(T*K / 256) + groups) and the block finds its
  // group by a scan of the device-side group counts.  XCD-aware order: blocks
  // are dealt round-robin to the 8 XCDs by linear id, so each XCD is given a
  // contiguous run of the LIVE logical tiles (n tile fastest, then item): the
  // blocks that share an expert's weight tiles and token rows run together on
  // one XCD's L2, and every XCD gets an eighth of the work.  (Dealing out the
  // grid's upper bound instead put its dead items -- those past the last live
  // token tile -- on the last XCDs: at 2048 tokens over 128 experts 128 of 192
  // items are live, and two XCDs sat idle.)
  // the group scan's scratch lives in the first stage buffer (no copy is issued
  // before every wave has read the scan's result)
  int* scan_s = reinterpret_cast<int*>(lds);
  int* item_s = scan_s + 8;
  const int gx = gridDim.x;
  const int L = blockIdx.x + gx * blockIdx.y;
  // (tile_deal_rule: XCD L % 8 owns a contiguous run of the live tiles, its
  // k-th block takes tile k of it, blocks past the run have no work; the grid
  // holds at least `live` blocks, so every tile is taken)
  auto deal = [&](int live, int& lt) { return tile_deal_rule(live, L, &lt); };
  int lt = 0;

  int count, base, t0, expert = 0, kq = 0;
  const uint16_t* wp = a.w;
  if (a.grp_expert) {
    // thread g holds group g's token-tile count (<= 512 groups); block-wide
    // inclusive scan in group order; the owner of the block's item publishes it
    const int ng = *a.n_groups;
    const int c = tid < ng ? a.grp_count[tid] : 0;
    const int tiles = (c + kTileTok - 1) / kTileTok;
    int x = tiles;                       // wave inclusive scan (64 lanes)
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) scan_s[w] = x;
    if (tid == 0) item_s[0] = -1;
    __syncthreads();
    int before = 0, items = 0;
    for (int q = 0; q < NW; ++q) {
      const int v = scan_s[q];
      if (q < w) before += v;
      items += v;
    }
    const bool mine = deal(gx * items, lt);
    const int item = lt / gx;
    const int incl = before + x, excl = incl - tiles;
    if (mine && tid < ng && item >= excl && item < incl) {
      item_s[0] = tid;
      item_s[1] = (item - excl) * kTileTok;
    }
    __syncthreads();
    const int g = item_s[0];
    if (g < 0) return;                   // past the last live token tile (uniform)
    t0 = item_s[1];
    count = a.grp_count[g];
    base = a.grp_offset[g];
    expert = a.grp_expert[g];
    wp += (long long)expert * a.w_group_stride;
    __syncthreads();                     // item_s read by every wave before the copies
  } else {
    // dense: gridDim.y = token tiles x K slices (kgrid > 1: fp32 partials, one
    // per slice, at y + slice * part_stride; the slice is the slowest index, so
    // an XCD's run shares one K slice of the weights)
    if (!deal(gx * (int)gridDim.y, lt)) return;   // (the grid is exact here)
    const int items = (int)gridDim.y / (a.kgrid > 1 ? a.kgrid : 1);
    const int r = lt / gx;
    kq = r / items;
    count = a.T;
    base = 0;
    t0 = (r - kq * items) * kTileTok;
    if (t0 >= count) return;
  }
  const int nb0 = (lt % gx) * kRB;

  const int KB = a.K / 32;
  const int NB = (a.N + 15) / 16;
  const int S = a.grp_expert || a.kgrid <= 1 ? KB : KB / a.kgrid;   // one 32-wide fragment per stage
  const int s0 = kq * S;                 // the block's first fragment of K

  // ---- loads: wave w moves fragments f = w + 8j (j < 4) of each stage, one
  // 1 KiB fragment per buffer_load_dwordx4 ... lds (lane l's 16 bytes land at
  // l * 16 of the fragment's LDS slot; the MUBUF form is tracked by vmcnt
  // alone, so LDS reads issued around it keep their own lgkmcnt waits).
  // f < 16: A row block f (the packed weights are already in operand order).
  // f >= 16: B token tile f - 16, lane l = token l%16, k (l/16)*8 .. +8 of its
  // routed row.  Offsets are bytes from the expert's weights / from x.
  const __amdgpu_buffer_rsrc_t wsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(wp), 0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t xsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.x), 0, 0x7fffffff, 0x00020000);
  int voff[FPW];
#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int f = w + NW * j;
    const int nb = min(nb0 + f, NB - 1);           // rows past N: any valid block
    voff[j] = f < kRB ? ((nb * KB + s0) * 512 + lane * 8) * 2 : 0;
  }
  auto issue = [&](int s, int buf) {
    u32x4_t* dst = lds + buf * kStageFrags * 64;
#pragma unroll
    for (int j = 0; j < FPW; ++j) {
      const int f = w + NW * j;
      if (f < kRB)   // wave-uniform: j and w fix f
        copy_frag_lds(wsrc, dst + f * 64, voff[j] + s * 1024);
      else
        copy_frag_lds(xsrc, dst + f * 64, voff[j] + s * 64);
    }
  };

#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int f = w + NW * j;
    if (f >= kRB) {
      const int c = min(t0 + (f - kRB) * 16 + (lane & 15), count - 1);   // absent: any valid row
      const int row = a.pair_row ? a.pair_row[base + c] : base + c;
      voff[j] = (row * a.ldx + s0 * 32 + (lane >> 4) * 8) * 2;
    }
  }
  // output rows of this lane's WT tokens, loaded ahead of the main loop (the
  // epilogue's stores would otherwise wait on these loads one token at a time)
  int orow[WT];
#pragma unroll
  for (int j = 0; j < WT; ++j) {
    const int tc = min(t0 + (wn * WT + j) * 16 + (lane & 15), count - 1);
    orow[j] = a.pair_out_row ? a.pair_out_row[base + tc] : base + tc;
  }
  f32x4_t acc[8][WT];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < WT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // this wave's copies of a stage have landed once at most `after` stages
  // issued later are outstanding (FPW copies each); after <= kStages - 2
  static_assert(kStages >= 3 && kStages <= 5, "wait_landed covers 0 .. 3 later stages");
  auto wait_landed = [&](int after) {
    if (after >= 3) wait_vmcnt<3 * FPW>();
    else if (after == 2) wait_vmcnt<2 * FPW>();
    else if (after == 1) wait_vmcnt<FPW>();
    else wait_vmcnt<0>();
  };
  for (int s = 0; s < kStages - 1 && s < S; ++s) issue(s, s);
  // Two wave groups run half a stage apart: waves 0-3 (group 0) and 4-7 (group
  // 1), one of each per SIMD.  Group 1 takes one barrier before the loop and
  // group 0 one after it, so between two barriers one group reads its operands
  // of a stage from LDS while the other runs the previous stage's MFMAs, and the
  // SIMD's matrix core has work in both halves.  Every wave executes the same
  // loop: wait for its copies of stage s, barrier, 12 operand reads, the copies
  // of stage s + kStages - 1 (none past the last stage: the waits count the
  // stages actually issued after the awaited one), barrier, 32 MFMAs.  Ordering:
  //  * a stage is read only after every wave's copies of it landed: group 0
  //    waits for stage s before its first barrier of iteration s; group 1, which
  //    reads it one barrier later, waits for stage s + 1 before its second
  //    barrier of iteration s (the barrier after which group 0 reads s + 1), and
  //    for stage 0 before its extra barrier;
  //  * a buffer is refilled (stage s + kStages - 1 into the buffer of s - 1)
  //    only after both groups' reads of it completed: each wave waits for its
  //    operand reads (lgkmcnt 0) before the barrier that starts its MFMAs.
  // Each accumulator sums its stages in the same order as a one-group loop.
  {
    const bool g1 = w >= 4;
    if (g1) {
      wait_landed(min(S - 1, kStages - 2));                  // stage 0
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_barrier" ::: "memory");
    }
    for (int s = 0; s < S; ++s) {
      wait_landed(min(S - 1 - s, kStages - 2));              // stage s
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      const u32x4_t* st = lds + (s % kStages) * kStageFrags * 64;
      u32x4_t af[8], bf[WT];
#pragma unroll
      for (int j = 0; j < WT; ++j) bf[j] = st[(kRB + wn * WT + j) * 64 + lane];
#pragma unroll
      for (int i = 0; i < 8; ++i) af[i] = st[(wm * 8 + i) * 64 + lane];
      __builtin_amdgcn_sched_barrier(0);
      if (s + kStages - 1 < S) issue(s + kStages - 1, (s + kStages - 1) % kStages);
      __builtin_amdgcn_sched_barrier(0);
      if (g1 && s + 1 < S) wait_landed(min(S - 2 - s, kStages - 2));   // stage s + 1
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < WT; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (!g1) asm volatile("s_barrier" ::: "memory");
  }

  // ---- epilogue: lane holds rows 4*(lane/16)+e of each row block, token lane%16 ----
  const int q4 = (lane >> 4) * 4;
  if (EPI == EPI_SWIGLU_BF16) {
    // The h tile goes out through LDS: the waves store their SwiGLU values as
    // [token][128 h columns + 8] bf16, then 16 threads write each token's
    // 256-byte row segment in 16-byte stores -- directly, a store instruction
    // wrote 8 bytes into each of 16 scattered rows per lane group.
    const int I = a.N / 2;
    const uint16_t* bp = a.bias ? a.bias + (long long)expert * a.bias_group_stride : nullptr;
    wait_vmcnt<0>();                     // the ring's last copies have landed
    uint16_t* hs = reinterpret_cast<uint16_t*>(lds);
    int* orow_s = reinterpret_cast<int*>(hs + kTileTok * kHsLd);
    if (tid < kTileTok) {
      const int tc = min(t0 + tid, count - 1);
      orow_s[tid] = a.pair_out_row ? a.pair_out_row[base + tc] : base + tc;
    }
    __syncthreads();                     // every wave is past its last operand reads
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int nbg = nb0 + wm * 8 + 2 * p;           // gate row block (even), up = nbg + 1
      if (nbg + 1 >= NB) continue;                    // h columns past I (never stored)
      const int n = (nbg >> 1) * 16 + q4;             // logical intermediate index
      const int nl = (wm * 4 + p) * 16 + q4;          // its column in the tile's 128
      float gb[4] = {0.f, 0.f, 0.f, 0.f}, ub[4] = {0.f, 0.f, 0.f, 0.f};
      if (bp) {
#pragma unroll
        for (int e = 0; e < 4; ++e) { gb[e] = bf2f(bp[n + e]); ub[e] = bf2f(bp[I + n + e]); }
      }
#pragma unroll
      for (int j = 0; j < WT; ++j) {
        const int tl = (wn * WT + j) * 16 + (lane & 15);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = swiglu_value(a, acc[2 * p][j][e] + gb[e], acc[2 * p + 1][j][e] + ub[e]);
        *reinterpret_cast<uint2*>(hs + tl * kHsLd + nl) = uint2{pack2bf(o[0], o[1]), pack2bf(o[2], o[3])};
      }
    }
    __syncthreads();
    // N % 32 == 0, so I % 16 == 0: an 8-column piece is all below I or all past it
    const int c8 = (tid & 15) * 8;
    const int n = (nb0 >> 1) * 16 + c8;
    if (n < I) {
      for (int tl = tid >> 4; tl < kTileTok; tl += 32) {
        if (t0 + tl >= count) break;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(hs + tl * kHsLd + c8);
        *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(a.y) + (long long)orow_s[tl] * a.ldy + n) = v;
      }
    }
  } else {   // EPI_SCALE_F32
    // (K slices: the bias joins the first slice's partial)
    const uint16_t* bp = a.bias && kq == 0 ? a.bias + (long long)expert * a.bias_group_stride : nullptr;
    // all WT affinities up front (y is float too, so loads among the stores
    // could not be moved past them)
    float sc[WT];
#pragma unroll
    for (int j = 0; j < WT; ++j) sc[j] = a.pair_scale ? a.pair_scale[orow[j]] : 1.0f;
    // The tile goes out through LDS, half (128 rows) at a time: the waves of
    // that half store their scaled accumulators as [token][row], then every
    // thread writes 16 contiguous bytes of a token's 512-byte row segment --
    // directly, a store instruction wrote 64 bytes into each of 16 scattered
    // output rows, and the stores took ~40 % of the down projection's time.
    wait_vmcnt<0>();                     // the ring's last copies have landed
    float* stg = reinterpret_cast<float*>(lds);
    int* orow_s = reinterpret_cast<int*>(stg + kTileTok * kStgLd);
    if (tid < kTileTok) {
      const int tc = min(t0 + tid, count - 1);
      orow_s[tid] = a.pair_out_row ? a.pair_out_row[base + tc] : base + tc;
    }
    __syncthreads();                     // every wave is past its last operand reads
    float* ybase = static_cast<float*>(a.y) + kq * a.part_stride;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (wm == half) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int n = (nb0 + wm * 8 + i) * 16 + q4;
          float bb[4] = {0.f, 0.f, 0.f, 0.f};
          if (bp) {
#pragma unroll
            for (int e = 0; e < 4; ++e) bb[e] = (n + e < a.N) ? bf2f(bp[n + e]) : 0.f;
          }
#pragma unroll
          for (int j = 0; j < WT; ++j) {
            const int tl = (wn * WT + j) * 16 + (lane & 15);
            *reinterpret_cast<f32x4_t*>(stg + tl * kStgLd + i * 16 + q4) =
                f32x4_t{(acc[i][j][0] + bb[0]) * sc[j], (acc[i][j][1] + bb[1]) * sc[j],
                        (acc[i][j][2] + bb[2]) * sc[j], (acc[i][j][3] + bb[3]) * sc[j]};
          }
        }
      }
      __syncthreads();
      const int c4 = (tid & 31) * 4;                  // row offset within the half
      const int n = (nb0 + half * 8) * 16 + c4;
      for (int tl = tid >> 5; tl < kTileTok; tl += 16) {
        if (t0 + tl >= count) break;
        const f32x4_t v = *reinterpret_cast<const f32x4_t*>(stg + tl * kStgLd + c4);
        float* y = ybase + (long long)orow_s[tl] * a.ldy + n;
        if (n + 3 < a.N) {
          *reinterpret_cast<f32x4_t*>(y) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < a.N) y[e] = v[e];
        }
      }
      __syncthreads();                   // the half is read before the next one is written
    }
  }
  wait_vmcnt<0>();                       // no copy into LDS outlives the block
}


int gemm_tile_lds_bytes() { return kLdsBytes; }

bool gemm_tile_supported(int N, int K, int epi) {
  if (K % kStageK != 0 || K <= 0 || N <= 0) return false;
  if (epi == EPI_SWIGLU_BF16) return N % 32 == 0;
  return epi == EPI_SCALE_F32;
}

bool gemm_tile_kgrid_ok(int K, int kgrid) {
  const int KB = K / kStageK;
  return kgrid >= 1 && kgrid <= 8 && K % kStageK == 0 && KB % kgrid == 0;
}

// K slices for a dense tiled GEMM whose output tiles leave CUs idle (a short
// prefill pass: the attention output projection at 2048 tokens has 64 tiles):
// the largest of 2, 4, 8 that keeps tiles x slices within one block per CU and
// at least 16 stages per slice.  The partials cost T * N * 4 bytes per slice
// written and read again by the consumer.
int gemm_tile_kgrid(int N, int K, int T) {
  static_assert(kTileRows == 256 && kTileTok == 256 && kStageK == 32, "tile_kgrid_rule's tile shape");
  return tile_kgrid_rule(N, K, T, device_cus());
}

hipError_t gemm_tile_launch(const GemmArgs& a, int epi, int groups_max, long long total_rows,
                            hipStream_t s) {
  if (!gemm_tile_supported(a.N, a.K, epi) || groups_max <= 0 || total_rows <= 0)
    return hipErrorInvalidValue;
  // the SwiGLU epilogue writes h in 16-byte pieces
  if (epi == EPI_SWIGLU_BF16 && ((a.ldy & 7) || (reinterpret_cast<uintptr_t>(a.y) & 15)))
    return hipErrorInvalidValue;
  // K slices: dense fp32 partials only, each slice's rows clear of the next's
  const int kg = a.kgrid > 1 ? a.kgrid : 1;
  if (kg > 1 && (a.grp_expert || epi != EPI_SCALE_F32 || a.pair_scale || !gemm_tile_kgrid_ok(a.K, kg) ||
                 a.part_stride < total_rows * a.ldy))
    return hipErrorInvalidValue;
  // work items: every group's token tiles; with total_rows = sum of the group
  // sizes, sum_g ceil(c_g / 256) <= ceil(total_rows / 256) + groups
  const long long items = (total_rows + kTileTok - 1) / kTileTok + (a.grp_expert ? groups_max : 0);
  if (items * kg > 65535) return hipErrorInvalidValue;
  const dim3 grid((a.N + kTileRows - 1) / kTileRows, (unsigned)(items * kg));
  // 128 KiB of dynamic LDS is above the default launch limit (set per kernel)
  if (epi == EPI_SWIGLU_BF16) {
    if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_tile_kernel<EPI_SWIGLU_BF16>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes))
      return e;
    return timed_launch(gemm_tile_kernel<EPI_SWIGLU_BF16>, grid, dim3(512), kLdsBytes, s, a);
  }
  if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_tile_kernel<EPI_SCALE_F32>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes))
    return e;
  return timed_launch(gemm_tile_kernel<EPI_SCALE_F32>, grid, dim3(512), kLdsBytes, s, a);
}

}  // namespace mkd
