// Decode attention for one new token per sequence (GQA, split-K over the KV
// length) on gfx950 MFMA: two kernels.
//
// attn_fused_kernel, grid (chunk, kv_head g, sequence b), block = 4 waves:
//  1. prep: the GQA query heads of kv head g and the new k / v rows of g are
//     taken from the fp32 projections, rounded (Qwen flow), per-head RMSNorm'd,
//     RoPE'd (rotate-half, contiguous halves) into LDS.  Every block of (b, g)
//     recomputes this (a few hundred elements; all of a wave's loads are issued
//     before any use) instead of a separate launch.
//  2. split-K attention over its 64*TPW positions; wave w owns TPW tiles of 16
//     positions.  Per tile:
//       S = K_tile . q^T   v_mfma_f32_16x16x32_bf16, A = 16 K rows (HBM, each
//                          lane 4 x 16 B of one row), B = the gqa query heads
//                          (16 columns, >= gqa zero).  D lane l holds
//                          S[pos 4*(l/16)+i][head l%16].
//       p = exp(s - m_head) with the wave's per-head max.
//       O += P . V        v_mfma_f32_16x16x32_bf16 over two tiles (one 16x16x16
//                          when a wave holds a single tile): the S layout above
//                          IS the A layout (row = head l%16, k = positions
//                          4*(l/16)+i; two tiles give a lane group's 8 k slots),
//                          so P never leaves registers.  B = V
//                          [pos 4*(l/16)+j][d label l%16]: the d labels are
//                          permuted so that lane column c = l%16 owns the D/16
//                          contiguous elements c*D/16.. of its four position
//                          rows (one 16 B / 8 B load per row straight from
//                          HBM); d-tile dt's operand is element dt of those
//                          rows, two byte-permutes -- no transpose through LDS.
//     Positions t < n_prior[b] read the cache (flat [B, nkv, S_max, d], or block
//     [num_blocks, blk_len, nkv, d] through the sequence's block table: the
//     paged layout of attention_block_tkg.py:199-206, 1473-1685), t == n_prior[b]
//     is the new token
//     (from LDS), t > n_prior[b] are masked.  With round_qwen the score is
//     bf16(bf16(q.k) * scale) as in the reference's fused kernel.  The 4 wave
//     partials merge in LDS into (max, sum, unnormalised O) per head, written
//     to the chunk's slot of part_ml / part_o; the chunk holding position
//     n_prior[b] also stages the new k / v rows for the scatter.
// attn_combine_kernel, grid (q head, sequence), block = 4 waves: log-sum-exp
//  merge of the chunks (waves take every 4th chunk, online rescaling, LDS
//  reduce), optional sink logit, bf16 output; the blocks of the first head of
//  each kv group then scatter the new k / v rows into the caches at
//  write_pos[b] -- after every chunk has read the cache, because the kernels
//  run in stream order.
//  (A single kernel with a last-arriving-block combine was measured slower:
//  the device-scope fence and the counter atomic cost ~9 us per block on
//  this part, more than a kernel boundary.)
// Both kernels issue their independent global loads (cache rows, partials)
// before the dependent math so that one memory latency covers them.
#include "common.h"
#include "mkd_internal.h"
#include "attn_common.h"
#include "coherent.h"

namespace mkd {

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4v;

MKD_DEV f32x4_t mfma16x16x16(uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4v, a),
                                                   __builtin_bit_cast(bf16x4v, b), c, 0, 0, 0);
}

// The GQA + 2 heads of kv group g of sequence b, prepared (attention_block_tkg.py:
// 915-1138) by the 4 waves of a block: wave w takes heads w, w+4, ... of
// [q heads of g | k of g | v of g]; all loads first, then the math.
template <int D, int GQA, int MP = 8>
MKD_DEV void prep_heads(const AttnArgs& a, int rope_mode, int b, int g, int w, int lane,
                        uint16_t (*q_dst)[D], uint16_t* k_dst, uint16_t* v_dst,
                        uint16_t* k_dst2 = nullptr, uint16_t* v_dst2 = nullptr) {
  constexpr int NR = (GQA + 2 + 3) / 4;
  HeadPrep<D, MP> hp[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int h = w + 4 * r;
    if (h < GQA + 2) {
      const int kind = h < GQA ? 0 : h - GQA + 1;
      const int head = h < GQA ? g * GQA + h : (kind == 1 ? a.nq + g : a.nq + a.nkv + g);
      hp[r].load(a, rope_mode, b, head, kind, lane);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int h = w + 4 * r;
    if (h < GQA + 2) {
      const int kind = h < GQA ? 0 : h - GQA + 1;
      hp[r].finish(a, rope_mode, kind, h < GQA ? q_dst[h] : (kind == 1 ? k_dst : v_dst), lane,
                   kind == 1 ? k_dst2 : (kind == 2 ? v_dst2 : nullptr));
    }
  }
}

// Large grids: the heads of (b, g) are prepared once here, block (g, b), into
// a.prep [B, nkv, gqa + 2, d], instead of in every one of its chunk blocks.
// MP = 1 (the projection comes whole, a.qkv_nparts <= 1): without the partial
// sums' registers the kernel fits 8 waves per SIMD -- a prefill pass's grid of
// (kv heads x tokens) small blocks is a chain of load round trips, and twice the
// resident blocks halve their number.
// kv_write (a prefill pass): token b's prepared k / v rows of kv head g also go
// to their cache row, before any attention block reads it (the combine
// kernel later stores the same values again).
template <int D, int GQA, int MP = 8>
__global__ void __launch_bounds__(256, MP == 1 ? 8 : 1) attn_prep_kernel(AttnArgs a, int rope_mode, int kv_write) {
  const int g = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint16_t* dst = a.prep + ((long long)b * a.nkv + g) * (GQA + 2) * D;
  uint16_t *k2 = nullptr, *v2 = nullptr;
  if (kv_write) {
    const long long row = kv_write_row(a, b);
    if (row >= 0) {
      const long long off = a.block_table ? (row * a.nkv + g) * D
                                          : seq_of(a, b) * a.cache_b_stride + g * a.cache_h_stride + row * D;
      k2 = a.k_cache + off;
      v2 = a.v_cache + off;
    }
  }
  prep_heads<D, GQA, MP>(a, rope_mode, b, g, w, lane, reinterpret_cast<uint16_t(*)[D]>(dst),
                         dst + GQA * D, dst + (GQA + 1) * D, k2, v2);
}

// the one-part form wherever the projection comes whole (bf16, or fp32 without
// K-slice partials: HeadPrep then sums exactly one part)
template <int D, int GQA>
static void launch_prep(const AttnArgs& a, int rope_mode, hipStream_t s, bool kv_write = false) {
  const int kw = kv_write ? 1 : 0;
  if (!a.qkv || a.qkv_nparts <= 1)
    hipLaunchKernelGGL((attn_prep_kernel<D, GQA, 1>), dim3(a.nkv, a.B), dim3(256), 0, s, a, rope_mode, kw);
  else
    hipLaunchKernelGGL((attn_prep_kernel<D, GQA, 8>), dim3(a.nkv, a.B), dim3(256), 0, s, a, rope_mode, kw);
}

// One split-K chunk block (c, g, b).  COH: the block's outputs (partials and
// staged k / v rows) are read by later blocks of the same launch -- they are
// stored device-coherent and the block then sets *flag (also when the chunk
// lies past the sequence and the block does nothing else).  ONE: the caller
// has established one new token per sequence, no mask, a flat cache and heads
// prepared here (no a.prep), so those cases' code -- runtime branches around
// conditional loads in the score and P.V loops -- is not compiled in.
template <int D, int GQA, int TPW, bool COH, int NW = 4, bool ONE = false>
MKD_DEV void attn_chunk_block(const AttnArgs& a, int rope_mode, int c, int g, int b, unsigned* flag) {
  constexpr int NK = D / 32;                  // QK MFMAs per tile (k = 32)
  constexpr int NDT = D / 16;                 // PV d-tiles
  constexpr int CP = NW * TPW * 16;           // positions per block (NW waves)
  constexpr int VW = D / 32;                  // dwords of a lane's V row segment
  __shared__ float m_s[NW][16], l_s[NW][16];
  __shared__ __attribute__((aligned(16))) float o_s[NW][GQA][D];
  __shared__ __attribute__((aligned(16))) uint16_t q_s[GQA][D];
  __shared__ __attribute__((aligned(16))) uint16_t kn_s[D];
  __shared__ __attribute__((aligned(16))) uint16_t vn_s[D];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int chunk0 = c * CP;

  // ---- 0. the wave's K and V rows from the cache: they depend on nothing
  // computed here, so their loads are issued first and overlap the prep.  A
  // flat cache's rows are loaded before the prior length n is known (rows of
  // the chunk below S_max; rows at or past n are never used: their scores are
  // masked and their V values zeroed where they are read), so that the length's
  // own round trip is not in front of them; a block table's rows need the
  // table and the length first.  With 4 tiles per wave (large grids) the
  // registers cost more occupancy than the overlap gains, and the rows are
  // loaded where they are used. ----
  constexpr bool PRE = TPW <= 2;
  const bool flat = ONE || a.block_table == nullptr;
  int n = a.S_max;                            // row bound until the prior length is read
  // lane l's k elements of QK step kk: d = 32 kk + 8 (l / 16) .. + 8 -- the four
  // lanes of a row read 64 consecutive bytes per step (half a cache line),
  // not four 16-byte pieces 64 bytes apart
  const int dq = (lane >> 4) * 8;
  const int wbase = chunk0 + w * TPW * 16;
  const int vc = (lane & 15) * (D / 16);      // lane's V row segment (d labels)
  // Row pointers first, then the loads: with a block table every pointer is
  // itself a load, and interleaving them would make each data load wait.
  // V rows of tile `tile0` for the PV operand: position tile0 + 4*(l/16) + j
  // (rows below n; n is S_max until the prior length is known).
  auto v_ptrs = [&](int tile0, bool live, const uint16_t* (&p)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = tile0 + (lane >> 4) * 4 + j;
      p[j] = (live && t < n) ? kv_row<D>(a, a.v_cache, b, g, t) : nullptr;
    }
  };
  auto v_load = [&](const uint16_t* const (&p)[4], uint32_t (&dst)[4][VW]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (VW == 4) {
        const u32x4_t v = p[j] ? ld16(p[j] + vc) : u32x4_t{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[j][e] = v[e];
      } else {
        const uint2 v = p[j] ? *reinterpret_cast<const uint2*>(p[j] + vc) : uint2{0, 0};
        dst[j][0] = v.x;
        dst[j][1] = v.y;
      }
    }
  };
  // K row of tile `tile0` for the score operand: position tile0 + l%16
  auto k_ptr = [&](int tile0, bool live) {
    const int t = tile0 + (lane & 15);
    return (live && t < n) ? kv_row<D>(a, a.k_cache, b, g, t) : nullptr;
  };
  auto k_load = [&](const uint16_t* kr, u32x4_t (&dst)[NK]) {
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) dst[kk] = kr ? ld16(kr + dq + kk * 32) : u32x4_t{0, 0, 0, 0};
  };
  u32x4_t kpre[PRE ? TPW : 1][NK];
  uint32_t vpre[PRE ? TPW : 1][4][VW];
  auto pre_loads = [&]() {
    if (flat) {
      // every row address valid (clamped below S_max), so the loads carry no
      // condition and the wait for the prior length -- loaded before them --
      // can count them out; the rows past n are masked where they are used
      const uint16_t* kc = a.k_cache + seq_of(a, b) * a.cache_b_stride + g * a.cache_h_stride;
      const uint16_t* vc0 = a.v_cache + seq_of(a, b) * a.cache_b_stride + g * a.cache_h_stride;
#pragma unroll
      for (int tt = 0; tt < TPW; ++tt) {
        const int tk = min(wbase + tt * 16 + (lane & 15), a.S_max - 1);
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) kpre[tt][kk] = ld16(kc + (long long)tk * D + dq + kk * 32);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int tv = min(wbase + tt * 16 + (lane >> 4) * 4 + jj, a.S_max - 1);
          const uint16_t* vr = vc0 + (long long)tv * D + vc;
          if constexpr (VW == 4) {
            const u32x4_t v = ld16(vr);
#pragma unroll
            for (int e = 0; e < 4; ++e) vpre[tt][jj][e] = v[e];
          } else {
            const uint2 v = *reinterpret_cast<const uint2*>(vr);
            vpre[tt][jj][0] = v.x;
            vpre[tt][jj][1] = v.y;
          }
        }
      }
      return;
    }
    const uint16_t* kp[TPW];
    const uint16_t* vp[TPW][4];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      kp[tt] = k_ptr(wbase + tt * 16, true);
      v_ptrs(wbase + tt * 16, true, vp[tt]);
    }
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      k_load(kp[tt], kpre[tt]);
      v_load(vp[tt], vpre[tt]);
    }
  };

  // ---- 1. the kv group's prepared heads [q heads of g | k of g | v of g]:
  // copied from attn_prep_kernel's output (large grids), or prepared here --
  // wave w takes heads w, w+4, ...: their loads go out first (a wave's vector
  // loads complete in issue order, so the math need not wait for the cache
  // rows behind them), then the prior length and the cache rows ----
  constexpr int NR = (GQA + 2 + NW - 1) / NW;
  HeadPrep<D> hp[NR];
  if (ONE || !a.prep) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int h = w + NW * r;
      if (h < GQA + 2) {
        const int kind = h < GQA ? 0 : h - GQA + 1;
        const int head = h < GQA ? g * GQA + h : (kind == 1 ? a.nq + g : a.nq + a.nkv + g);
        hp[r].load(a, rope_mode, b, head, kind, lane);
      }
    }
  }
  const int n_raw = prior_raw_vmem(a, b);
  if (PRE && flat) pre_loads();
  n = __builtin_amdgcn_readfirstlane(prior_clamp(a, n_raw));
  // the window: n cache positions, then the sequence's NT new tokens (NT = 1:
  // this row's own, in LDS; more: every new row's prepared k / v in `prep`)
  const int NT = ONE ? 1 : new_tokens(a), seq = seq_of(a, b), tk = tok_of(a, b);
  const uint16_t* act0 =                      // new token 0's prepared heads
      NT > 1 ? a.prep + ((long long)seq * NT * a.nkv + g) * (GQA + 2) * D : nullptr;
  const long long act_stride = (long long)a.nkv * (GQA + 2) * D;                     // per new token
  const int total = n + NT;
  // a chunk past the sequence exits at once -- except in the ONE form: there
  // the exit would depend on n, and the compiler then sinks the cache-row loads
  // below it, behind n's round trip; the block instead runs with every
  // position masked (its partial, M = -inf, L = 0, is never read)
  if (!ONE && chunk0 >= total) {              // whole block: uniform exit
    if constexpr (COH) coh_publish(flag);
    return;
  }
  if (PRE && !flat) pre_loads();
  if (!ONE && a.prep) {
    const uint16_t* src = a.prep + ((long long)b * a.nkv + g) * (GQA + 2) * D;
    for (int i = threadIdx.x * 8; i < (GQA + 2) * D; i += NW * 64 * 8) {
      const int h = i / D, d = i % D;
      uint16_t* dst = h < GQA ? &q_s[h][d] : (h == GQA ? &kn_s[d] : &vn_s[d]);
      *reinterpret_cast<u32x4_t*>(dst) = ld16(src + i);
    }
  } else {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int h = w + NW * r;
      if (h < GQA + 2) {
        const int kind = h < GQA ? 0 : h - GQA + 1;
        hp[r].finish(a, rope_mode, kind, h < GQA ? q_s[h] : (kind == 1 ? kn_s : vn_s), lane);
      }
    }
  }
  __syncthreads();

  // q fragments (B operand): lane l -> head l%16, d = (l/16)*(D/4) + kk*8 .. +8
  const int hcol = lane & 15;
  u32x4_t qf[NK];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk)
    qf[kk] = hcol < GQA ? *reinterpret_cast<const u32x4_t*>(&q_s[hcol][dq + kk * 32])
                        : u32x4_t{0, 0, 0, 0};

  // ---- 2. scores for the wave's tiles (without the up-front copies: the K
  // rows of LB tiles are loaded together, then their MFMAs run) ----
#ifndef MKD_ATTN_LB
#define MKD_ATTN_LB 2
#endif
  constexpr int LB = PRE ? 1 : MKD_ATTN_LB;
  float s[TPW][4];
  u32x4_t kl[LB][NK];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int t = wbase + tt * 16 + (lane & 15);  // A row owned by this lane
    if (!PRE && tt % LB == 0) {
      const uint16_t* kp[LB];
#pragma unroll
      for (int u = 0; u < LB; ++u) kp[u] = k_ptr(wbase + (tt + u) * 16, tt + u < TPW);
#pragma unroll
      for (int u = 0; u < LB; ++u) k_load(kp[u], kl[u]);
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      u32x4_t kf;
      if constexpr (PRE) kf = kpre[tt][kk];
      else kf = kl[tt % LB][kk];
      if (NT == 1) {
        if (t == n) kf = *reinterpret_cast<const u32x4_t*>(&kn_s[dq + kk * 32]);
      } else if (t >= n && t < total) {
        kf = ld16(act0 + (t - n) * act_stride + GQA * D + dq + kk * 32);
      }
      acc = mfma16x16x32(kf, qf[kk], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tp = wbase + tt * 16 + (lane >> 4) * 4 + i;   // position of acc[i]
      float sc = a.round_qwen ? rbf(rbf(acc[i]) * a.scale) : acc[i] * a.scale;
      bool ok = tp < total && hcol < GQA;
      if (!ONE && ok && a.mask) {
        const int mt = (tp < n) ? tp : (a.mask_s_ctx - NT + (tp - n));
        ok = a.mask[(((long long)mt * (a.B / NT) + seq) * a.nq + g * GQA + hcol) * NT + tk] != 0;
      }
      s[tt][i] = ok ? sc : -INFINITY;
    }
  }
  // per-head max over the wave's positions (lanes sharing l%16)
  float m = -INFINITY;
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, s[tt][i]);
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float lsum = 0.f;
  uint2 pa[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = (m == -INFINITY) ? 0.f : expf(s[tt][i] - m);
      lsum += p[i];
    }
    pa[tt] = uint2{pack2bf(p[0], p[1]), pack2bf(p[2], p[3])};
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // ---- O = P V ----
  f32x4_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint32_t vl[LB][4][VW];
  uint2 bprev[NDT];                           // an even tile's V operands (paired tiles)
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int tile0 = wbase + tt * 16;
    if (!PRE && tt % LB == 0) {
      const uint16_t* vp[LB][4];
#pragma unroll
      for (int u = 0; u < LB; ++u) v_ptrs(tile0 + u * 16, tt + u < TPW, vp[u]);
#pragma unroll
      for (int u = 0; u < LB; ++u) v_load(vp[u], vl[u]);
    }
    uint32_t v[4][VW];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        if constexpr (PRE) v[j][e] = vpre[tt][j][e];
        else v[j][e] = vl[tt % LB][j][e];
      }
    // the new token's row comes from LDS (at most one j per lane); rows past it
    // (read before n was known) are zero
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = tile0 + (lane >> 4) * 4 + j;
      if (NT == 1 && t == n) {
#pragma unroll
        for (int e = 0; e < VW; ++e) v[j][e] = *reinterpret_cast<const uint32_t*>(&vn_s[vc + 2 * e]);
      } else if (NT > 1 && t >= n && t < total) {
        const uint16_t* vr = act0 + (t - n) * act_stride + (GQA + 1) * D + vc;
#pragma unroll
        for (int e = 0; e < VW; ++e) v[j][e] = *reinterpret_cast<const uint32_t*>(vr + 2 * e);
      } else if (t >= total) {
#pragma unroll
        for (int e = 0; e < VW; ++e) v[j][e] = 0u;
      }
    }
    // the B operand's 16-bit halves from two V rows: one byte permute per
    // dword (selector 0x05040100: bytes 0-1 of each row; 0x07060302: bytes 2-3)
    uint2 bop[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int e = dt >> 1;
      const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
      bop[dt] = uint2{__builtin_amdgcn_perm(v[1][e], v[0][e], sel), __builtin_amdgcn_perm(v[3][e], v[2][e], sel)};
    }
    if constexpr (TPW % 2 == 0) {
      // tiles in pairs on the 32-deep MFMA: lane group q's k slots 8q .. 8q+7
      // are positions 4q .. 4q+3 of the even tile, then of the odd tile -- the
      // same order in the P operand (its two 4-position halves) and in the V
      // operand (its two row quads)
      if (tt % 2 == 0) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) bprev[dt] = bop[dt];
      } else {
        const u32x4_t pp = {pa[tt - 1].x, pa[tt - 1].y, pa[tt].x, pa[tt].y};
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          o[dt] = mfma16x16x32(pp, u32x4_t{bprev[dt].x, bprev[dt].y, bop[dt].x, bop[dt].y}, o[dt]);
      }
    } else {   // one tile per wave: the 16-deep MFMA
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] = mfma16x16x16(pa[tt], bop[dt], o[dt]);
    }
  }

  // ---- merge the NW waves into this chunk's partial ----
  if (lane < 16) { m_s[w][lane] = m; l_s[w][lane] = lsum; }
  // o[dt][i] = O[head 4*(l/16)+i][d = vc + dt]: NDT contiguous floats per head
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = (lane >> 4) * 4 + i;
    if (h < GQA)
#pragma unroll
      for (int q = 0; q < NDT / 4; ++q)
        *reinterpret_cast<f32x4_t*>(&o_s[w][h][vc + 4 * q]) =
            f32x4_t{o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]};
  }
  __syncthreads();
  // four consecutive d of one head per thread (one 16-byte store)
  for (int idx = threadIdx.x * 4; idx < GQA * D; idx += NW * 256) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < NW; ++q) M = fmaxf(M, m_s[q][h]);
    float L = 0.f;
    f32x4_t O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const float f = (m_s[q][h] == -INFINITY) ? 0.f : expf(m_s[q][h] - M);
      L += l_s[q][h] * f;
      O += *reinterpret_cast<const f32x4_t*>(&o_s[q][h][d]) * f;
    }
    const int hq = g * GQA + h;
    const long long po = (((long long)b * a.nq + hq) * a.n_chunks + c) * D + d;
    const long long ml = (((long long)b * a.nq + hq) * a.n_chunks + c) * 2;
    if constexpr (COH) {
      coh_st16(coh_rsrc(a.part_o), (int)(po * 4), __builtin_bit_cast(u32x4_t, O));
      if (d == 0) coh_st8(coh_rsrc(a.part_ml), (int)(ml * 4), __float_as_uint(M), __float_as_uint(L));
    } else {
      *reinterpret_cast<f32x4_t*>(a.part_o + po) = O;
      if (d == 0) *reinterpret_cast<float2*>(a.part_ml + ml) = float2{M, L};
    }
  }

  // the chunk holding the new token stages its k / v rows for the scatter
  if (NT == 1 && n >= chunk0 && n < chunk0 + CP)
    for (int i = threadIdx.x; i < D; i += NW * 64) {
      const long long ko = (((long long)b * 2 + 0) * a.nkv + g) * D + i;
      const long long vo = (((long long)b * 2 + 1) * a.nkv + g) * D + i;
      if constexpr (COH) {
        const __amdgpu_buffer_rsrc_t kr = coh_rsrc(a.kv_new);
        coh_st2(kr, (int)(ko * 2), kn_s[i]);
        coh_st2(kr, (int)(vo * 2), vn_s[i]);
      } else {
        a.kv_new[ko] = kn_s[i];
        a.kv_new[vo] = vn_s[i];
      }
    }
  if constexpr (COH) coh_publish(flag);
}

template <int D, int GQA, int TPW>
__global__ void __launch_bounds__(256) attn_fused_kernel(AttnArgs a, int rope_mode) {
  attn_chunk_block<D, GQA, TPW, false>(a, rope_mode, blockIdx.x, blockIdx.y, blockIdx.z, nullptr);
}

// Combine: block (head h, sequence b), 4 waves; wave w takes chunks w, w+4, ...
// in batches of U whose loads are all issued before any use, with a
// running (max, sum, O) per wave rescaled when a batch raises the max; the 4
// wave results then merge in LDS in wave order, with the sink logit if any.
// The new k / v rows of the scatter are loaded at the start as well.
// COH: the chunk partials and staged rows come from earlier blocks of the same
// launch -- one wave first waits for the n_wait flags at wait_fl (the kv group's
// chunk blocks), every read of them is device-coherent, the bf16 output is
// stored device-coherent and *flag is set at the end.
template <int D, int U, bool COH>
MKD_DEV void attn_combine_block(const AttnArgs& a, int h, int b, const unsigned* wait_fl, int n_wait,
                                unsigned* flag, unsigned* err) {
  constexpr int EL = D / 64;
  __shared__ float m_s[4], l_s[4];
  __shared__ float acc_s[4][D];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int CP = a.chunk;
  const int n = prior_len(a, b);
  const int nch = (n + new_tokens(a) + CP - 1) / CP;
  const long long ml0 = ((long long)b * a.nq + h) * a.n_chunks * 2;   // floats
  const long long po0 = ((long long)b * a.nq + h) * a.n_chunks * D;
  const __amdgpu_buffer_rsrc_t mlr = coh_rsrc(a.part_ml), por = coh_rsrc(a.part_o);
  // chunk k's (max, sum) and this lane's EL values of its O partial
  auto ld_ml = [&](int k) -> float2 {
    if constexpr (COH) {
      const coh_u32x2 v = coh_ld8(mlr, (int)((ml0 + 2 * k) * 4));
      return float2{__uint_as_float(v.x), __uint_as_float(v.y)};
    } else {
      return *reinterpret_cast<const float2*>(a.part_ml + ml0 + 2 * k);
    }
  };
  auto ld_po = [&](int k, float (&dst)[EL]) {
    const long long o = po0 + (long long)k * D + lane * EL;
    if constexpr (COH) {
      if constexpr (EL == 2) {
        const coh_u32x2 v = coh_ld8(por, (int)(o * 4));
        dst[0] = __uint_as_float(v.x);
        dst[1] = __uint_as_float(v.y);
      } else {
#pragma unroll
        for (int e = 0; e < EL; ++e) dst[e] = __uint_as_float(coh_ld4(por, (int)((o + e) * 4)));
      }
    } else {
#pragma unroll
      for (int e = 0; e < EL; ++e) dst[e] = a.part_o[o + e];
    }
  };
  if constexpr (COH) {
    if (w == 0) coh_wait_all(wait_fl, n_wait, err);
    __syncthreads();
  }

  // scatter operands: the first query head of each kv group writes that group's rows
  const int gqa = a.nq / a.nkv;
  const bool scatter = a.update_cache && h % gqa == 0 && threadIdx.x < D;
  uint16_t knew = 0, vnew = 0;
  if (scatter && a.s_tkg > 1) {   // several new tokens: row b's prepared k / v
    const int g = h / gqa;
    const uint16_t* src = a.prep + ((long long)b * a.nkv + g) * (gqa + 2) * D;
    knew = src[gqa * D + threadIdx.x];
    vnew = src[(gqa + 1) * D + threadIdx.x];
  } else if (scatter) {
    const int g = h / gqa;
    const long long ko = (((long long)b * 2 + 0) * a.nkv + g) * D + threadIdx.x;
    const long long vo = (((long long)b * 2 + 1) * a.nkv + g) * D + threadIdx.x;
    if constexpr (COH) {   // aligned dwords (a 16-bit load would be waited for at issue)
      const __amdgpu_buffer_rsrc_t kr = coh_rsrc(a.kv_new);
      const uint32_t kw = coh_ld4(kr, (int)((ko & ~1LL) * 2)), vw = coh_ld4(kr, (int)((vo & ~1LL) * 2));
      knew = (uint16_t)((ko & 1) ? kw >> 16 : kw);
      vnew = (uint16_t)((vo & 1) ? vw >> 16 : vw);
    } else {
      knew = a.kv_new[ko];
      vnew = a.kv_new[vo];
    }
  }

  float m = -INFINITY, L = 0.f, acc[EL];
#pragma unroll
  for (int e = 0; e < EL; ++e) acc[e] = 0.f;
  for (int k0 = w; k0 < nch; k0 += 4 * U) {
    float mk[U], lk[U], pv[U][EL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + 4 * u;
      const int kc = k < nch ? k : k0;       // in-range address; masked below
      const float2 mlv = ld_ml(kc);
      mk[u] = mlv.x;
      lk[u] = mlv.y;
      ld_po(kc, pv[u]);
      if (k >= nch) mk[u] = -INFINITY;
    }
    float bm = m;
#pragma unroll
    for (int u = 0; u < U; ++u) bm = fmaxf(bm, mk[u]);
    if (bm == -INFINITY) continue;           // nothing live yet (uniform)
    const float r = (m == -INFINITY) ? 0.f : expf(m - bm);
    L *= r;
#pragma unroll
    for (int e = 0; e < EL; ++e) acc[e] *= r;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float wk = mk[u] == -INFINITY ? 0.f : expf(mk[u] - bm);
      L += lk[u] * wk;
#pragma unroll
      for (int e = 0; e < EL; ++e) acc[e] += pv[u][e] * wk;
    }
    m = bm;
  }
#pragma unroll
  for (int e = 0; e < EL; ++e) acc_s[w][lane * EL + e] = acc[e];
  if (lane == 0) { m_s[w] = m; l_s[w] = L; }
  __syncthreads();
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    float M = fmaxf(fmaxf(m_s[0], m_s[1]), fmaxf(m_s[2], m_s[3]));
    if (a.sink) M = fmaxf(M, a.sink[h]);
    float Lt = 0.f, o = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float f = (m_s[q] == -INFINITY) ? 0.f : expf(m_s[q] - M);
      Lt += l_s[q] * f;
      o += acc_s[q][d] * f;
    }
    if (a.sink) Lt += expf(a.sink[h] - M);
    const uint16_t ov = (uint16_t)f2bf(Lt > 0.f ? o / Lt : 0.f);
    const long long oo = ((long long)b * a.nq + h) * D + d;
    if constexpr (COH) coh_st2(coh_rsrc(a.attn_out), (int)(oo * 2), ov);
    else a.attn_out[oo] = ov;
    // in-place KV scatter of the new rows (attention_block_tkg.py:1144-1470),
    // after every chunk has read the cache (kernels run in stream order)
    if (scatter) {
      const int g = h / gqa;
      const long long row = kv_write_row(a, b);
      if (row >= 0) {
        const long long off = a.block_table
                                  ? (row * a.nkv + g) * D + d
                                  : seq_of(a, b) * a.cache_b_stride + g * a.cache_h_stride + row * D + d;
        a.k_cache[off] = knew;
        a.v_cache[off] = vnew;
      }
    }
  }
  if constexpr (COH) coh_publish(flag);
}

template <int D, int U>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a) {
  attn_combine_block<D, U, false>(a, blockIdx.x, blockIdx.y, nullptr, 0, nullptr, nullptr);
}

// ---- joined launch: chunk blocks | combine blocks | projection blocks ----
constexpr int kJoinMaxF = 32;        // weight fragments per wave (nq * d <= 4096)
// The projection blocks start their weight stream this long after they start
// (wall clock, 100 MHz ticks): the chunk blocks' cache and projection loads,
// which the whole launch waits on, are served first; the weights still arrive
// long before the combine is done.  Measured at bs=1, Qwen3-30B-A3B shape,
// KV 2048 (decode step tok/s): no delay 320.5, 1 us 321.9, 1.5 us 324.4,
// 2.5 us 326.2, 4 us 324.7.
constexpr unsigned kJoinWeightDelay = 250;

// Output-projection block: 16 rows (row block rb) of y = attn_out . W_out^T for
// the B tokens, 4 waves over K quarters.  The weight fragments do not depend on
// the attention, so they are loaded first (after the start delay above); then
// one wave waits for the ncf
// combine flags, the B attention rows go to LDS (device-coherent loads), and
// the MFMAs run (A = weight fragment, B = tokens: lane l holds token l%16, k
// (l/16)*8 .. +8; D lane l holds rows 4*(l/16)+i of token l%16).  The wave
// partials are added in wave order.  With a router stage the rows are stored
// device-coherent and *oflag is set.
MKD_DEV void oproj_block(const AttnArgs& a, const AttnJoinArgs& j, int rb, const unsigned* cfl, int ncf,
                         unsigned* oflag) {
  extern __shared__ u32x4_t xs[];            // [B][K / 8]
  __shared__ f32x4_t red[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = a.nq * a.d, KB = K / 32, nf = KB / 4, kb0 = w * nf;
  // fragments past nf (K < 4096) repeat the last one and meet zero operands:
  // no branch in the unrolled loop
  {
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < kJoinWeightDelay) __builtin_amdgcn_s_sleep(2);
  }
  const uint16_t* wrow = j.w_out + ((long long)rb * KB + kb0) * 512 + lane * 8;
  u32x4_t wf[kJoinMaxF];
#pragma unroll
  for (int u = 0; u < kJoinMaxF; ++u)
    wf[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + min(u, nf - 1) * 512));
  if (w == 0) coh_wait_all(cfl, ncf, j.err);
  __syncthreads();
  const __amdgpu_buffer_rsrc_t xr = coh_rsrc(a.attn_out);
  const int per_row = K / 8, n16 = a.B * per_row;
  constexpr int kXs = kJoinMaxB * 4096 / 8 / 256;     // 16-byte pieces per thread at most
  u32x4_t xt[kXs];
#pragma unroll
  for (int q = 0; q < kXs; ++q) {
    const int i = threadIdx.x + 256 * q;
    if (i < n16) xt[q] = coh_ld16(xr, i * 16);
  }
#pragma unroll
  for (int q = 0; q < kXs; ++q) {
    const int i = threadIdx.x + 256 * q;
    if (i < n16) xs[i] = xt[q];
  }
  __syncthreads();
  const int c = lane & 15;
  const bool tok = c < a.B;
  const u32x4_t* xrow = xs + (tok ? c : 0) * per_row + (lane >> 4);
  f32x4_t acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // eight operand reads, then their eight MFMAs (masked, not branched)
#pragma unroll
  for (int u0 = 0; u0 < kJoinMaxF; u0 += 8) {
    u32x4_t xv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int u = u0 + q;
      const uint32_t m = (tok && u < nf) ? 0xffffffffu : 0u;
      const u32x4_t t = xrow[(kb0 + min(u, nf - 1)) * 4];
      xv[q] = u32x4_t{t[0] & m, t[1] & m, t[2] & m, t[3] & m};
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q & 3] = mfma16x16x32(wf[u0 + q], xv[q], acc[q & 3]);
  }
  red[w][lane] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (w == 0 && c < a.B) {
    const f32x4_t v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
    const int n0 = rb * 16 + (lane >> 4) * 4;
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = v[i] + ((j.bias && n0 + i < j.N) ? bf2f(j.bias[n0 + i]) : 0.f);
    if (j.rw) {   // read back by the router blocks (N % 16 == 0)
      coh_st16(coh_rsrc(j.y), (int)(((long long)c * j.N + n0) * 4),
               u32x4_t{__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])});
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n0 + i < j.N) j.y[(long long)c * j.N + n0 + i] = o[i];
    }
  }
  if (j.rw) coh_publish(oflag);
}

// ---- merge + projection blocks (one token, d = 128, with the router stage) ----
// Block (ks, nr) merges the chunk partials of query heads 4 ks .. +4 itself (one
// wave per head, the combine's online log-sum-exp merge over every chunk of the
// sequence) and projects them onto output rows 128 nr .. +128: the K-split
// partial ks of y = attn . W_out^T.  This folds the combine stage into the
// projection -- one flag hop and one device-coherent read of partials fewer
// than combine blocks followed by projection blocks.  Wave w holds row tiles
// 8 nr + 2 w, +1 over the block's whole 512-wide K slice (32 fragments), so no
// cross-wave sum is needed; the router blocks add the nq / 4 partials in order.
constexpr int kMpHeads = 4;                 // query heads per merge + projection block
constexpr int kMpRows = 128;                // output rows per block (d = 128)
constexpr int kMpBatch = 20;                // chunk partials in flight per wave (two waves per SIMD with the polling loop)
static_assert(kMpBatch <= 32, "one (max, sum) load per lane covers a batch");
constexpr int kMpMaxParts = 8;              // K slices (nq <= 32)

int attn_join_y_parts(int nq) { return nq % kMpHeads == 0 ? std::min(nq / kMpHeads, kMpMaxParts) : 1; }

__host__ __device__ static inline int attn_join_mp_blocks(int nq, int N) { return (nq / kMpHeads) * ((N + kMpRows - 1) / kMpRows); }

bool attn_join_mp_ok(const AttnArgs& a, const AttnJoinArgs& j) {
  return j.rw && a.B == 1 && a.d == 128 && a.nq % kMpHeads == 0 && a.s_tkg <= 1 && !a.prefill &&
         a.nq / kMpHeads <= kMpMaxParts && j.N <= 2048;
}

template <int GQA>
MKD_DEV void mp_block(const AttnArgs& a, const AttnJoinArgs& j, int ks, int nr, unsigned* oflag) {
  constexpr int D = 128, FT = kMpHeads * D / 32;    // fragments per row tile of the K slice (16)
  __shared__ __attribute__((aligned(16))) uint32_t ob_s[kMpHeads * D / 2];   // bf16 pairs of the 4 heads
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int N = j.N, KB = a.nq * D / 32, NRB = (N + 15) / 16;
  const int h0 = ks * kMpHeads, h = h0 + w;
  {
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < kJoinWeightDelay) __builtin_amdgcn_s_sleep(2);
  }
  u32x4_t wf[2][FT];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rt = min(nr * (kMpRows / 16) + w * 2 + i, NRB - 1);
    const uint16_t* wrow = j.w_out + ((long long)rt * KB + ks * FT) * 512 + lane * 8;
#pragma unroll
    for (int u = 0; u < FT; ++u)
      wf[i][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + u * 512));
  }
  // the chunk flags of the kv groups of the block's heads (with the data-polled
  // exchange the partials themselves are polled below)
  if (!j.dpoll) {
    if (w == 0) {
      const int g0 = h0 / GQA, g1 = (h0 + kMpHeads - 1) / GQA;
      for (int g = g0; g <= g1; ++g) coh_wait_all(j.flags + (long long)g * a.n_chunks, a.n_chunks, j.err);
    }
    __syncthreads();
  }

  // ---- merge head h: lane l of the ml load holds chunk c0 + l % 32, the
  // partial loads hold d = 2 l, 2 l + 1 of chunk c0 + u ----
  const int CP = a.chunk;
  const int n = prior_len(a, 0);
  const int nch = (n + 1 + CP - 1) / CP;
  const long long ml0 = (long long)h * a.n_chunks * 2, po0 = (long long)h * a.n_chunks * D;
  const __amdgpu_buffer_rsrc_t mlr = coh_rsrc(a.part_ml), por = coh_rsrc(a.part_o);
  float M = -INFINITY, Ls = 0.f, acc0 = 0.f, acc1 = 0.f;
  for (int c0 = 0; c0 < nch; c0 += kMpBatch) {
    const int cl = c0 + (lane & 31);
    const bool live = cl < nch && lane < kMpBatch;     // this batch's chunks only
    coh_u32x2 mlv;
    coh_u32x2 pv[kMpBatch];
    for (unsigned it = 0;; ++it) {
      mlv = coh_ld8(mlr, (int)((ml0 + 2 * min(cl, nch - 1)) * 4));
#pragma unroll
      for (int u = 0; u < kMpBatch; ++u)
        pv[u] = coh_ld8(por, (int)((po0 + (long long)min(c0 + u, nch - 1) * D + 2 * lane) * 4));
      if (!j.dpoll) break;
      // every word this wave reads written (kPollEmpty: not yet)
      bool ok = !live || (mlv.x != kPollEmpty && mlv.y != kPollEmpty);
#pragma unroll
      for (int u = 0; u < kMpBatch; ++u)
        ok = ok && (c0 + u >= nch || (pv[u].x != kPollEmpty && pv[u].y != kPollEmpty));
      if (__all(ok) || coh_poll_giveup(it, j.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    const float mk = live ? __uint_as_float(mlv.x) : -INFINITY;
    const float lk = live ? __uint_as_float(mlv.y) : 0.f;
    const float bm = fmaxf(M, wave_max(mk));
    if (bm == -INFINITY) continue;               // nothing live yet (uniform)
    const float r = M == -INFINITY ? 0.f : expf(M - bm);
    const float fk = mk == -INFINITY ? 0.f : expf(mk - bm);
    Ls = Ls * r + wave_sum(lk * fk);
    acc0 *= r;
    acc1 *= r;
#pragma unroll
    for (int u = 0; u < kMpBatch; ++u) {
      const float f = lane_f(fk, u);             // 0 past the last chunk
      acc0 += __uint_as_float(pv[u].x) * f;
      acc1 += __uint_as_float(pv[u].y) * f;
    }
    M = bm;
  }
  if (a.sink) {
    const float sk = a.sink[h];
    const float M2 = fmaxf(M, sk);
    const float r = M == -INFINITY ? 0.f : expf(M - M2);
    Ls = Ls * r + expf(sk - M2);
    acc0 *= r;
    acc1 *= r;
  }
  ob_s[w * (D / 2) + lane] = Ls > 0.f ? pack2bf(acc0 / Ls, acc1 / Ls) : 0u;
  __syncthreads();

  // ---- MFMAs: B operand lane l = token l % 16 (token 0 only), k (l / 16) * 8 .. + 8 ----
  const int c = lane & 15;
  const uint32_t m = c == 0 ? 0xffffffffu : 0u;
  const u32x4_t* xq = reinterpret_cast<const u32x4_t*>(ob_s) + (lane >> 4);
  f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int u = 0; u < FT; ++u) {
    const u32x4_t t = xq[u * 4];
    const u32x4_t xv = u32x4_t{t[0] & m, t[1] & m, t[2] & m, t[3] & m};
    acc[0] = mfma16x16x32(wf[0][u], xv, acc[0]);
    acc[1] = mfma16x16x32(wf[1][u], xv, acc[1]);
  }
  if (c == 0) {
    const __amdgpu_buffer_rsrc_t yr = coh_rsrc(j.y);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rt = nr * (kMpRows / 16) + w * 2 + i;
      const int n0 = rt * 16 + (lane >> 4) * 4;
      if (rt >= NRB || n0 >= N) continue;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = acc[i][e] + ((ks == 0 && j.bias) ? bf2f(j.bias[n0 + e]) : 0.f);
      coh_st16(yr, (int)(((long long)ks * N + n0) * 4),
               u32x4_t{__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])});
    }
  }
  if (!j.dpoll) coh_publish(oflag);
  // in-place KV scatter of the new rows (attention_block_tkg.py:1144-1470): the
  // first query head of each kv group, in the row-0 blocks, once every chunk of
  // the group has read the cache (its flags); nothing in this launch reads the
  // new rows, so the stores go after the block's results
  if (nr == 0 && a.update_cache && h % GQA == 0) {
    const int g = h / GQA;
    if (j.dpoll) coh_wait_all(j.flags + (long long)g * a.n_chunks, a.n_chunks, j.err);
    const long long row = kv_write_row(a, 0);
    if (row >= 0) {
      const __amdgpu_buffer_rsrc_t kr = coh_rsrc(a.kv_new);
      const long long ko = (long long)g * D + 2 * lane, vo = ((long long)a.nkv + g) * D + 2 * lane;
      const uint32_t kw = coh_ld4(kr, (int)(ko * 2)), vw = coh_ld4(kr, (int)(vo * 2));
      const long long off = a.block_table ? (row * a.nkv + g) * D + 2 * lane
                                          : g * a.cache_h_stride + row * D + 2 * lane;
      *reinterpret_cast<uint32_t*>(a.k_cache + off) = kw;
      *reinterpret_cast<uint32_t*>(a.v_cache + off) = vw;
    }
  }
}

// ---- one token, d = 128: the 512-thread form of the joined launch ----
// (chunk blocks of 8 waves x 16 positions, merge + projection blocks whose
// weight stream and merge polls run in different waves, K-sliced router blocks)
//
// A wave's vector loads complete in issue order, so a wave that streams 32
// weight fragments and then polls the chunk partials sees the partials only
// after its weights have arrived (measured: merged at 10.7 us, the chunk
// partials written by ~6 us).  Here waves 0-3 of a merge + projection block
// only stream the block's weights (the MFMA operands) and waves 4-7 only poll
// and merge one query head each, handing the bf16 head rows over in LDS.
template <int GQA>
MKD_DEV void mp_block8(const AttnArgs& a, const AttnJoinArgs& j, int ks, int nr) {
  constexpr int D = 128, FT = kMpHeads * D / 32;    // fragments per row tile of the K slice (16)
  __shared__ __attribute__((aligned(16))) uint32_t ob_s[kMpHeads * D / 2];   // bf16 pairs of the 4 heads
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int N = j.N, KB = a.nq * D / 32, NRB = (N + 15) / 16;
  const int h0 = ks * kMpHeads;
  u32x4_t wf[2][FT];
  if (w < 4) {
    // the block's weights: they depend on nothing, but are needed only after
    // the merge -- started after a short hold so that the chunk blocks' cache
    // and head loads, which the whole launch waits on, are served first
    {
      const unsigned long long t0 = wall_clock64();
      while (wall_clock64() - t0 < kJoinWeightDelay) __builtin_amdgcn_s_sleep(2);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rt = min(nr * (kMpRows / 16) + w * 2 + i, NRB - 1);
      const uint16_t* wrow = j.w_out + ((long long)rt * KB + ks * FT) * 512 + lane * 8;
#pragma unroll
      for (int u = 0; u < FT; ++u)
        wf[i][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + u * 512));
    }
  } else {
    // ---- merge head h = h0 + w - 4 (lane l of the ml load: chunk c0 + l % 32;
    // the partial loads: d = 2 l, 2 l + 1 of chunk c0 + u), polled until no word
    // holds the empty marker ----
    const int h = h0 + w - 4;
    const int CP = a.chunk;
    const int n = prior_len(a, 0);
    const int nch = (n + 1 + CP - 1) / CP;
    const long long ml0 = (long long)h * a.n_chunks * 2, po0 = (long long)h * a.n_chunks * D;
    const __amdgpu_buffer_rsrc_t mlr = coh_rsrc(a.part_ml), por = coh_rsrc(a.part_o);
    float M = -INFINITY, Ls = 0.f, acc0 = 0.f, acc1 = 0.f;
    for (int c0 = 0; c0 < nch; c0 += kMpBatch) {
      const int cl = c0 + (lane & 31);
      const bool live = cl < nch && lane < kMpBatch;
      coh_u32x2 mlv;
      coh_u32x2 pv[kMpBatch];
      for (unsigned it = 0;; ++it) {
        mlv = coh_ld8(mlr, (int)((ml0 + 2 * min(cl, nch - 1)) * 4));
#pragma unroll
        for (int u = 0; u < kMpBatch; ++u)
          pv[u] = coh_ld8(por, (int)((po0 + (long long)min(c0 + u, nch - 1) * D + 2 * lane) * 4));
        bool ok = !live || (mlv.x != kPollEmpty && mlv.y != kPollEmpty);
#pragma unroll
        for (int u = 0; u < kMpBatch; ++u)
          ok = ok && (c0 + u >= nch || (pv[u].x != kPollEmpty && pv[u].y != kPollEmpty));
        if (__all(ok) || coh_poll_giveup(it, j.err)) break;
        __builtin_amdgcn_s_sleep(1);
      }
      const float mk = live ? __uint_as_float(mlv.x) : -INFINITY;
      const float lk = live ? __uint_as_float(mlv.y) : 0.f;
      const float bm = fmaxf(M, wave_max(mk));
      if (bm == -INFINITY) continue;
      const float r = M == -INFINITY ? 0.f : expf(M - bm);
      const float fk = mk == -INFINITY ? 0.f : expf(mk - bm);
      Ls = Ls * r + wave_sum(lk * fk);
      acc0 *= r;
      acc1 *= r;
#pragma unroll
      for (int u = 0; u < kMpBatch; ++u) {
        const float f = lane_f(fk, u);
        acc0 += __uint_as_float(pv[u].x) * f;
        acc1 += __uint_as_float(pv[u].y) * f;
      }
      M = bm;
    }
    if (a.sink) {
      const float sk = a.sink[h];
      const float M2 = fmaxf(M, sk);
      const float r = M == -INFINITY ? 0.f : expf(M - M2);
      Ls = Ls * r + expf(sk - M2);
      acc0 *= r;
      acc1 *= r;
    }
    ob_s[(w - 4) * (D / 2) + lane] = Ls > 0.f ? pack2bf(acc0 / Ls, acc1 / Ls) : 0u;
    // in-place KV scatter of the new rows (attention_block_tkg.py:1144-1470):
    // the first query head of each kv group, in the row-0 blocks, once every
    // chunk of the group has read the cache (its flags); nothing in this
    // launch reads the new rows
    if (nr == 0 && a.update_cache && h % GQA == 0) {
      const int g = h / GQA;
      coh_wait_all(j.flags + (long long)g * a.n_chunks, a.n_chunks, j.err);
      const long long row = kv_write_row(a, 0);
      if (row >= 0) {
        const __amdgpu_buffer_rsrc_t kr = coh_rsrc(a.kv_new);
        const long long ko = (long long)g * D + 2 * lane, vo = ((long long)a.nkv + g) * D + 2 * lane;
        const uint32_t kw = coh_ld4(kr, (int)(ko * 2)), vw = coh_ld4(kr, (int)(vo * 2));
        const long long off = a.block_table ? (row * a.nkv + g) * D + 2 * lane
                                            : g * a.cache_h_stride + row * D + 2 * lane;
        *reinterpret_cast<uint32_t*>(a.k_cache + off) = kw;
        *reinterpret_cast<uint32_t*>(a.v_cache + off) = vw;
      }
    }
  }
  lds_barrier();   // ob_s; the weight waves' loads stay in flight
  if (w >= 4) return;
  // ---- MFMAs (waves 0-3): B operand lane l = token l % 16 (token 0 only) ----
  const int c = lane & 15;
  const uint32_t m = c == 0 ? 0xffffffffu : 0u;
  const u32x4_t* xq = reinterpret_cast<const u32x4_t*>(ob_s) + (lane >> 4);
  f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int u = 0; u < FT; ++u) {
    const u32x4_t t = xq[u * 4];
    const u32x4_t xv = u32x4_t{t[0] & m, t[1] & m, t[2] & m, t[3] & m};
    acc[0] = mfma16x16x32(wf[0][u], xv, acc[0]);
    acc[1] = mfma16x16x32(wf[1][u], xv, acc[1]);
  }
  if (c == 0) {
    const __amdgpu_buffer_rsrc_t yr = coh_rsrc(j.y);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int rt = nr * (kMpRows / 16) + w * 2 + i;
      const int n0 = rt * 16 + (lane >> 4) * 4;
      if (rt >= NRB || n0 >= N) continue;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = acc[i][e] + ((ks == 0 && j.bias) ? bf2f(j.bias[n0 + e]) : 0.f);
      coh_st16(yr, (int)(((long long)ks * N + n0) * 4),
               u32x4_t{__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])});
    }
  }
}

// K-sliced router block (one token): block kp owns the K slice [kp * KS, (kp
// + 1) * KS) of the 2048-wide residual (KS = 256: 8 fragments of 32) and every
// expert (wave w: expert row blocks w, w + 8, ...).  It reads only its slice of
// the projection's K-split partials (8 KB instead of the whole 64 KB rows),
// forms r = bf16(x + bf16(y)) there, stores that slice of r and the slice's
// sum of squares, and the partial logits sum_k W[e, k] * (r_k * gamma_k) of
// the slice (fp32 operand as bf16 hi + lo) -- the post-attention RMSNorm's
// 1 / rms is one factor of every logit, which the expert launch applies once
// it has added the slices' sums of squares (and with which it forms the
// experts' bf16 input (r * gamma) * rinv itself).
constexpr int kRsKb = 8;                      // fragments of 32 per K slice
MKD_DEV void router_kslice_block(const AttnJoinArgs& j, int kp) {
  __shared__ __attribute__((aligned(16))) u32x4_t ops[2][kRsKb * 4];   // hi / lo operands of the slice
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int N = j.N, KB = N / 32;
  const int KS = kRsKb * 32, k0 = kp * KS;
  const int nerb = j.E / 16;
  // the weights of the wave's expert row blocks (at most 2 per wave: E <= 256)
  u32x4_t wf[2][kRsKb];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (w + 8 * i >= nerb) break;               // wave-uniform
    const uint16_t* wrow = j.rw + ((long long)(w + 8 * i) * KB + kp * kRsKb) * 512 + lane * 8;
#pragma unroll
    for (int u = 0; u < kRsKb; ++u)
      wf[i][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + u * 512));
  }
  if (w == 0) {
    // lane l: elements k0 + 4 l .. + 4 of the slice -- the residual, gamma and
    // the o_parts partials of y (polled until no word holds the empty marker)
    const int k = k0 + 4 * lane;
    const uint2 xr = *reinterpret_cast<const uint2*>(j.rx + k);
    const uint2 gr = *reinterpret_cast<const uint2*>(j.rgamma + k);
    const __amdgpu_buffer_rsrc_t yr = coh_rsrc(j.y);
    u32x4_t p[kMpMaxParts];
    for (unsigned it = 0;; ++it) {
#pragma unroll
      for (int q = 0; q < kMpMaxParts; ++q) p[q] = coh_ld16(yr, (int)(((long long)min(q, j.o_parts - 1) * N + k) * 4));
      bool ok = true;
#pragma unroll
      for (int q = 0; q < kMpMaxParts; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) ok = ok && p[q][e] != kPollEmpty;
      if (__all(ok) || coh_poll_giveup(it, j.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    f32x4_t y = __builtin_bit_cast(f32x4_t, p[0]);
#pragma unroll
    for (int q = 1; q < kMpMaxParts; ++q)
      if (q < j.o_parts) y += __builtin_bit_cast(f32x4_t, p[q]);
    const float xv[4] = {bf_lo(xr.x), bf_hi(xr.x), bf_lo(xr.y), bf_hi(xr.y)};
    const float gv[4] = {bf_lo(gr.x), bf_hi(gr.x), bf_lo(gr.y), bf_hi(gr.y)};
    float r[4], ss = 0.f;
    uint32_t hi[2], lo[2];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[e] = rbf(xv[e] + rbf(y[e]));
      ss += r[e] * r[e];
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float v0 = r[2 * e] * gv[2 * e], v1 = r[2 * e + 1] * gv[2 * e + 1];
      const uint32_t h0 = f2bf(v0), h1 = f2bf(v1);
      hi[e] = h0 | (h1 << 16);
      lo[e] = f2bf(v0 - bf2f(h0)) | (f2bf(v1 - bf2f(h1)) << 16);
    }
    *reinterpret_cast<uint2*>(j.rresid + k) = uint2{pack2bf(r[0], r[1]), pack2bf(r[2], r[3])};
    // operands in B order: 16-byte piece lane / 2 (8 elements), half lane % 2
    reinterpret_cast<uint2*>(ops[0])[lane] = uint2{hi[0], hi[1]};
    reinterpret_cast<uint2*>(ops[1])[lane] = uint2{lo[0], lo[1]};
    ss = wave_sum(ss);
    if (lane == 0) j.rss[kp] = ss;
  }
  lds_barrier();   // the operands; the weight loads stay in flight
  // MFMAs: B lane l = token l % 16 (token 0 only), k (l / 16) * 8 .. + 8 of each fragment
  const int c = lane & 15;
  const uint32_t m = c == 0 ? 0xffffffffu : 0u;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int erb = w + 8 * i;
    if (erb >= nerb) break;                     // wave-uniform
    f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int u = 0; u < kRsKb; ++u) {
      const u32x4_t h = ops[0][u * 4 + (lane >> 4)], l = ops[1][u * 4 + (lane >> 4)];
      acc[0] = mfma16x16x32(wf[i][u], u32x4_t{h[0] & m, h[1] & m, h[2] & m, h[3] & m}, acc[0]);
      acc[1] = mfma16x16x32(wf[i][u], u32x4_t{l[0] & m, l[1] & m, l[2] & m, l[3] & m}, acc[1]);
    }
    if (c == 0)
      *reinterpret_cast<f32x4_t*>(j.rparts + (long long)kp * j.E + erb * 16 + (lane >> 4) * 4) = acc[0] + acc[1];
  }
}

// The 512-thread joined launch at one token (d = 128): chunk blocks (8 waves x
// 16 positions: 128-position chunks), merge + projection blocks, K-sliced
// router blocks.
template <int GQA>
__global__ void __launch_bounds__(512) attn_joined_mp_kernel(AttnArgs a, AttnJoinArgs j, int rope_mode) {
  const int bid = blockIdx.x;
  const int na = a.n_chunks * a.nkv;
  if (bid < na) {
    if (!a.mask && !a.block_table && !a.prep)
      attn_chunk_block<128, GQA, 1, true, 8, true>(a, rope_mode, bid % a.n_chunks, bid / a.n_chunks, 0, j.flags + bid);
    else
      attn_chunk_block<128, GQA, 1, true, 8>(a, rope_mode, bid % a.n_chunks, bid / a.n_chunks, 0, j.flags + bid);
    return;
  }
  const int ksn = a.nq / kMpHeads, nmp = attn_join_mp_blocks(a.nq, j.N);
  if (bid < na + nmp) {
    const int q = bid - na;
    mp_block8<GQA>(a, j, q % ksn, q / ksn);
  } else {
    router_kslice_block(j, bid - na - nmp);
  }
}

int attn_join_kslice_parts(int B, int nq, int nkv, int d, int S_max, int E, int N) {
  const int gqa = nkv > 0 ? nq / nkv : 0;
  if (B != 1 || d != 128 || nq % kMpHeads || nq / kMpHeads > kMpMaxParts || gqa * nkv != nq ||
      (gqa != 1 && gqa != 2 && gqa != 4 && gqa != 8 && gqa != 16) || E % 16 || E > 256 ||
      N % (kRsKb * 32) || N / (kRsKb * 32) > 8 || N > 2048 || attn_chunk_for(B, nkv, S_max) != 128)
    return 0;
  // one block per CU (512 threads, > 128 VGPRs): the whole grid resident at once
  const int blocks = (S_max + 1 + 127) / 128 * nkv + attn_join_mp_blocks(nq, N) + N / (kRsKb * 32);
  const int cus = device_cus();
  if (cus <= 0 || blocks > cus) return 0;
  return N / (kRsKb * 32);
}

bool attn_join_kslice_ok(const AttnArgs& a, const AttnJoinArgs& j) {
  return attn_join_mp_ok(a, j) && a.chunk == 128 && j.E % 16 == 0 && j.E <= 256 && j.N % (kRsKb * 32) == 0 &&
         j.N / (kRsKb * 32) <= 8 && j.rx_f32 && j.o_parts <= kMpMaxParts;
}

// ---- router stage: the post-attention residual, norm and router logits ----
constexpr int kJoinRouterF = 8;      // router weight fragments per wave
constexpr int kJoinRouterMaxN = 3072;

__host__ __device__ static inline int router_parts_of(int N) { return (N / 32 + kJoinRouterF - 1) / kJoinRouterF; }
int attn_join_router_parts(int N) { return router_parts_of(N); }

static int router_join_blocks(int E, int N) { return ((E / 16) * router_parts_of(N) + 3) / 4; }

bool attn_join_router_supported(int B, int E, int N) {
  return B >= 1 && B <= kJoinMaxB && E >= 16 && E % 16 == 0 && E <= 512 && N % 32 == 0 &&
         N <= kJoinRouterMaxN && router_parts_of(N) <= 16;
}

// Router block rbk (after the projection blocks): wave gw = 4 rbk + w computes
// experts 16 erb .. +16 over the K part kp (kJoinRouterF fragments of 32) of
// the router GEMM, as router_norm_gemm_kernel does (router_topk.py:69-1207 with
// the Qwen fused post-attention norm, moe_fused_nki.py:159-276): the weights,
// the residual rows and gamma are loaded first; one wave waits for the nof
// projection flags; the block then reads the projection rows device-coherent,
// forms r = bf16(x + bf16(y)) and each token's sum of squares (in a fixed
// order: thread, wave, then waves 0..3), and writes y = (r * gamma) * rinv once
// to LDS in B-operand order (bf16 hi + lo for an fp32 router input, one 16-byte
// piece per thread and row chunk), from where every wave reads its operands.
// Block 0 also writes r and bf16(y), the residual and expert input of the rest
// of the layer.
// RC = the row chunks (16 bytes) per thread, ceil(B N / 8 / 256).
template <int RC, int PM>
MKD_DEV void router_block(const AttnArgs& a, const AttnJoinArgs& j, int rbk, const unsigned* ofl, int nof) {
  extern __shared__ u32x4_t xs[];             // [B][N / 8] y hi, [B][N / 8] y lo, [N / 8] gamma
  __shared__ float ssw[4][kJoinMaxB];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int N = j.N, KB = N / 32, nkp = router_parts_of(N);
  const int nwv = (j.E / 16) * nkp;
  const int gw = min(rbk * 4 + w, nwv - 1);   // a wave past the last one repeats it, storing nothing
  const bool wlive = rbk * 4 + w < nwv;
  const int erb = gw / nkp, kp = gw % nkp;
  const int kb0 = kp * kJoinRouterF, nf = min(kJoinRouterF, KB - kb0);
  const int B = a.B, per_row = N / 8, nch = B * per_row;
  constexpr int kRC = RC;
  constexpr int kGC = kJoinRouterMaxN / 8 / 256 + 1;           // gamma chunks per thread at most
  u32x4_t xr[kRC], gr[kGC];
#pragma unroll
  for (int q = 0; q < kRC; ++q) {
    const int i = min((int)threadIdx.x + 256 * q, nch - 1);
    xr[q] = ld16(j.rx + (long long)i * 8);
  }
#pragma unroll
  for (int q = 0; q < kGC; ++q) gr[q] = ld16(j.rgamma + min((int)threadIdx.x + 256 * q, per_row - 1) * 8);
  {
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < kJoinWeightDelay) __builtin_amdgcn_s_sleep(2);
  }
  const uint16_t* wrow = j.rw + ((long long)erb * KB + kb0) * 512 + lane * 8;
  u32x4_t wf[kJoinRouterF];
#pragma unroll
  for (int u = 0; u < kJoinRouterF; ++u)
    wf[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + min(u, nf - 1) * 512));
  if (!j.dpoll) {
    if (w == 0) coh_wait_all(ofl, nof, j.err);
    __syncthreads();
  }

  // r = bf16(x + bf16(y)) (kept in registers), per-token sums of squares; y is
  // the sum of the j.o_parts K-split partials (PM at most), in order (with the
  // data-polled exchange, loaded until no word reads kPollEmpty)
  const __amdgpu_buffer_rsrc_t yr = coh_rsrc(j.y);
  u32x4_t y0[kRC], y1[kRC];
  {
    u32x4_t p0[kRC][PM], p1[kRC][PM];
    for (unsigned it = 0;; ++it) {
#pragma unroll
      for (int q = 0; q < kRC; ++q) {
        const int i = min((int)threadIdx.x + 256 * q, nch - 1);
#pragma unroll
        for (int pp = 0; pp < PM; ++pp) {
          const int off = (min(pp, j.o_parts - 1) * nch + i) * 32;
          p0[q][pp] = coh_ld16(yr, off);
          p1[q][pp] = coh_ld16(yr, off + 16);
        }
      }
      if (!j.dpoll) break;
      bool ok = true;
#pragma unroll
      for (int q = 0; q < kRC; ++q)
#pragma unroll
        for (int pp = 0; pp < PM; ++pp)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            ok = ok && p0[q][pp][e] != kPollEmpty && p1[q][pp][e] != kPollEmpty;
      if (__all(ok) || coh_poll_giveup(it, j.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int q = 0; q < kRC; ++q) {
      f32x4_t s0 = __builtin_bit_cast(f32x4_t, p0[q][0]), s1 = __builtin_bit_cast(f32x4_t, p1[q][0]);
#pragma unroll
      for (int pp = 1; pp < PM; ++pp)
        if (pp < j.o_parts) {
          s0 += __builtin_bit_cast(f32x4_t, p0[q][pp]);
          s1 += __builtin_bit_cast(f32x4_t, p1[q][pp]);
        }
      y0[q] = __builtin_bit_cast(u32x4_t, s0);
      y1[q] = __builtin_bit_cast(u32x4_t, s1);
    }
  }
  u32x4_t* yhi = xs;
  u32x4_t* ylo = xs + nch;
  u32x4_t* gs = xs + 2 * nch;
#pragma unroll
  for (int q = 0; q < kGC; ++q) {
    const int i = (int)threadIdx.x + 256 * q;
    if (i < per_row) gs[i] = gr[q];
  }
  float ss[kJoinMaxB] = {0.f, 0.f, 0.f, 0.f};
  u32x4_t rreg[kRC];
#pragma unroll
  for (int q = 0; q < kRC; ++q) {
    const int i = (int)threadIdx.x + 256 * q;
    const int t = i / per_row;
    const float yv[8] = {__uint_as_float(y0[q][0]), __uint_as_float(y0[q][1]), __uint_as_float(y0[q][2]),
                         __uint_as_float(y0[q][3]), __uint_as_float(y1[q][0]), __uint_as_float(y1[q][1]),
                         __uint_as_float(y1[q][2]), __uint_as_float(y1[q][3])};
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float r0 = rbf(bf_lo(xr[q][e]) + rbf(yv[2 * e]));
      const float r1 = rbf(bf_hi(xr[q][e]) + rbf(yv[2 * e + 1]));
      s += r0 * r0;
      s += r1 * r1;
      rreg[q][e] = pack2bf(r0, r1);
    }
#pragma unroll
    for (int tt = 0; tt < kJoinMaxB; ++tt)
      if (tt == t && i < nch) ss[tt] += s;
  }
#pragma unroll
  for (int tt = 0; tt < kJoinMaxB; ++tt) {
    const float v = wave_sum(ss[tt]);
    if (lane == 0) ssw[w][tt] = v;
  }
  __syncthreads();
  float rinv[kJoinMaxB];
#pragma unroll
  for (int tt = 0; tt < kJoinMaxB; ++tt)
    rinv[tt] = 1.0f / sqrtf((((ssw[0][tt] + ssw[1][tt]) + ssw[2][tt]) + ssw[3][tt]) * j.rinv_h + j.reps);

  // y = (r * gamma) * rinv of the thread's chunks -> LDS (hi, lo); block 0 also
  // writes r and bf16(y)
#pragma unroll
  for (int q = 0; q < kRC; ++q) {
    const int i = (int)threadIdx.x + 256 * q;
    if (i >= nch) continue;
    const int t = i / per_row;
    float rv = rinv[0];
#pragma unroll
    for (int tt = 1; tt < kJoinMaxB; ++tt)
      if (tt == t) rv = rinv[tt];
    const u32x4_t gp = gs[i - t * per_row];
    u32x4_t hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v0 = (bf_lo(rreg[q][e]) * bf_lo(gp[e])) * rv;
      float v1 = (bf_hi(rreg[q][e]) * bf_hi(gp[e])) * rv;
      if (!j.rx_f32) { v0 = rbf(v0); v1 = rbf(v1); }
      const uint32_t h0 = f2bf(v0), h1 = f2bf(v1);
      hi[e] = h0 | (h1 << 16);
      lo[e] = f2bf(v0 - bf2f(h0)) | (f2bf(v1 - bf2f(h1)) << 16);
    }
    yhi[i] = hi;
    ylo[i] = lo;
    if (rbk == 0) {
      st16(j.rresid + (long long)i * 8, rreg[q]);
      st16(j.rhnorm + (long long)i * 8, hi);
    }
  }
  __syncthreads();

  // MFMAs: lane l = token l%16, k (l/16)*8 .. +8 of each fragment (masked, not branched)
  const int c = lane & 15;
  const bool tok = c < B;
  const int o0 = (tok ? c : 0) * per_row + (lane >> 4);
  f32x4_t acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kJoinRouterF; ++u) {
    const int o = o0 + (kb0 + min(u, nf - 1)) * 4;
    const uint32_t m = (tok && u < nf) ? 0xffffffffu : 0u;
    const u32x4_t h = yhi[o], l = ylo[o];
    acc[u & 1] = mfma16x16x32(wf[u], u32x4_t{h[0] & m, h[1] & m, h[2] & m, h[3] & m}, acc[u & 1]);
    if (j.rx_f32)
      acc[2 + (u & 1)] = mfma16x16x32(wf[u], u32x4_t{l[0] & m, l[1] & m, l[2] & m, l[3] & m}, acc[2 + (u & 1)]);
  }
  if (wlive && tok) {
    const f32x4_t v = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    float* pp = j.rparts + (long long)kp * B * j.E + (long long)c * j.E + erb * 16 + (lane >> 4) * 4;
    *reinterpret_cast<f32x4_t*>(pp) = v;
  }
}

template <int D, int GQA, int TPW>
__global__ void __launch_bounds__(256) attn_joined_kernel(AttnArgs a, AttnJoinArgs j, int rope_mode) {
  const int bid = blockIdx.x;
  const int na = a.n_chunks * a.nkv * a.B, nc = a.nq * a.B;
  if (bid < na) {
    const int c = bid % a.n_chunks, gb = bid / a.n_chunks;
    attn_chunk_block<D, GQA, TPW, true>(a, rope_mode, c, gb % a.nkv, gb / a.nkv, j.flags + bid);
    return;
  }
  if (j.mp) {   // merge + projection blocks, then the router blocks
    const int ksn = a.nq / kMpHeads, nmp = attn_join_mp_blocks(a.nq, j.N);
    if (bid < na + nmp) {
      const int q = bid - na;
      if constexpr (D == 128) mp_block<GQA>(a, j, q % ksn, q / ksn, j.flags + na + nc + q);
    } else {
      // one token of N <= 2048 (attn_join_mp_ok): one row chunk per thread
      router_block<1, kMpMaxParts>(a, j, bid - na - nmp, j.flags + na + nc, nmp);
    }
    return;
  }
  if (bid < na + nc) {
    const int hb = bid - na, h = hb % a.nq, b = hb / a.nq;
    attn_combine_block<D, 16, true>(a, h, b, j.flags + ((long long)b * a.nkv + h / GQA) * a.n_chunks,
                                    a.n_chunks, j.flags + bid, j.err);
  } else if (bid < na + nc + (j.N + 15) / 16) {
    const int rb = bid - na - nc;
    oproj_block(a, j, rb, j.flags + na, nc, j.flags + na + nc + rb);
  } else {
    const int rbk = bid - na - nc - (j.N + 15) / 16, no = (j.N + 15) / 16;
    switch ((a.B * j.N / 8 + 255) / 256) {   // row chunks per thread
      case 1: router_block<1, 1>(a, j, rbk, j.flags + na + nc, no); break;
      case 2: router_block<2, 1>(a, j, rbk, j.flags + na + nc, no); break;
      case 3: router_block<3, 1>(a, j, rbk, j.flags + na + nc, no); break;
      case 4: router_block<4, 1>(a, j, rbk, j.flags + na + nc, no); break;
      case 5: router_block<5, 1>(a, j, rbk, j.flags + na + nc, no); break;
      default: router_block<6, 1>(a, j, rbk, j.flags + na + nc, no); break;
    }
  }
}

// chunk flags, combine flags, projection flags (router stage)
int attn_join_flag_words(int B, int nq, int nkv, int n_chunks, int N) {
  return n_chunks * nkv * B + nq * B + (N + 15) / 16;
}

bool attn_join_supported(const AttnArgs& a, int N) {
  const int gqa = a.nkv > 0 ? a.nq / a.nkv : 0;
  const int K = a.nq * a.d;
  return !a.prep && !a.prefill && a.s_tkg <= 1 && a.B >= 1 && a.B <= kJoinMaxB && (a.chunk == 64 || a.chunk == 128) &&
         (a.d == 64 || a.d == 128) && (gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8 || gqa == 16) &&
         gqa * a.nkv == a.nq && K % 128 == 0 && K / 128 <= kJoinMaxF && N > 0 &&
         (long long)a.B * K * 2 <= 32768;
}

template <int D, int GQA>
static hipError_t launch_join(const AttnArgs& a, const AttnJoinArgs& j, int rope_mode, hipStream_t s) {
  const int blocks = a.n_chunks * a.nkv * a.B +
                     (j.mp ? attn_join_mp_blocks(a.nq, j.N) : a.nq * a.B + (j.N + 15) / 16) +
                     (j.rw ? router_join_blocks(j.E, j.N) : 0);
  const size_t lds = std::max((size_t)a.B * a.nq * a.d * 2, j.rw ? (size_t)(2 * a.B + 1) * j.N * 2 : 0);
  if (a.chunk == 64) return timed_launch(attn_joined_kernel<D, GQA, 1>, dim3(blocks), dim3(256), lds, s, a, j, rope_mode);
  return timed_launch(attn_joined_kernel<D, GQA, 2>, dim3(blocks), dim3(256), lds, s, a, j, rope_mode);
}

hipError_t attn_join_launch(const AttnArgs& ain, const AttnJoinArgs& jin, int rope_mode, hipStream_t s) {
  AttnJoinArgs j = jin;
  AttnArgs a = ain;
  j.mp = attn_join_mp_ok(a, j) ? 1 : 0;
  j.o_parts = j.mp ? a.nq / kMpHeads : 1;
  j.dpoll = (j.mp && j.poll_po && j.poll_pml && j.poll_y) ? 1 : 0;
  if (j.dpoll) {   // this launch's own exchange buffers, filled with kPollEmpty
    a.part_o = j.poll_po;
    a.part_ml = j.poll_pml;
    j.y = j.poll_y;
  }
  if (!attn_join_supported(a, j.N) || !j.w_out || !j.y || !j.flags || !j.err) return hipErrorInvalidValue;
  if (j.rw && (!attn_join_router_supported(a.B, j.E, j.N) || j.N % 16 || !j.rx || !j.rgamma ||
               !j.rparts || !j.rresid || !j.rhnorm))
    return hipErrorInvalidValue;
  if (j.rss) {   // the K-sliced router form (the 512-thread launch)
    if (!j.dpoll || !attn_join_kslice_ok(a, j)) return hipErrorInvalidValue;
    const int blocks = a.n_chunks * a.nkv + attn_join_mp_blocks(a.nq, j.N) + j.N / (kRsKb * 32);
    switch (a.nq / a.nkv) {
      case 1: return timed_launch(attn_joined_mp_kernel<1>, dim3(blocks), dim3(512), 0, s, a, j, rope_mode);
      case 2: return timed_launch(attn_joined_mp_kernel<2>, dim3(blocks), dim3(512), 0, s, a, j, rope_mode);
      case 4: return timed_launch(attn_joined_mp_kernel<4>, dim3(blocks), dim3(512), 0, s, a, j, rope_mode);
      case 8: return timed_launch(attn_joined_mp_kernel<8>, dim3(blocks), dim3(512), 0, s, a, j, rope_mode);
      case 16: return timed_launch(attn_joined_mp_kernel<16>, dim3(blocks), dim3(512), 0, s, a, j, rope_mode);
    }
    return hipErrorInvalidValue;
  }
  const int gqa = a.nq / a.nkv;
  if (a.d == 128) {
    switch (gqa) {
      case 1: return launch_join<128, 1>(a, j, rope_mode, s);
      case 2: return launch_join<128, 2>(a, j, rope_mode, s);
      case 4: return launch_join<128, 4>(a, j, rope_mode, s);
      case 8: return launch_join<128, 8>(a, j, rope_mode, s);
      case 16: return launch_join<128, 16>(a, j, rope_mode, s);
    }
  } else {
    switch (gqa) {
      case 1: return launch_join<64, 1>(a, j, rope_mode, s);
      case 2: return launch_join<64, 2>(a, j, rope_mode, s);
      case 4: return launch_join<64, 4>(a, j, rope_mode, s);
      case 8: return launch_join<64, 8>(a, j, rope_mode, s);
      case 16: return launch_join<64, 16>(a, j, rope_mode, s);
    }
  }
  return hipErrorInvalidValue;
}

template <int D, int GQA, int TPW>
static hipError_t launch_attn(const AttnArgs& a, int rope_mode, hipStream_t s) {
  return timed_launch(attn_fused_kernel<D, GQA, TPW>, dim3(a.n_chunks, a.nkv, a.B), dim3(256), 0, s,
                      a, rope_mode);
}

template <int D, int GQA>
static hipError_t launch_tpw(const AttnArgs& a, int rope_mode, hipStream_t s) {
  if (a.prefill && (!a.prep || !a.update_cache)) return hipErrorInvalidValue;
  if (a.s_tkg > 1 && (!a.prep || a.prefill || a.window > 0 || a.B % a.s_tkg)) return hipErrorInvalidValue;
  if (a.prep) {   // (a prefill pass: the prepared k / v rows go to the cache as well)
    launch_prep<D, GQA>(a, rope_mode, s, a.prefill);
    if (hipError_t e = hipGetLastError()) return e;
  }
  const int chunk = a.chunk;
  if (chunk == 64) return launch_attn<D, GQA, 1>(a, rope_mode, s);
  if (chunk == 128) return launch_attn<D, GQA, 2>(a, rope_mode, s);
  if (chunk == 256) return launch_attn<D, GQA, 4>(a, rope_mode, s);
  return hipErrorInvalidValue;
}

int attn_chunk_for(int B, int nkv, int S_max) {
  // positions per block: enough blocks to cover the CUs several times over
  for (int chunk : {256, 128}) {
    const long long blocks = (long long)B * nkv * ((S_max + 1 + chunk - 1) / chunk);
    if (blocks >= 1024) return chunk;
  }
  // one token: 128, so that the joined launch's merge + projection blocks read
  // the chunk partials of a head in one batch up to 2560 positions (measured at
  // KV 2048, Qwen3-30B-A3B shape: 384.0 against 382.0 tok/s with 64)
  return B == 1 ? 128 : 64;
}

hipError_t attn_combine_launch(const AttnArgs& a, hipStream_t s) {
  // chunks per wave in one batch of loads: 8 covers up to 32 chunks
  const bool small = a.n_chunks <= 32;
  if (a.d == 128) {
    if (small) hipLaunchKernelGGL((attn_combine_kernel<128, 8>), dim3(a.nq, a.B), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((attn_combine_kernel<128, 16>), dim3(a.nq, a.B), dim3(256), 0, s, a);
  } else if (a.d == 64) {
    if (small) hipLaunchKernelGGL((attn_combine_kernel<64, 8>), dim3(a.nq, a.B), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((attn_combine_kernel<64, 16>), dim3(a.nq, a.B), dim3(256), 0, s, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t attn_prep_launch(const AttnArgs& a, int rope_mode, hipStream_t s) {
  if (!a.prep) return hipErrorInvalidValue;
  const int gqa = a.nq / a.nkv;
#define MKD_PREP(D, G) launch_prep<D, G>(a, rope_mode, s)
  if (a.d == 128) {
    switch (gqa) {
      case 1: MKD_PREP(128, 1); break;
      case 2: MKD_PREP(128, 2); break;
      case 4: MKD_PREP(128, 4); break;
      case 8: MKD_PREP(128, 8); break;
      case 16: MKD_PREP(128, 16); break;
      default: return hipErrorInvalidValue;
    }
  } else if (a.d == 64) {
    switch (gqa) {
      case 1: MKD_PREP(64, 1); break;
      case 2: MKD_PREP(64, 2); break;
      case 4: MKD_PREP(64, 4); break;
      case 8: MKD_PREP(64, 8); break;
      case 16: MKD_PREP(64, 16); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
  }
#undef MKD_PREP
  return hipGetLastError();
}

template <int D, int GQA>
static hipError_t launch_prep_write(const AttnArgs& a, int rope_mode, hipStream_t s) {
  launch_prep<D, GQA>(a, rope_mode, s, true);
  return hipGetLastError();
}

hipError_t attn_prep_write_launch(const AttnArgs& a, int rope_mode, hipStream_t s) {
  if (!a.prep || !a.prefill || !a.update_cache) return hipErrorInvalidValue;
  const int gqa = a.nq / a.nkv;
#define MKD_PW(D_)                                              \
  switch (gqa) {                                                \
    case 1: return launch_prep_write<D_, 1>(a, rope_mode, s);   \
    case 2: return launch_prep_write<D_, 2>(a, rope_mode, s);   \
    case 4: return launch_prep_write<D_, 4>(a, rope_mode, s);   \
    case 8: return launch_prep_write<D_, 8>(a, rope_mode, s);   \
    case 16: return launch_prep_write<D_, 16>(a, rope_mode, s); \
  }
  if (a.d == 128) { MKD_PW(128) }
  else if (a.d == 64) { MKD_PW(64) }
#undef MKD_PW
  return hipErrorInvalidValue;
}

hipError_t attn_decode_launch(const AttnArgs& a, int rope_mode, hipStream_t s) {
  const int gqa = a.nq / a.nkv;
  if (a.d == 128) {
    switch (gqa) {
      case 1: return launch_tpw<128, 1>(a, rope_mode, s);
      case 2: return launch_tpw<128, 2>(a, rope_mode, s);
      case 4: return launch_tpw<128, 4>(a, rope_mode, s);
      case 8: return launch_tpw<128, 8>(a, rope_mode, s);
      case 16: return launch_tpw<128, 16>(a, rope_mode, s);
    }
  } else if (a.d == 64) {
    switch (gqa) {
      case 1: return launch_tpw<64, 1>(a, rope_mode, s);
      case 2: return launch_tpw<64, 2>(a, rope_mode, s);
      case 4: return launch_tpw<64, 4>(a, rope_mode, s);
      case 8: return launch_tpw<64, 8>(a, rope_mode, s);
      case 16: return launch_tpw<64, 16>(a, rope_mode, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace mkd
