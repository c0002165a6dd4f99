// Weight-streaming skinny GEMM for decode:  Y[t, n] = sum_k X[t, k] * W[n, k]
//
// Decode GEMMs have a handful of tokens (1..128) against large weight matrices,
// so they are HBM-bound on the weight stream.  Weights are repacked once into
// MFMA fragment order ("frag layout"):
//
//   packed[nb][kb][lane][j] = W[nb*16 + lane%16][kb*32 + (lane/16)*8 + j]
//
// i.e. one v_mfma_f32_16x16x32_bf16 A-operand (16 rows x 32 k) is a contiguous
// 1 KiB block and every wave-wide 16-byte load is one fully coalesced 1 KiB
// transaction.  A row block of 16 output features is a contiguous 16*K*2-byte
// run, so a wave streams straight through HBM.
//
// Work split: block = nsplit waves, all on the same 16-row block (RB = 2 row
// blocks for the fused gate/up case), each wave owning K/nsplit of the
// contraction; partial 16x16 tiles are reduced through LDS in a fixed order
// (deterministic), then one epilogue is applied.  Tokens sit in the MFMA N
// dimension (16 per tile, TN tiles per block).
//
// Grouped mode (MoE): blockIdx.y selects a routed expert group; the group's
// token rows come from the routing tables and the expert's weights from
// w + expert * w_group_stride.
#include "common.h"
#include "gemm_epi.h"
#include "gemm_frag.h"
#include "mkd_internal.h"
#include "router_select.h"
#include "coherent.h"
#include "poll_word.h"

namespace mkd {

// ---------------------------------------------------------------------------
// Packing: any [G][N][K] (k-contiguous) or [G][K][N] (n-contiguous) bf16 source
// into frag layout.  `interleave_half` > 0 reorders row blocks as
// [rows 0..15 | rows h..h+15 | rows 16..31 | rows h+16..h+31 | ...] with
// h = interleave_half, which puts a gate block next to its up block.
// ---------------------------------------------------------------------------
__global__ void pack_frag_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                 int G, int N, int K, long long src_g_stride,
                                 long long src_row_stride, long long src_col_stride,
                                 int interleave_half) {
  // N is the logical row count; the packed matrix has ceil(N/16)*16 rows, the
  // padding rows are zero.
  const int KB = K / 32, NB = (N + 15) / 16;
  const long long total = (long long)G * NB * KB * 64;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    long long r = idx >> 6;
    const int kb = (int)(r % KB); r /= KB;
    const int nb = (int)(r % NB);
    const int g = (int)(r / NB);
    int row_block = nb;
    if (interleave_half > 0) {
      const int pair = nb >> 1;
      row_block = (nb & 1) ? (interleave_half / 16 + pair) : pair;
    }
    const int n = row_block * 16 + (lane & 15);
    const int k0 = kb * 32 + (lane >> 4) * 8;
    uint16_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (n < N) {
      const uint16_t* s = src + g * src_g_stride + n * src_row_stride + k0 * src_col_stride;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = s[j * src_col_stride];
    }
    uint16_t* d = dst + idx * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) d[j] = v[j];
  }
}

template <int RB, int TN, bool XF32, int EPI>
__global__ void __launch_bounds__(1024) gemm_frag_kernel(GemmArgs a) {
  frag_body<RB, TN, XF32, EPI>(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Grouped gate/up + SwiGLU with the router top-k folded in, for a few tokens
// (router_topk.py:868-887 selection, moe_tkg gate/up): every block forms the
// top-k, the routing weights and the expert groups of all T tokens from the
// router's split-K partial logits itself (select_small: the values of
// router_select_kernel), keeps the tables in LDS for its own columns, and block
// (0,0,0) also writes them out for the down projection.  The partials are
// T * E * nparts floats read from L2 by every block; the select launch and its
// dependent round trip leave the decode step.
template <int PER>
__global__ void __launch_bounds__(1024) gemm_frag_sel_kernel(GemmArgs a, RouterArgs r) {
  __shared__ int s_ng;
  __shared__ int s_gexp[kSelMaxPairs], s_gcnt[kSelMaxPairs], s_goff[kSelMaxPairs];
  __shared__ int s_ptok[kSelMaxPairs], s_pslot[kSelMaxPairs];
  __shared__ float s_w[kSelMaxPairs];
  const bool lead = (blockIdx.x | blockIdx.y | blockIdx.z) == 0;
  const int lane = threadIdx.x & 63;
  RouterArgs q = r;
  q.n_groups = &s_ng;
  q.grp_expert = s_gexp; q.grp_count = s_gcnt; q.grp_offset = s_goff;
  q.pair_token = s_ptok; q.pair_slot = s_pslot; q.slot_w = s_w;
  if (!lead) q.logits_out = nullptr, q.aff_full = nullptr, q.idx_out = nullptr, q.topk_out = nullptr;
  if (r.T == 1 && r.E <= 128 && 4 * r.E <= (int)blockDim.x)
    select_one(q, [&](int t, float (&l)[2]) { load_logits<2>(q, t, lane, l); });
  else
    select_small<PER>(q, [&](int t, float (&l)[PER]) { load_logits<PER>(q, t, lane, l); });
  __syncthreads();
  if (lead) {
    const int ng = s_ng, np = r.T * r.K;
    if (threadIdx.x == 0) *r.n_groups = ng;
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
      r.grp_expert[i] = s_gexp[i];
      r.grp_count[i] = s_gcnt[i];
      r.grp_offset[i] = s_goff[i];
    }
    for (int i = threadIdx.x; i < np; i += blockDim.x) {
      r.pair_token[i] = s_ptok[i];
      r.pair_slot[i] = s_pslot[i];
      if (r.slot_w) r.slot_w[i] = s_w[i];
    }
  }
  GemmArgs b = a;
  b.n_groups = &s_ng;
  b.grp_expert = s_gexp; b.grp_count = s_gcnt; b.grp_offset = s_goff;
  b.pair_row = s_ptok; b.pair_out_row = s_pslot;
  frag_body<2, 1, false, EPI_SWIGLU_BF16>(b, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Gate/up and down of the routed experts in ONE launch for a few tokens
// (moe_tkg.py selective experts; the router top-k as in gemm_frag_sel_kernel).
// Blocks [0, ngu) are the gate/up tiles of gemm_frag_sel_kernel (tile =
// bid % n_gu, group = bid / n_gu); they store their SwiGLU columns of h
// device-coherent and then set their flag word.  Blocks [ngu, ngu + gmax * ndb)
// take 64 output rows of one group's down projection: they form the routing
// themselves like every block, issue their whole weight slice (8 waves = 4 row
// blocks x 2 K halves, NFD fragments each) right away, then wait until all n_gu
// flags of their group are set, read that group's h rows device-coherent and
// finish -- the down weights stream while the gate/up blocks run, and the
// kernel boundary between the two projections is gone.  Workgroups are
// dispatched in index order and the gate/up blocks wait on nothing, so every
// awaited block is already resident; the waits are bounded regardless
// (coh_wait_all).  Occupancy: at most 4 waves per SIMD (128 VGPRs), so at one
// token the last down blocks are dispatched as gate/up blocks retire --
// measured at bs = 1 (Qwen3-30B-A3B shape): 25.5 us per launch against 27.5 us
// with all 640 blocks resident at 6 waves per SIMD (80 VGPRs); 2, 3, 4 and 5
// waves per SIMD are within 0.3 us of each other.
// DRB: row blocks per down wave (1: 64 output rows per down block, 2: 128), chosen
// so that the whole grid is resident at once where it can be.
template <int PER, int NFD, int DRB>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) moe_fused_kernel(MoeFusedArgs f) {
  __shared__ int s_ng;
  __shared__ int s_gexp[kSelMaxPairs], s_gcnt[kSelMaxPairs], s_goff[kSelMaxPairs];
  __shared__ int s_ptok[kSelMaxPairs], s_pslot[kSelMaxPairs];
  __shared__ float s_w[kSelMaxPairs];
  __shared__ OneTokenSel sel;
  __shared__ float s_rinv;
  __shared__ __attribute__((aligned(16))) uint16_t s_hn[kFusedHnMax];   // the experts' input (K-sliced router form)
  __shared__ f32x4_t s_red[DRB][4][64];
  __shared__ u32x4_t s_h[kFusedMaxRows][NFD * 8];   // h rows of a down block's group
  const int bid = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const RouterArgs& r = f.r;
  // One token whose selection key is the logit (Qwen, or top-k on logits then a
  // softmax over the top-k): the experts are ranked first and published to the
  // group tables, and only the down blocks form the routing weights, after
  // their weight loads are out (select_one_experts / select_one_weights) -- the
  // gate/up blocks issue their weight loads without waiting for the softmax.
  const bool one = r.T == 1 && r.E <= 128 && 4 * r.E <= (int)blockDim.x;
  const bool split = one && r.nparts <= 8 &&
                     ((r.mode & 8) || !(r.mode & 3));   // Qwen flow, or neither pre-norm nor sigmoid
  const bool lead = split ? bid == f.ngu : bid == 0;   // writes the routing outputs
  RouterArgs q = r;
  q.n_groups = &s_ng;
  q.grp_expert = s_gexp; q.grp_count = s_gcnt; q.grp_offset = s_goff;
  q.pair_token = s_ptok; q.pair_slot = s_pslot; q.slot_w = s_w;
  if (!lead) q.logits_out = nullptr, q.aff_full = nullptr, q.idx_out = nullptr, q.topk_out = nullptr;
  const bool gu_role = bid < f.ngu;
  // the block's routing tables (LDS)
  int *t_ng = &s_ng, *t_gexp = s_gexp, *t_gcnt = s_gcnt, *t_goff = s_goff, *t_ptok = s_ptok, *t_pslot = s_pslot;
  float* t_w = s_w;
  float lg[2];
  // K-sliced router form: the post-attention residual and gamma for the
  // experts' input, loaded before the routing (4 elements per thread)
  const bool hn_self = split && r.ss_parts && f.hn_r;
  const int H = f.gu.K;
  uint2 hr = {0u, 0u}, hg = {0u, 0u};
  if (hn_self && (int)threadIdx.x * 4 < H) {
    hr = *reinterpret_cast<const uint2*>(f.hn_r + threadIdx.x * 4);
    hg = *reinterpret_cast<const uint2*>(f.hn_gamma + threadIdx.x * 4);
  }
  // a down block's weight slice does not depend on the routing: its row block
  // and K half are fixed, only the expert offset is not -- so the routing comes
  // first, then the loads
  if (split) {
    // the joined attention launch's router stage leaves <= 8 partial logits
    // (and, K-sliced, <= 8 slice sums of squares: logits = rinv * sum)
    float raw[8][2], ssr[8];
    select_one_experts(q,
        [&]() {
#pragma unroll
          for (int p = 0; p < 8; ++p)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              raw[p][j] = q.parts[min(p, q.nparts - 1) * q.part_stride + min(lane + 64 * j, q.E - 1)];
          if (q.ss_parts)
#pragma unroll
            for (int p = 0; p < 8; ++p) ssr[p] = q.ss_parts[min(p, q.nss - 1)];
        },
        [&](float (&l)[2]) {
          float rinv = 1.f;
          if (q.ss_parts) {
            float t = 0.f;
#pragma unroll
            for (int p = 0; p < 8; ++p)
              if (p < q.nss) t += ssr[p];
            rinv = 1.0f / sqrtf(t * q.ss_inv_h + q.ss_eps);
            if (lane == 0) s_rinv = rinv;
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            float v = 0.f;
#pragma unroll
            for (int p = 0; p < 8; ++p)
              if (p < q.nparts) v += raw[p][j];
            if (q.ss_parts) v *= rinv;
            l[j] = q.bias ? v + bf2f(q.bias[min(lane + 64 * j, q.E - 1)]) : v;
          }
        },
        [] {}, sel, lg);
    if (hn_self && (int)threadIdx.x * 4 < H) {   // rinv in LDS since select_one_experts' barrier
      const float ri = s_rinv;
      *reinterpret_cast<uint2*>(s_hn + threadIdx.x * 4) =
          uint2{pack2bf((bf_lo(hr.x) * bf_lo(hg.x)) * ri, (bf_hi(hr.x) * bf_hi(hg.x)) * ri),
                pack2bf((bf_lo(hr.y) * bf_lo(hg.y)) * ri, (bf_hi(hr.y) * bf_hi(hg.y)) * ri)};
    }
    t_ng = &sel.ng; t_gexp = sel.gexp; t_gcnt = sel.gcnt; t_goff = sel.goff;
    t_ptok = sel.ptok; t_pslot = sel.pslot; t_w = sel.w;
  } else if (one) {
    if (r.nparts <= 8) select_one(q, [&](int t, float (&l)[2]) { load_logits<2, 8>(q, t, lane, l); });
    else select_one(q, [&](int t, float (&l)[2]) { load_logits<2>(q, t, lane, l); });
  } else {
    select_small<PER>(q, [&](int t, float (&l)[PER]) { load_logits<PER>(q, t, lane, l); });
  }
  __syncthreads();
  if (lead && !split) {
    const int ng = s_ng, np = r.T * r.K;
    if (threadIdx.x == 0) *r.n_groups = ng;
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
      r.grp_expert[i] = s_gexp[i];
      r.grp_count[i] = s_gcnt[i];
      r.grp_offset[i] = s_goff[i];
    }
    for (int i = threadIdx.x; i < np; i += blockDim.x) {
      r.pair_token[i] = s_ptok[i];
      r.pair_slot[i] = s_pslot[i];
      if (r.slot_w) r.slot_w[i] = s_w[i];
    }
  }
  if (gu_role) {
    GemmArgs b = f.gu;
    if (hn_self) b.x = s_hn;             // the operand from LDS (generic loads)
    b.n_groups = t_ng;
    b.grp_expert = t_gexp; b.grp_count = t_gcnt; b.grp_offset = t_goff;
    b.pair_row = t_ptok; b.pair_out_row = t_pslot;
    frag_body<2, 1, false, EPI_SWIGLU_BF16, true>(b, bid % f.n_gu, bid / f.n_gu, 0);
    if (!f.poll_h) coh_publish(f.flags + bid);
    return;
  }
  // ---- down role ----
  const GemmArgs& d = f.dn;
  const int db = bid - f.ngu;
  const int g = db / f.ndb, qd = db - g * f.ndb;
  if (g >= *t_ng) return;
  const int ex = t_gexp[g], count = t_gcnt[g], base = t_goff[g];
  const int KB = d.K / 32;
  const int rbk = qd * 4 * DRB + (wave & 3); // 16-row blocks rbk + 4 i of the output
  const int kh = wave >> 2;                  // K half
  const int kb0 = kh * NFD;
  u32x4_t wf[DRB][NFD];
#pragma unroll
  for (int i = 0; i < DRB; ++i) {
    const uint16_t* wrow =
        d.w + (long long)ex * d.w_group_stride + ((long long)(rbk + 4 * i) * KB + kb0) * 512 + lane * 8;
#pragma unroll
    for (int u = 0; u < NFD; ++u)
      wf[i][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + u * 512));
  }
  if (lead && hn_self && f.hn_out)
    for (int i = threadIdx.x * 8; i < H; i += blockDim.x * 8)
      *reinterpret_cast<u32x4_t*>(f.hn_out + i) = *reinterpret_cast<const u32x4_t*>(s_hn + i);
  if (split && wave == 0) {
    q.slot_w = lead ? r.slot_w : nullptr;
    select_one_weights(q, sel, lg);   // sel.w: read after the barriers below
    if (lead && threadIdx.x < r.K) {   // the group tables too (one group per slot)
      if (threadIdx.x == 0) *r.n_groups = r.K;
      r.grp_expert[threadIdx.x] = sel.gexp[threadIdx.x];
      r.grp_count[threadIdx.x] = 1;
      r.grp_offset[threadIdx.x] = threadIdx.x;
      r.pair_token[threadIdx.x] = 0;
      r.pair_slot[threadIdx.x] = threadIdx.x;
    }
  }
  const int c = lane & 15;
  const int prow = c < count ? t_pslot[base + c] : -1;   // h row and output row of the column
  if (!f.poll_h) {
    if (wave == 0) coh_wait_all(f.flags + g * f.n_gu, f.n_gu, f.err);
    __syncthreads();
  }
  // the group's h rows (count <= kFusedMaxRows, K = 64 NFD) into LDS with one
  // device-coherent 16-byte load per thread, then the B operands from LDS; with
  // the data-polled h, loaded until no 16-bit word reads the empty marker (the
  // gate/up epilogue never stores it), bounded like the flag waits: the block
  // gives up together once its own polls ran out or another wait already did
  {
    const __amdgpu_buffer_rsrc_t hr = coh_rsrc(d.x);
    const int per_row = d.K / 8;                       // 16-byte pieces per row
    for (unsigned it = 0;; ++it) {
      int miss = 0;
      for (int i = threadIdx.x; i < count * per_row; i += blockDim.x) {
        const int rr = i / per_row, pc = i - rr * per_row;
        const int row = t_pslot[base + rr];
        const u32x4_t v = coh_ld16(hr, (int)(((long long)row * d.ldx + pc * 8) * 2));
        s_h[rr][pc] = v;
#pragma unroll
        for (int e = 0; e < 4; ++e) miss |= poll_bf16x2_empty(v[e]);
      }
      if (!f.poll_h) break;
      if (!__syncthreads_or(miss)) break;
      if (__syncthreads_or(threadIdx.x == 0 && coh_poll_giveup(it, f.err))) break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  // B operands four at a time (the weights already hold DRB * NFD * 4 registers)
  f32x4_t acc[DRB];
#pragma unroll
  for (int i = 0; i < DRB; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u0 = 0; u0 < NFD; u0 += 4) {
    u32x4_t xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xv[j] = c < count ? s_h[c][(kb0 + u0 + j) * 4 + (lane >> 4)] : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < DRB; ++i) acc[i] = mfma16x16x32(wf[i][u0 + j], xv[j], acc[i]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < DRB; ++i) s_red[i][wave & 3][lane] = acc[i];
  }
  __syncthreads();
  if (kh != 0 || prow < 0) return;
  const float sc = t_w[prow];
#pragma unroll
  for (int i = 0; i < DRB; ++i) {
    const f32x4_t hi = s_red[i][wave][lane];
    const int n0 = (rbk + 4 * i) * 16 + (lane >> 4) * 4;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = acc[i][e] + hi[e];
      if (d.bias) v += bf2f(d.bias[(long long)ex * d.bias_group_stride + n0 + e]);
      o[e] = v * sc;
    }
    *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(d.y) + (long long)prow * d.ldy + n0) =
        f32x4_t{o[0], o[1], o[2], o[3]};
  }
}


// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <int RB, int TN, bool XF32, int EPI>
static hipError_t launch_t(const GemmArgs& a, int n_tiles, int groups, int ttiles, hipStream_t s) {
  const int kg = a.kgrid > 1 ? a.kgrid : 1;
  const int nsplit = a.K / (a.KW * kg);
  if (nsplit < 1 || nsplit > 16 || nsplit * a.KW * kg != a.K) return hipErrorInvalidValue;
  if (kg > 1 && EPI != EPI_F32) return hipErrorInvalidValue;
  dim3 grid(n_tiles, groups, ttiles * kg);
  dim3 block(64 * nsplit);
  const size_t lds = nsplit > 1 ? (size_t)nsplit * RB * TN * 4 * 64 * sizeof(float) : 0;
  return timed_launch(gemm_frag_kernel<RB, TN, XF32, EPI>, grid, block, lds, s, a);
}

bool gemm_sel_supported(int T, int K, int E, int nsplit) {
  return T >= 1 && T <= nsplit && T * K <= kSelMaxPairs && K >= 1 && K <= 8 && K <= E && E <= 256;
}

hipError_t gemm_sel_launch(const GemmArgs& a, const RouterArgs& r, int groups_max, hipStream_t s) {
  const int nsplit = a.KW > 0 ? a.K / a.KW : 0;
  if (nsplit < 1 || nsplit > 16 || nsplit * a.KW != a.K || (a.kgrid > 1) ||
      !gemm_sel_supported(r.T, r.K, r.E, nsplit) || a.T != r.T || !r.parts || r.nparts < 1 ||
      r.nparts > 16 || !r.n_groups || !r.grp_expert || !r.grp_count || !r.grp_offset ||
      !r.pair_token || !r.pair_slot || !a.grp_expert || groups_max < 1 || groups_max > kSelMaxPairs)
    return hipErrorInvalidValue;
  const dim3 grid((a.N + 31) / 32, groups_max, (a.T + 15) / 16), block(64 * nsplit);
  const size_t lds = nsplit > 1 ? (size_t)nsplit * 2 * 4 * 64 * sizeof(float) : 0;
  const int per = (r.E + 63) / 64;
  if (per <= 1) return timed_launch(gemm_frag_sel_kernel<1>, grid, block, lds, s, a, r);
  if (per <= 2) return timed_launch(gemm_frag_sel_kernel<2>, grid, block, lds, s, a, r);
  return timed_launch(gemm_frag_sel_kernel<4>, grid, block, lds, s, a, r);
}

bool moe_fused_supported(int T, int K, int E, int H, int I) {
  const int KB = I / 32;
  return T >= 1 && T <= kFusedMaxRows && T * K <= kSelMaxPairs && K >= 1 && K <= 8 && K <= E && E <= 256 &&
         H % 256 == 0 && H % 64 == 0 && I % 64 == 0 && (KB / 2 == 12 || KB / 2 == 8) &&
         (2 * I) % 32 == 0 && (2 * I) / 32 <= 256;
}

int moe_fused_flag_words(int T, int K, int E, int I) {
  const int gmax = E < T * K ? E : T * K;
  return gmax * ((2 * I) / 32);
}

int device_cus() {
  static int cus = -1;
  if (cus < 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    cus = n;
  }
  return cus;
}

hipError_t moe_fused_launch(MoeFusedArgs f, int groups_max, hipStream_t s) {
  const RouterArgs& r = f.r;
  const GemmArgs& a = f.gu;
  if (!moe_fused_supported(r.T, r.K, r.E, a.K, f.dn.K) || a.T != r.T || f.dn.N != a.K ||
      a.N != 2 * f.dn.K || a.KW * 8 != a.K || a.kgrid > 1 || !r.parts || r.nparts < 1 ||
      r.nparts > 16 || !r.n_groups || !r.grp_expert || !r.grp_count || !r.grp_offset ||
      !r.pair_token || !r.pair_slot || !a.grp_expert || !f.flags || !f.err || groups_max < 1 ||
      groups_max > kSelMaxPairs || (f.dn.ldx & 7) || (f.dn.ldy & 3))
    return hipErrorInvalidValue;
  if (r.ss_parts) {   // the K-sliced router form: the kernel's split routing must apply
    const bool split = r.T == 1 && r.E <= 128 && r.nparts <= 8 && ((r.mode & 8) || !(r.mode & 3));
    if (!split || r.nss < 1 || r.nss > 8 || !f.hn_r || !f.hn_gamma || a.K > kFusedHnMax || a.K % 8 ||
        a.K > 4 * 512)
      return hipErrorInvalidValue;
  }
  if (f.poll_h) {   // h goes to the launch's own pre-filled buffer
    f.gu.y = f.poll_h;
    f.dn.x = f.poll_h;
  }
  f.n_gu = a.N / 32;
  f.ngu = f.n_gu * groups_max;
  // 128 output rows per down block where that makes the whole grid resident at
  // two blocks per CU (at one token: 384 gate/up + 128 down blocks); the last
  // down blocks are otherwise dispatched only as gate/up blocks retire, and
  // then stream their weights and form the routing after the gate/up work
  const int drb = (f.dn.N % 128 == 0 && f.ngu + (f.dn.N / 128) * groups_max <= 2 * device_cus()) ? 2 : 1;
  f.ndb = f.dn.N / (64 * drb);
  const dim3 grid(f.ngu + f.ndb * groups_max), block(512);
  const size_t lds = (size_t)8 * 2 * 4 * 64 * sizeof(float);
  const int per = (r.E + 63) / 64;
  const int nfd = (f.dn.K / 32) / 2;
#define MKD_FUSED(P, N)                                                                      \
  if (per <= P && nfd == N)                                                                  \
    return drb == 2 ? timed_launch(moe_fused_kernel<P, N, 2>, grid, block, lds, s, f)       \
                    : timed_launch(moe_fused_kernel<P, N, 1>, grid, block, lds, s, f)
  MKD_FUSED(1, 8); MKD_FUSED(1, 12);
  MKD_FUSED(2, 8); MKD_FUSED(2, 12);
  MKD_FUSED(4, 8); MKD_FUSED(4, 12);
#undef MKD_FUSED
  return hipErrorInvalidValue;
}


int choose_kw(int K, int max_kw, long long blocks) {
  // Per-wave K slice (a multiple of 32 dividing K into <= 16 waves, <= max_kw).
  // The longest slice is cheapest per fragment (fewer partial sums to reduce),
  // but a launch of few blocks needs more waves per block to keep enough loads
  // in flight: take the longest slice that gives >= kMinWaves waves in total,
  // else the most waves whose slices still hold >= 64 elements.  Measured at
  // decode shapes: o_proj 2048x4096 (128 blocks) 7.2 us at 16 waves vs 8.1 us
  // at 8; lm_head 151936x2048 (9496 blocks) 94 us at 4 waves vs 99 us at 8.
  constexpr long long kMinWaves = 2048;
  int best = -1, most = -1;
  for (int kw = (max_kw < K ? max_kw : K) / 32 * 32; kw >= 32; kw -= 32) {
    if (K % kw || K / kw > 16) continue;
    if (blocks * (K / kw) >= kMinWaves) return kw;
    if (best < 0) best = kw;
    if (kw >= 64 || most < 0) most = kw;
  }
  return most > 0 ? most : best;
}

int choose_kw_split(int K, int kgrid) {
  // per-wave slice for a K split over kgrid blocks of <= 4 waves each
  if (K % kgrid) return -1;
  const int kb = K / kgrid;
  for (int kw : {512, 256, 128, 64, 32}) {
    if (kb % kw == 0 && kb / kw <= 4) return kw;
  }
  return -1;
}

hipError_t gemm_launch(GemmArgs a, int epi, bool xf32, int tn, int groups_max,
                       int max_tokens_per_group, hipStream_t s) {
  const int RB = (epi == EPI_SWIGLU_BF16) ? 2 : 1;
  const int n_tiles = (a.N + 16 * RB - 1) / (16 * RB);
  int ttiles = (max_tokens_per_group + 16 * tn - 1) / (16 * tn);
  const int groups = a.grp_expert ? groups_max : 1;
  if (a.grp_expert && ttiles > 1 && (a.kgrid <= 1)) {   // grouped: one tile per block, walking the group
    a.t_loop = 1;
    ttiles = 1;
  }
#define MKD_G(RB_, TN_, XF_, EPI_) \
  if (RB == RB_ && tn == TN_ && xf32 == XF_ && epi == EPI_) return launch_t<RB_, TN_, XF_, EPI_>(a, n_tiles, groups, ttiles, s);
  MKD_G(1, 1, false, EPI_F32) MKD_G(1, 2, false, EPI_F32) MKD_G(1, 4, false, EPI_F32)
  MKD_G(1, 1, true, EPI_F32) MKD_G(1, 2, true, EPI_F32) MKD_G(1, 4, true, EPI_F32)
  MKD_G(1, 1, false, EPI_BF16) MKD_G(1, 2, false, EPI_BF16) MKD_G(1, 4, false, EPI_BF16)
  MKD_G(1, 1, false, EPI_RESID_BF16) MKD_G(1, 2, false, EPI_RESID_BF16) MKD_G(1, 4, false, EPI_RESID_BF16)
  MKD_G(2, 1, false, EPI_SWIGLU_BF16) MKD_G(2, 2, false, EPI_SWIGLU_BF16)
  MKD_G(1, 1, false, EPI_SCALE_F32) MKD_G(1, 2, false, EPI_SCALE_F32) MKD_G(1, 4, false, EPI_SCALE_F32)
#undef MKD_G
  return hipErrorInvalidValue;
}

hipError_t pack_frag_launch(const uint16_t* src, uint16_t* dst, int G, int N, int K,
                            long long g_stride, long long row_stride, long long col_stride,
                            int interleave_half, hipStream_t s) {
  const long long total = (long long)G * ((N + 15) / 16) * (K / 32) * 64;
  if (total <= 0) return hipErrorInvalidValue;
  const int threads = 256;
  long long blocks = (total + threads - 1) / threads;
  if (blocks > 65535LL * 16) blocks = 65535LL * 16;
  hipLaunchKernelGGL(pack_frag_kernel, dim3((unsigned)blocks), dim3(threads), 0, s, src, dst, G,
                     N, K, g_stride, row_stride, col_stride, interleave_half);
  return hipGetLastError();
}

}  // namespace mkd
