// The weight-streaming frag GEMM body (gemm.hip's kernels and the joined
// expert launches): stream_batch issues a batch of weight fragments and their
// x operands, frag_body walks one block's K slice and applies the epilogue.
#pragma once
#include "common.h"
#include "gemm_epi.h"
#include "mkd_internal.h"

namespace mkd {

// B consecutive fragments of every row block: every weight and x load of the
// batch is issued before the first MFMA.  Lanes of absent tokens (xrow < 0)
// read x row 0 instead -- their output column is never written, and MFMA
// columns are independent.  fp32 x rows are
// carried as a bf16 hi + lo pair (two MFMAs).
template <int RB, int TN, bool XF32, int B>
MKD_DEV void stream_batch(const uint16_t* const (&wrow)[RB], int f, int kb0, int koff,
                          const int (&xrow)[TN], const GemmArgs& a, f32x4_t (&acc)[RB][TN]) {
  u32x4_t wf[RB][B];
#pragma unroll
  for (int u = 0; u < B; ++u)
#pragma unroll
    for (int r = 0; r < RB; ++r)
      wf[r][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow[r] + (f + u) * 512));
  // the weight loads go out before the x addresses are formed: in grouped mode
  // the token rows come from a routing table whose load may still be in flight
  __builtin_amdgcn_sched_barrier(0);
  const void* xp[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    int xr = xrow[tn];
    asm volatile("" : "+v"(xr));         // formed here, not hoisted out of the k loop
    const long long off = (long long)(xr >= 0 ? xr : 0) * a.ldx + koff;
    xp[tn] = XF32 ? static_cast<const void*>(static_cast<const float*>(a.x) + off)
                  : static_cast<const void*>(static_cast<const uint16_t*>(a.x) + off);
  }
  if constexpr (XF32) {
    f32x4_t xa[B][TN], xb[B][TN];
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const float* p = static_cast<const float*>(xp[tn]) + (kb0 + f + u) * 32;
        xa[u][tn] = *reinterpret_cast<const f32x4_t*>(p);
        xb[u][tn] = *reinterpret_cast<const f32x4_t*>(p + 4);
      }
    if constexpr (TN == 1) __builtin_amdgcn_sched_barrier(0);   // every load ahead of the MFMAs
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const float xs[8] = {xa[u][tn][0], xa[u][tn][1], xa[u][tn][2], xa[u][tn][3],
                             xb[u][tn][0], xb[u][tn][1], xb[u][tn][2], xb[u][tn][3]};
        u32x4_t hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t h0 = f2bf(xs[2 * j]), h1 = f2bf(xs[2 * j + 1]);
          hi[j] = h0 | (h1 << 16);
          lo[j] = f2bf(xs[2 * j] - bf2f(h0)) | (f2bf(xs[2 * j + 1] - bf2f(h1)) << 16);
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          acc[r][tn] = mfma16x16x32(wf[r][u], hi, acc[r][tn]);
          acc[r][tn] = mfma16x16x32(wf[r][u], lo, acc[r][tn]);
        }
      }
  } else {
    u32x4_t xv[B][TN];
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        xv[u][tn] = ld16(static_cast<const uint16_t*>(xp[tn]) + (kb0 + f + u) * 32);
    // one token tile: every load ahead of the MFMAs (a latency-bound launch);
    // more tiles: MFMA work to hide, so the compiler interleaves (measured
    // 46 -> 23 us for the QKV / o_proj GEMMs at 64 tokens)
    if constexpr (TN == 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r][tn] = mfma16x16x32(wf[r][u], xv[u][tn], acc[r][tn]);
  }
}

// ---------------------------------------------------------------------------
// The GEMM.
// ---------------------------------------------------------------------------
// (rbase, group, bz): the block's RB-row-block tile, routed group, and token
// tile * kgrid + K block -- blockIdx in the plain launch.  COH: the outputs are
// stored device-coherent (read by other blocks of the same launch).
template <int RB, int TN, bool XF32, int EPI, bool COH = false, int UNR = 8 / RB>
MKD_DEV void frag_body(const GemmArgs& a, int rbase, int group, int bz) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kg = a.kgrid > 1 ? a.kgrid : 1;
  const int kblk = bz % kg;

  // ---- token columns of this block ----
  int count, base;                       // tokens in this group / first pair
  const uint16_t* w = a.w;
  if (a.grp_expert) {
    // the group's table entries are read together with the group count (one
    // memory round trip; group < gridDim.y <= the tables' length)
    const int ng = *a.n_groups;
    count = a.grp_count[group];
    base = a.grp_offset[group];
    const int ex = a.grp_expert[group];
    asm volatile("" ::"s"(ng), "s"(count), "s"(base), "s"(ex));   // no sinking past the exit
    if (group >= ng) return;
    w += (long long)ex * a.w_group_stride;
  } else {
    count = a.T;
    base = 0;
  }
  for (int ttile = bz / kg;; ++ttile) {
  const int t0 = ttile * 16 * TN;
  if (t0 >= count) return;
  if (ttile > bz / kg) __syncthreads();   // the previous tile's reduction buffer is free

  // x row of each token column owned by this lane (one column per TN tile)
  int xrow[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int c = t0 + tn * 16 + (lane & 15);
    if (c < count)
      xrow[tn] = a.pair_row ? a.pair_row[base + c] : (base + c);
    else
      xrow[tn] = -1;
  }

  const int KB = a.K / 32;
  const int NF = a.KW / 32;              // fragments per wave
  const int kb0 = (kblk * (int)(blockDim.x >> 6) + wave) * NF;
  const int koff = (lane >> 4) * 8;

  f32x4_t acc[RB][TN];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[r][tn] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint16_t* wrow[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r)
    wrow[r] = w + ((long long)(rbase * RB + r) * KB + kb0) * 512 + lane * 8;

  // Stream the fragments: a wave issues a batch of UNROLL*RB fragment loads
  // (8 KiB) before the MFMAs that consume them; batches carry no guards so
  // they stay in registers, and the remainder (< UNROLL) is taken as batches of
  // 4/2/1 so short slices still keep several loads in flight.  (Measured at
  // decode shapes: 8 fragments per batch with up to 16 waves per block beat
  // 16- and 32-fragment batches with fewer waves.)
  constexpr int UNROLL = UNR;
  int f = 0;
  for (; f + UNROLL <= NF; f += UNROLL)
    stream_batch<RB, TN, XF32, UNROLL>(wrow, f, kb0, koff, xrow, a, acc);
  if constexpr (UNROLL > 8)
    if (f + 8 <= NF) { stream_batch<RB, TN, XF32, 8>(wrow, f, kb0, koff, xrow, a, acc); f += 8; }
  if constexpr (UNROLL > 4)
    if (f + 4 <= NF) { stream_batch<RB, TN, XF32, 4>(wrow, f, kb0, koff, xrow, a, acc); f += 4; }
  if constexpr (UNROLL > 2)
    if (f + 2 <= NF) { stream_batch<RB, TN, XF32, 2>(wrow, f, kb0, koff, xrow, a, acc); f += 2; }
  if constexpr (UNROLL > 1)
    if (f < NF) stream_batch<RB, TN, XF32, 1>(wrow, f, kb0, koff, xrow, a, acc);

  gemm_finish<RB, TN, EPI, COH>(a, acc, lane, wave, rbase, group, t0, base, xrow, kblk);
  if (!a.t_loop) return;
  }
}

}  // namespace mkd
