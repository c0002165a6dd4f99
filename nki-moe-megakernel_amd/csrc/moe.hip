// Router top-k, token->expert grouping and the MoE epilogue.
//
// router_select: one block over fp32 logits [T, E] (E <= 512, K <= 8, T <= 128),
//   rank-based top-k (value desc, index asc: the lowest index wins an exact
//   tie), optionally followed by the expert grouping.  Modes (bit field):
//     bit0 act      0 softmax, 1 sigmoid
//     bit1 pre_norm activation on all E before top-k (ACT1) else on the top-k (ACT2)
//     bit2 norm     L1-renormalise the top-k (ACT1 path)
//     bit3 qwen     Qwen fused flow: top-k on logits, softmax value at the top-k
//                   rounded to bf16, then bf16 L1 renormalisation
//   Outputs: expert index [T,K] (int32), top-k affinities [T,K] fp32, per-slot
//   weights [T*K] (same values), and optionally the scattered / full
//   affinities [T,E].
// moe_route: single block of 1024 threads; counting sort of the T*K (token, k)
//   slots by expert into compact groups (live experts in ascending id order;
//   the slots within a group in any order -- every consumer indexes by slot).
// moe_finalize: out[t] = bf16(sum_k y[t*K + k]) (fp32 sum in k order), then the
//   bf16 residual add.
#include "common.h"
#include "mkd_internal.h"
#include "router_select.h"
#include "launch_rules.h"

namespace mkd {

template <int PER>
__global__ void __launch_bounds__(1024) router_select_kernel(RouterArgs a) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  // the first token's logits are loaded before anything else (their latency
  // covers the LDS set-up; the first block barrier comes after the per-token
  // phase, which only touches the wave's own LDS rows)
  float lfirst[PER];
  if (wv < a.T) load_logits<PER>(a, wv, lane, lfirst);
  select_body<PER>(a, [&](int t, float (&l)[PER]) {
    if (t == wv) {
#pragma unroll
      for (int j = 0; j < PER; ++j) l[j] = lfirst[j];
    } else {
      load_logits<PER>(a, t, lane, l);
    }
  });
}

// Many tokens without grouping (a long prefill pass): block b selects tokens
// 16b .. 16b + 15, one per wave, with the arithmetic of router_select_kernel.
template <int PER>
__global__ void __launch_bounds__(1024) router_select_multi_kernel(RouterArgs a) {
  const int t0 = blockIdx.x * 16;
  RouterArgs q = a;
  q.T = min(16, a.T - t0);
  q.parts = a.parts + (long long)t0 * a.E;
  if (a.logits_out) q.logits_out = a.logits_out + (long long)t0 * a.E;
  if (a.aff_full) q.aff_full = a.aff_full + (long long)t0 * a.E;
  if (a.idx_out) q.idx_out = a.idx_out + t0 * a.K;
  if (a.topk_out) q.topk_out = a.topk_out + t0 * a.K;
  if (a.slot_w) q.slot_w = a.slot_w + t0 * a.K;
  const int lane = threadIdx.x & 63;
  select_body<PER>(q, [&](int t, float (&l)[PER]) { load_logits<PER>(q, t, lane, l); });
}

hipError_t router_select_multi_launch(const RouterArgs& a, hipStream_t s) {
  if (a.E > kMaxE || a.K > 8 || a.K < 1 || a.K > a.E || a.T < 1 || a.nparts > 16 || a.n_groups)
    return hipErrorInvalidValue;
  const dim3 grid((a.T + 15) / 16);
  const int per = (a.E + 63) / 64;
  if (per <= 1) hipLaunchKernelGGL(router_select_multi_kernel<1>, grid, dim3(1024), 0, s, a);
  else if (per <= 2) hipLaunchKernelGGL(router_select_multi_kernel<2>, grid, dim3(1024), 0, s, a);
  else if (per <= 4) hipLaunchKernelGGL(router_select_multi_kernel<4>, grid, dim3(1024), 0, s, a);
  else hipLaunchKernelGGL(router_select_multi_kernel<8>, grid, dim3(1024), 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
moe_route_kernel(const int* __restrict__ idx, int T, int K, int E, int* __restrict__ n_groups,
                 int* __restrict__ grp_expert, int* __restrict__ grp_count,
                 int* __restrict__ grp_offset, int* __restrict__ pair_token,
                 int* __restrict__ pair_slot, int cs, int nc, int* __restrict__ chunk_off) {
  __shared__ int cnt[kMaxE], off[kMaxE], cursor[kMaxE];
  __shared__ int wtot[16];
  // split form (chunk_off set): per-chunk counts [nc][E] of the cs-slot chunks
  __shared__ int cntc[kRouteChunkCounts];
  const bool split = chunk_off != nullptr;
  // Each pass takes CH slots per thread whose expert indices are all loaded
  // before any is used (one memory round trip per pass, not per slot).
  constexpr int CH = 16;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nt = (int)blockDim.x;
  const int TK = T * K;
  for (int e = tid; e < E; e += nt) { cnt[e] = 0; cursor[e] = 0; }
  if (split)
    for (int i = tid; i < nc * E; i += nt) cntc[i] = 0;
  __syncthreads();
  for (int p0 = 0; p0 < TK; p0 += CH * nt) {
    int ev[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int p = p0 + u * nt + tid;
      ev[u] = p < TK ? idx[p] : -1;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      if (ev[u] < 0 || ev[u] >= E) continue;
      if (split) atomicAdd(&cntc[((p0 + u * nt + tid) / cs) * E + ev[u]], 1);
      else atomicAdd(&cnt[ev[u]], 1);
    }
  }
  __syncthreads();
  if (split) {   // the experts' totals, chunk by chunk in order
    for (int e = tid; e < E; e += nt) {
      int t = 0;
      for (int c = 0; c < nc; ++c) t += cntc[c * E + e];
      cnt[e] = t;
    }
    __syncthreads();
  }
  // exclusive scans over the experts (E <= 512, the first 8 waves) of the pair
  // counts and the live-group ids, packed as count | live << 20 (counts < 2^20):
  // a wave scan, then the totals of the waves before
  const int c = tid < E ? cnt[tid] : 0;
  const int live = c > 0 ? 1 : 0;
  int x = c | (live << 20);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wtot[w] = x;
  __syncthreads();
  int before = 0, total = 0;
  for (int q = 0; q < nt / 64; ++q) {
    const int v = wtot[q];
    if (q < w) before += v;
    total += v;
  }
  const int incl = before + x;
  if (tid < E) {
    const int excl_cnt = (incl & 0xfffff) - c;
    const int excl_live = (incl >> 20) - live;
    off[tid] = excl_cnt;
    if (live) {
      grp_expert[excl_live] = tid;
      grp_count[excl_live] = c;
      grp_offset[excl_live] = excl_cnt;
    }
  }
  if (tid == 0) *n_groups = total >> 20;
  if (split) {   // chunk c's slots of expert e start at its group offset plus the earlier chunks' counts
    if (tid < E) {
      int run = (incl & 0xfffff) - c;
      for (int q = 0; q < nc; ++q) {
        chunk_off[q * E + tid] = run;
        run += cntc[q * E + tid];
      }
    }
    return;      // moe_route_scatter_kernel places the slots
  }
  __syncthreads();
  for (int p0 = 0; p0 < TK; p0 += CH * nt) {
    int ev[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int p = p0 + u * nt + tid;
      ev[u] = p < TK ? idx[p] : -1;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int e = ev[u];
      if (e < 0 || e >= E) continue;
      const int p = p0 + u * nt + tid;
      const int q = off[e] + atomicAdd(&cursor[e], 1);
      pair_token[q] = p / K;
      pair_slot[q] = p;
    }
  }
}

// Split routing, second half: block c places the slots of chunk c (cs slots
// from c * cs) at chunk_off[c][e] onwards, ranked by LDS atomics.
__global__ void __launch_bounds__(256)
moe_route_scatter_kernel(const int* __restrict__ idx, int TK, int K, int E, int cs,
                         const int* __restrict__ chunk_off, int* __restrict__ pair_token,
                         int* __restrict__ pair_slot) {
  __shared__ int base_s[kMaxE], cursor[kMaxE];
  constexpr int CH = 8;
  const int tid = threadIdx.x, nt = (int)blockDim.x;
  const int c = blockIdx.x, p_lo = c * cs, p_hi = min(TK, p_lo + cs);
  for (int e = tid; e < E; e += nt) {
    base_s[e] = chunk_off[c * E + e];
    cursor[e] = 0;
  }
  __syncthreads();
  for (int p0 = p_lo; p0 < p_hi; p0 += CH * nt) {
    int ev[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int p = p0 + u * nt + tid;
      ev[u] = p < p_hi ? idx[p] : -1;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int e = ev[u];
      if (e < 0 || e >= E) continue;
      const int p = p0 + u * nt + tid;
      const int q = base_s[e] + atomicAdd(&cursor[e], 1);
      pair_token[q] = p / K;
      pair_slot[q] = p;
    }
  }
}

// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
moe_finalize_kernel(const float* __restrict__ ybuf, int K, int H, const uint16_t* __restrict__ resid,
                    uint16_t* __restrict__ out, float* __restrict__ out_f32) {
  const int t = blockIdx.y;
  const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= H) return;
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < K; ++k) {
    const f32x4_t y = *reinterpret_cast<const f32x4_t*>(ybuf + ((long long)t * K + k) * H + i);
    s += y;
  }
  if (out_f32) *reinterpret_cast<f32x4_t*>(out_f32 + (long long)t * H + i) = s;
  if (out) {
    float o[4];
    for (int j = 0; j < 4; ++j) o[j] = rbf(s[j]);
    if (resid) {
      const uint2 r = *reinterpret_cast<const uint2*>(resid + (long long)t * H + i);
      o[0] += bf_lo(r.x); o[1] += bf_hi(r.x); o[2] += bf_lo(r.y); o[3] += bf_hi(r.y);
    }
    *reinterpret_cast<uint2*>(out + (long long)t * H + i) = uint2{pack2bf(o[0], o[1]), pack2bf(o[2], o[3])};
  }
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Router logits with the residual add and post-attention RMSNorm folded in, for
// T <= 4 tokens.  Grid (E/16 row blocks, KG contraction slices), one wave per
// block; the block writes the split-K partial logits that router_select sums:
//   r = bf16(x + bf16(o))            residual stream (slice written by row block 0)
//   y = (r * gamma) * rsqrt(mean_actual(r^2) + eps)   (bf16 copy of the slice written)
//   part[kg][t][e] = sum over the slice of y * W_router   (fp32 y as bf16 hi + lo)
// Every block reads the T full rows to form the sum of squares itself (a few KB
// from L2), which removes the separate norm launch (moe_fused_nki.py:70-153,
// router_topk.py:337-410).
constexpr int kFusedMaxT = 4;

// Contraction slices: enough blocks (>= ~128) with whole fragments per slice.
static int fused_kg(int E, int H) {
  const int KB = H / 32;
  int kg = 1;
  while (kg < 16 && (E / 16) * kg < 128 && KB % (kg * 2) == 0) kg *= 2;
  return kg;
}

bool router_fused_supported(int T, int E, int H) {
  return T >= 1 && T <= kFusedMaxT && E % 16 == 0 && E <= kMaxE && H % 32 == 0 && H > 0 &&
         (H / 32) % fused_kg(E, H) == 0 && (H / 32) / fused_kg(E, H) <= 8;
}

__global__ void __launch_bounds__(64) router_norm_gemm_kernel(RouterFusedArgs a, int kg) {
  const int lane = threadIdx.x;
  const int rb = blockIdx.x, kblk = blockIdx.y;
  const int T = a.r.T, E = a.r.E, H = a.H, KB = H / 32;
  const int nf = KB / kg;                // fragments of this slice
  const int kb0 = kblk * nf;
  const int tcol = lane & 15, koff = (lane >> 4) * 8;
  const bool live = tcol < T;
  constexpr int MAXF = 8;                // fragments per slice (router_fused_supported)

  // ---- loads, all independent: a 1/64 share of every row for the sum of
  // squares and the lane's operand values and gamma first, the weight
  // fragments last -- a wave's loads complete in issue order, so the norm runs
  // while the weights are in flight.  Addresses are clamped in range so every
  // load is unconditional; the values are masked where they are used. ----
  constexpr int MAXC = 4;                // row shares preloaded per token (H <= 2048)
  u32x4_t sx[kFusedMaxT][MAXC];
  f32x4_t sp[kFusedMaxT][MAXC], sq[kFusedMaxT][MAXC];
#pragma unroll
  for (int t = 0; t < kFusedMaxT; ++t)
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const long long row = (long long)min(t, T - 1) * H;
      const int cc = min(lane * 8 + c * 512, H - 8);
      sx[t][c] = ld16(a.x + row + cc);
      sp[t][c] = *reinterpret_cast<const f32x4_t*>(a.o + row + cc);
      sq[t][c] = *reinterpret_cast<const f32x4_t*>(a.o + row + cc + 4);
    }
  u32x4_t xb[MAXF], gb[MAXF];
  f32x4_t o0[MAXF], o1[MAXF];
  const int tr = live ? tcol : 0;
#pragma unroll
  for (int u = 0; u < MAXF; ++u) {
    const int k = (kb0 + min(u, nf - 1)) * 32 + koff;
    xb[u] = ld16(a.x + (long long)tr * H + k);
    gb[u] = ld16(a.gamma + k);
    o0[u] = *reinterpret_cast<const f32x4_t*>(a.o + (long long)tr * H + k);
    o1[u] = *reinterpret_cast<const f32x4_t*>(a.o + (long long)tr * H + k + 4);
  }
  u32x4_t wf[MAXF];
  const uint16_t* wrow = a.w + ((long long)rb * KB + kb0) * 512 + lane * 8;
#pragma unroll
  for (int u = 0; u < MAXF; ++u) wf[u] = ld16(wrow + min(u, nf - 1) * 512);
  // sum of squares of r over the whole row, lane share: H / 64 elements
  float ss[kFusedMaxT];
#pragma unroll
  for (int t = 0; t < kFusedMaxT; ++t) {
    ss[t] = 0.f;
    if (t >= T) continue;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      if (lane * 8 + c * 512 >= H) continue;
      const float ov[8] = {sp[t][c][0], sp[t][c][1], sp[t][c][2], sp[t][c][3],
                           sq[t][c][0], sq[t][c][1], sq[t][c][2], sq[t][c][3]};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xv_j = (j & 1) ? bf_hi(sx[t][c][j >> 1]) : bf_lo(sx[t][c][j >> 1]);
        const float r = rbf(xv_j + rbf(ov[j]));
        ss[t] += r * r;
      }
    }
    for (int c = lane * 8 + MAXC * 512; c < H; c += 512) {   // rows longer than MAXC shares
      const u32x4_t xv = ld16(a.x + (long long)t * H + c);
      const f32x4_t p = *reinterpret_cast<const f32x4_t*>(a.o + (long long)t * H + c);
      const f32x4_t q = *reinterpret_cast<const f32x4_t*>(a.o + (long long)t * H + c + 4);
      const float ov[8] = {p[0], p[1], p[2], p[3], q[0], q[1], q[2], q[3]};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float xv_j = (j & 1) ? bf_hi(xv[j >> 1]) : bf_lo(xv[j >> 1]);
        const float r = rbf(xv_j + rbf(ov[j]));
        ss[t] += r * r;
      }
    }
  }
  float rinv_t[kFusedMaxT];
#pragma unroll
  for (int t = 0; t < kFusedMaxT; ++t) rinv_t[t] = 1.0f / sqrtf(wave_sum(ss[t]) * a.inv_h + a.eps);
  float rinv = rinv_t[0];
#pragma unroll
  for (int t = 1; t < kFusedMaxT; ++t)
    if (tcol == t) rinv = rinv_t[t];

  // ---- operands: y for the lane's token and k range, MFMAs ----
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < MAXF; ++u) {
    if (u < nf) {
    const int k = (kb0 + u) * 32 + koff;
    const float ov[8] = {o0[u][0], o0[u][1], o0[u][2], o0[u][3], o1[u][0], o1[u][1], o1[u][2], o1[u][3]};
    float r[8], y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float xv_j = (j & 1) ? bf_hi(xb[u][j >> 1]) : bf_lo(xb[u][j >> 1]);
      const float g = (j & 1) ? bf_hi(gb[u][j >> 1]) : bf_lo(gb[u][j >> 1]);
      r[j] = rbf(xv_j + rbf(ov[j]));
      y[j] = live ? (r[j] * g) * rinv : 0.f;
    }
    if (rb == 0 && live) {   // the slice's residual and bf16 normalised rows
      u32x4_t ro, yo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ro[j] = pack2bf(r[2 * j], r[2 * j + 1]);
        yo[j] = pack2bf(y[2 * j], y[2 * j + 1]);
      }
      st16(a.resid_out + (long long)tcol * H + k, ro);
      st16(a.hnorm + (long long)tcol * H + k, yo);
    }
    u32x4_t hi, lo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float y0 = a.x_f32 ? y[2 * j] : rbf(y[2 * j]);
      const float y1 = a.x_f32 ? y[2 * j + 1] : rbf(y[2 * j + 1]);
      const uint32_t h0 = f2bf(y0), h1 = f2bf(y1);
      hi[j] = h0 | (h1 << 16);
      lo[j] = f2bf(y0 - bf2f(h0)) | (f2bf(y1 - bf2f(h1)) << 16);
    }
    acc = mfma16x16x32(wf[u], hi, acc);
    if (a.x_f32) acc = mfma16x16x32(wf[u], lo, acc);
    }
  }
  // D lane l: experts rb*16 + 4*(l/16) + i, token l%16 -> part[kblk][t][e]
  if (live) {
    float* pp = const_cast<float*>(a.r.parts) + kblk * a.r.part_stride + (long long)tcol * E + rb * 16 + (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) pp[i] = acc[i];
  }
}

hipError_t router_fused_launch(RouterFusedArgs a, hipStream_t s, RouterArgs* deferred) {
  if (!router_fused_supported(a.r.T, a.r.E, a.H) || !a.r.parts) return hipErrorInvalidValue;
  const int kg = fused_kg(a.r.E, a.H);
  a.r.nparts = kg;
  a.r.part_stride = (long long)a.r.T * a.r.E;
  if (hipError_t e = timed_launch(router_norm_gemm_kernel, dim3(a.r.E / 16, kg), dim3(64), 0, s, a, kg))
    return e;
  if (deferred) {
    *deferred = a.r;
    return hipSuccess;
  }
  return router_select_launch(a.r, s);
}

hipError_t router_select_launch(const RouterArgs& a, hipStream_t s) {
  if (a.E > kMaxE || a.K > 8 || a.K < 1 || a.K > a.E || a.T > 128 || a.T < 1 || a.nparts > 16)
    return hipErrorInvalidValue;
  const int per = (a.E + 63) / 64;
  if (per <= 1) hipLaunchKernelGGL(router_select_kernel<1>, dim3(1), dim3(1024), 0, s, a);
  else if (per <= 2) hipLaunchKernelGGL(router_select_kernel<2>, dim3(1), dim3(1024), 0, s, a);
  else if (per <= 4) hipLaunchKernelGGL(router_select_kernel<4>, dim3(1), dim3(1024), 0, s, a);
  else hipLaunchKernelGGL(router_select_kernel<8>, dim3(1), dim3(1024), 0, s, a);
  return hipGetLastError();
}

// Chunking of the split form: chunks of at least kRouteChunk slots, at most
// kRouteMaxChunks of them and nc * E counts within the LDS table; 0 = one block.
int moe_route_chunk(int TK, int E) {
  if (E > kMaxE) return 0;
  return route_chunk_rule(TK, E, kRouteChunk, kRouteMaxChunks, kRouteChunkCounts);
}

hipError_t moe_route_launch(const int* idx, int T, int K, int E, int* n_groups, int* grp_expert,
                            int* grp_count, int* grp_offset, int* pair_token, int* pair_slot,
                            hipStream_t s, int* chunk_off) {
  if (E > kMaxE || T < 0 || K < 1) return hipErrorInvalidValue;
  const int TK = T * K;
  const int cs = chunk_off ? moe_route_chunk(TK, E) : 0;
  const int nc = cs ? (TK + cs - 1) / cs : 0;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(1024), 0, s, idx, T, K, E, n_groups,
                     grp_expert, grp_count, grp_offset, pair_token, pair_slot, cs ? cs : 1, nc,
                     cs ? chunk_off : nullptr);
  if (hipError_t e = hipGetLastError()) return e;
  if (cs)
    hipLaunchKernelGGL(moe_route_scatter_kernel, dim3(nc), dim3(256), 0, s, idx, TK, K, E, cs,
                       chunk_off, pair_token, pair_slot);
  return hipGetLastError();
}

hipError_t moe_finalize_launch(const float* ybuf, int T, int K, int H, const uint16_t* resid,
                               uint16_t* out, float* out_f32, hipStream_t s) {
  if (H % 4 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(moe_finalize_kernel, dim3((H / 4 + 255) / 256, T), dim3(256), 0, s, ybuf, K,
                     H, resid, out, out_f32);
  return hipGetLastError();
}

}  // namespace mkd
