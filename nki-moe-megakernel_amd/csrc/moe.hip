// Router top-k, token->expert grouping and the MoE epilogue.
//
// router_topk: one wave per token over fp32 logits [T, E] (E <= 512, K <= 8).
//   Selection: K rounds of a wave arg-max on (value desc, index asc), i.e. the
//   lowest index wins an exact tie.  Modes (bit field):
//     bit0 act      0 softmax, 1 sigmoid
//     bit1 pre_norm activation on all E before top-k (ACT1) else on the top-k (ACT2)
//     bit2 norm     L1-renormalise the top-k (ACT1 path)
//     bit3 qwen     Qwen fused flow: top-k on logits, softmax value at the top-k
//                   rounded to bf16, then bf16 L1 renormalisation
//   Outputs: expert index [T,K] (int32), top-k affinities [T,K] fp32, per-slot
//   weights [T*K] (same values), and optionally the scattered / full
//   affinities [T,E].
// moe_route: single block; counting sort of the T*K (token, k) slots by expert
//   into compact groups (live experts in ascending id order).
// moe_finalize: out[t] = bf16(sum_k y[t*K + k]) (fp32 sum in k order), then the
//   bf16 residual add.
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

constexpr int kMaxE = 512;
constexpr int kMaxPerLane = kMaxE / 64;

struct VI { float v; int i; };
MKD_DEV bool better(VI a, VI b) { return a.v > b.v || (a.v == b.v && a.i < b.i); }

MKD_DEV VI wave_argmax(VI x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    VI y{__shfl_xor(x.v, o, 64), __shfl_xor(x.i, o, 64)};
    if (better(y, x)) x = y;
  }
  return x;
}

__global__ void __launch_bounds__(256)
router_topk_kernel(const float* __restrict__ logits, int T, int E, int K, int mode,
                   float* __restrict__ aff_full, int* __restrict__ idx_out,
                   float* __restrict__ topk_out, float* __restrict__ slot_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const bool sigm = mode & 1, pre = mode & 2, norm = mode & 4, qwen = mode & 8;
  const int per = (E + 63) / 64;
  float l[kMaxPerLane], a[kMaxPerLane];
  float mx = -INFINITY;
  for (int j = 0; j < per; ++j) {
    const int e = lane + 64 * j;
    l[j] = (e < E) ? logits[(long long)t * E + e] : -INFINITY;
    mx = fmaxf(mx, l[j]);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = 0; j < per; ++j) {
    const int e = lane + 64 * j;
    a[j] = (e < E) ? expf(l[j] - mx) : 0.f;
    sum += a[j];
  }
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  // selection key
  float key[kMaxPerLane];
  for (int j = 0; j < per; ++j) {
    const int e = lane + 64 * j;
    if (e >= E) { key[j] = -INFINITY; continue; }
    if (qwen || !pre) key[j] = l[j];
    else key[j] = sigm ? 1.0f / (1.0f + expf(-l[j])) : a[j] * inv;
  }
  int sel_i[8];
  float sel_v[8];
  for (int k = 0; k < K; ++k) {
    VI best{-INFINITY, 0x7fffffff};
    for (int j = 0; j < per; ++j) {
      VI c{key[j], lane + 64 * j};
      if (c.i < E && better(c, best)) best = c;
    }
    best = wave_argmax(best);
    sel_i[k] = best.i;
    sel_v[k] = best.v;
    for (int j = 0; j < per; ++j)
      if (lane + 64 * j == best.i) key[j] = -INFINITY;
  }
  // affinities of the selected experts
  float w[8];
  if (qwen) {
    float s = 0.f;
    for (int k = 0; k < K; ++k) { w[k] = rbf(expf(sel_v[k] - mx) * inv); s += w[k]; }
    const float r = 1.0f / s;
    for (int k = 0; k < K; ++k) w[k] = rbf(w[k] * r);
  } else if (pre) {
    for (int k = 0; k < K; ++k) w[k] = sel_v[k];
    if (norm) {
      float s = 0.f;
      for (int k = 0; k < K; ++k) s += w[k];
      const float r = 1.0f / s;
      for (int k = 0; k < K; ++k) w[k] *= r;
    }
  } else {  // ACT2 on the top-k logits
    if (sigm) {
      for (int k = 0; k < K; ++k) w[k] = 1.0f / (1.0f + expf(-sel_v[k]));
    } else {
      const float m2 = sel_v[0];
      float s = 0.f;
      for (int k = 0; k < K; ++k) { w[k] = expf(sel_v[k] - m2); s += w[k]; }
      const float r = 1.0f / s;
      for (int k = 0; k < K; ++k) w[k] *= r;
    }
  }
  if (lane < K) {
    float wl = 0.f; int il = 0;
    for (int k = 0; k < K; ++k) if (k == lane) { wl = w[k]; il = sel_i[k]; }
    if (idx_out) idx_out[t * K + lane] = il;
    if (topk_out) topk_out[t * K + lane] = wl;
    if (slot_w) slot_w[t * K + lane] = wl;
  }
  if (aff_full) {
    const bool full = pre && !norm && !qwen;
    for (int j = 0; j < per; ++j) {
      const int e = lane + 64 * j;
      if (e >= E) continue;
      float v = 0.f;
      if (full) {
        v = sigm ? 1.0f / (1.0f + expf(-l[j])) : a[j] * inv;
      } else {
        for (int k = 0; k < K; ++k) if (sel_i[k] == e) v = w[k];
      }
      aff_full[(long long)t * E + e] = v;
    }
  }
}

// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
moe_route_kernel(const int* __restrict__ idx, int T, int K, int E, int* __restrict__ n_groups,
                 int* __restrict__ grp_expert, int* __restrict__ grp_count,
                 int* __restrict__ grp_offset, int* __restrict__ pair_token,
                 int* __restrict__ pair_slot) {
  __shared__ int cnt[kMaxE], off[kMaxE], gid[kMaxE], cursor[kMaxE];
  __shared__ int scan[1024];
  const int tid = threadIdx.x;
  const int TK = T * K;
  for (int e = tid; e < E; e += blockDim.x) { cnt[e] = 0; cursor[e] = 0; }
  __syncthreads();
  for (int p = tid; p < TK; p += blockDim.x) {
    const int e = idx[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scans over experts: pair offsets and live-group ids (E <= blockDim)
  int c = (tid < E) ? cnt[tid] : 0;
  int live = c > 0 ? 1 : 0;
  scan[tid] = c | (live << 20);        // pack (count, live) -- counts < 2^20
  __syncthreads();
  for (int o = 1; o < (int)blockDim.x; o <<= 1) {
    const int v = (tid >= o) ? scan[tid - o] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  const int incl = scan[tid];
  if (tid < E) {
    const int excl_cnt = (incl & 0xfffff) - c;
    const int excl_live = (incl >> 20) - live;
    off[tid] = excl_cnt;
    gid[tid] = excl_live;
    if (live) {
      grp_expert[excl_live] = tid;
      grp_count[excl_live] = c;
      grp_offset[excl_live] = excl_cnt;
    }
  }
  if (tid == blockDim.x - 1) *n_groups = incl >> 20;
  __syncthreads();
  for (int p = tid; p < TK; p += blockDim.x) {
    const int e = idx[p];
    if (e < 0 || e >= E) continue;
    const int q = off[e] + atomicAdd(&cursor[e], 1);
    pair_token[q] = p / K;
    pair_slot[q] = p;
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
hipError_t router_topk_launch(const float* logits, int T, int E, int K, int mode, float* aff_full,
                              int* idx_out, float* topk_out, float* slot_w, hipStream_t s) {
  if (E > kMaxE || K > 8 || K < 1 || K > E) return hipErrorInvalidValue;
  hipLaunchKernelGGL(router_topk_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, K, mode,
                     aff_full, idx_out, topk_out, slot_w);
  return hipGetLastError();
}

hipError_t moe_route_launch(const int* idx, int T, int K, int E, int* n_groups, int* grp_expert,
                            int* grp_count, int* grp_offset, int* pair_token, int* pair_slot,
                            hipStream_t s) {
  if (E > kMaxE) return hipErrorInvalidValue;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(1024), 0, s, idx, T, K, E, n_groups,
                     grp_expert, grp_count, grp_offset, pair_token, pair_slot);
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
