// Decode attention for one new token per sequence, GQA, split-K over the KV length.
//
// qk_prep   : per (sequence, head) wave -- round the fp32 projections, per-head
//             RMSNorm over d, RoPE (rotate-half, contiguous halves), write q and
//             the new k/v rows (bf16) to a small staging buffer.
// attn_decode: grid (chunk, kv_head, sequence).  Each block owns `chunk`
//             consecutive KV positions of one kv head and all gqa query heads
//             sharing it, so every K/V byte is read from HBM exactly once.
//             Scores and the softmax numerator live in LDS; K rows are read as
//             16-byte vectors (one 256-byte row per lane), V rows coalesced
//             across the wave.  Emits (max, sum, unnormalised P*V) per chunk.
// attn_combine: merges the chunks (log-sum-exp), adds the optional sink logit,
//             writes bf16 output, and scatters the new k/v rows into the caches
//             at write_pos[b] (after all chunks have read the old cache).
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

constexpr int kAttnThreads = 256;
constexpr int kMaxGqa = 16;

// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) qk_prep_kernel(AttnArgs a, int rope_mode, int round_qwen) {
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int nh = a.nq + 2 * a.nkv;
  if (head >= nh) return;
  const int d = a.d;
  const int EL = d / 64;                 // elements per lane (1 or 2)
  float x[2];
  for (int e = 0; e < EL; ++e) {
    const int i = lane * EL + e;
    const long long off = (long long)b * a.ld_qkv + head * d + i;
    x[e] = a.qkv ? a.qkv[off] : bf2f(a.qkv_bf16[off]);
    if (round_qwen) x[e] = rbf(x[e]);
  }
  const bool is_q = head < a.nq;
  const bool is_k = !is_q && head < a.nq + a.nkv;
  if (is_q || is_k) {
    const uint16_t* nw = is_q ? a.q_norm : a.k_norm;
    if (nw) {
      float ss = 0.f;
      for (int e = 0; e < EL; ++e) ss += x[e] * x[e];
      ss = wave_sum(ss);
      const float rinv = 1.0f / sqrtf(ss * (1.0f / d) + a.qk_eps);
      for (int e = 0; e < EL; ++e) {
        x[e] = (x[e] * rinv) * bf2f(nw[lane * EL + e]);
        if (round_qwen) x[e] = rbf(x[e]);
      }
    }
    if (rope_mode) {
      float p[2];
      for (int e = 0; e < EL; ++e) p[e] = __shfl_xor(x[e], 32, 64);
      for (int e = 0; e < EL; ++e) {
        const int i = lane * EL + e;
        float c, s;
        if (rope_mode == 1) {
          c = a.cos[(long long)b * d + i];
          s = a.sin[(long long)b * d + i];
        } else {  // generate from position: angle = pos * inv_freq[i mod d/2]
          const float ang = (float)a.pos[b] * a.inv_freq[i % (d / 2)];
          c = cosf(ang);
          s = sinf(ang);
        }
        const float rot = (i < d / 2) ? -p[e] : p[e];
        if (round_qwen) {
          x[e] = rbf(rbf(x[e] * rbf(c)) + rbf(rot * rbf(s)));
        } else {
          x[e] = x[e] * c + rot * s;
        }
      }
    }
  }
  uint16_t* dst;
  if (is_q) dst = a.q_out + ((long long)b * a.nq + head) * d;
  else if (is_k) dst = a.kv_new + (((long long)b * 2 + 0) * a.nkv + (head - a.nq)) * d;
  else dst = a.kv_new + (((long long)b * 2 + 1) * a.nkv + (head - a.nq - a.nkv)) * d;
  for (int e = 0; e < EL; ++e) dst[lane * EL + e] = (uint16_t)f2bf(x[e]);
}

// ---------------------------------------------------------------------------
template <int D, int GQA>
__global__ void __launch_bounds__(kAttnThreads) attn_decode_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  float* q_s = smem;                          // [GQA][D]
  float* s_s = q_s + GQA * D;                 // [GQA][chunk]
  float* red = s_s + GQA * a.chunk;           // [kAttnThreads/ (D/2)][GQA][D] for PV reduce
  __shared__ float m_s[kMaxGqa], l_s[kMaxGqa];

  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  // prior length from device data: clamp into the cache so no read leaves it
  const int n = min(max(a.n_prior[b], 0), a.S_max);
  const int total = n + 1;                    // prior positions + the active token
  const int t_begin = c * a.chunk;
  if (t_begin >= total) return;
  const int t_end = min(t_begin + a.chunk, total);
  const int len = t_end - t_begin;

  const uint16_t* qg = a.q_out + ((long long)b * a.nq + g * GQA) * D;
  for (int i = tid; i < GQA * D; i += kAttnThreads) q_s[i] = bf2f(qg[i]);
  __syncthreads();

  const uint16_t* kbase = a.k_cache + b * a.cache_b_stride + g * a.cache_h_stride;
  const uint16_t* vbase = a.v_cache + b * a.cache_b_stride + g * a.cache_h_stride;
  const uint16_t* knew = a.kv_new + (((long long)b * 2 + 0) * a.nkv + g) * D;
  const uint16_t* vnew = a.kv_new + (((long long)b * 2 + 1) * a.nkv + g) * D;

  // ---- phase 1: scores ----
  for (int tl = tid; tl < len; tl += kAttnThreads) {
    const int t = t_begin + tl;
    const uint16_t* kr = (t < n) ? kbase + (long long)t * D : knew;
    float acc[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) acc[h] = 0.f;
#pragma unroll 4
    for (int i = 0; i < D; i += 8) {
      u32x4_t kv = ld16(kr + i);
      float kf[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) { kf[2 * j] = bf_lo(kv[j]); kf[2 * j + 1] = bf_hi(kv[j]); }
#pragma unroll
      for (int h = 0; h < GQA; ++h) {
        const f32x4_t q0 = *reinterpret_cast<const f32x4_t*>(q_s + h * D + i);
        const f32x4_t q1 = *reinterpret_cast<const f32x4_t*>(q_s + h * D + i + 4);
        acc[h] += q0[0] * kf[0] + q0[1] * kf[1] + q0[2] * kf[2] + q0[3] * kf[3] +
                  q1[0] * kf[4] + q1[1] * kf[5] + q1[2] * kf[6] + q1[3] * kf[7];
      }
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      float sc = a.round_qwen ? rbf(rbf(acc[h]) * a.scale) : acc[h] * a.scale;
      if (a.mask) {
        const int mt = (t < n) ? t : (a.mask_s_ctx - 1);
        if (!a.mask[((long long)mt * a.B + b) * a.nq + g * GQA + h]) sc = -INFINITY;
      }
      s_s[h * a.chunk + tl] = sc;
    }
  }
  __syncthreads();

  // ---- phase 2: chunk max / exp / sum (one wave per head) ----
  const int lane = tid & 63, wv = tid >> 6;
  for (int h = wv; h < GQA; h += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int tl = lane; tl < len; tl += 64) m = fmaxf(m, s_s[h * a.chunk + tl]);
    m = wave_max(m);
    float l = 0.f;
    for (int tl = lane; tl < len; tl += 64) {
      const float sv = s_s[h * a.chunk + tl];
      const float e = (m == -INFINITY) ? 0.f : expf(sv - m);
      s_s[h * a.chunk + tl] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) { m_s[h] = m; l_s[h] = l; }
  }
  __syncthreads();

  // ---- phase 3: P * V ----
  constexpr int NP = D / 2;                   // bf16 pairs per row
  constexpr int NQ = kAttnThreads / NP;       // position groups
  const int p = tid % NP, qg_ = tid / NP;
  float acc0[GQA], acc1[GQA];
#pragma unroll
  for (int h = 0; h < GQA; ++h) { acc0[h] = 0.f; acc1[h] = 0.f; }
  for (int tl = qg_; tl < len; tl += NQ) {
    const int t = t_begin + tl;
    const uint16_t* vr = (t < n) ? vbase + (long long)t * D : vnew;
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(vr + 2 * p);
    const float v0 = bf_lo(vv), v1 = bf_hi(vv);
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      const float e = s_s[h * a.chunk + tl];
      acc0[h] += e * v0;
      acc1[h] += e * v1;
    }
  }
#pragma unroll
  for (int h = 0; h < GQA; ++h) {
    red[(qg_ * GQA + h) * D + 2 * p] = acc0[h];
    red[(qg_ * GQA + h) * D + 2 * p + 1] = acc1[h];
  }
  __syncthreads();
  for (int o = tid; o < GQA * D; o += kAttnThreads) {
    const int h = o / D, i = o % D;
    float s = 0.f;
    for (int q = 0; q < NQ; ++q) s += red[(q * GQA + h) * D + i];
    const int hq = g * GQA + h;
    a.part_o[(((long long)b * a.nq + hq) * a.n_chunks + c) * D + i] = s;
    if (i == 0) {
      float* ml = a.part_ml + (((long long)b * a.nq + hq) * a.n_chunks + c) * 2;
      ml[0] = m_s[h];
      ml[1] = l_s[h];
    }
  }
}

// ---------------------------------------------------------------------------
__global__ void attn_combine_kernel(AttnArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int i = threadIdx.x;                  // blockDim = d
  const int d = a.d;
  const int nch = (min(max(a.n_prior[b], 0), a.S_max) + 1 + a.chunk - 1) / a.chunk;
  const float* ml = a.part_ml + ((long long)b * a.nq + h) * a.n_chunks * 2;
  float M = -INFINITY;
  for (int c = 0; c < nch; ++c) M = fmaxf(M, ml[2 * c]);
  if (a.sink) M = fmaxf(M, a.sink[h]);
  float L = 0.f, o = 0.f;
  const float* po = a.part_o + ((long long)b * a.nq + h) * a.n_chunks * d;
  for (int c = 0; c < nch; ++c) {
    const float mc = ml[2 * c];
    const float w = (mc == -INFINITY) ? 0.f : expf(mc - M);
    L += ml[2 * c + 1] * w;
    o += po[(long long)c * d + i] * w;
  }
  if (a.sink) L += expf(a.sink[h] - M);
  const float out = (L > 0.f) ? o / L : 0.f;
  a.attn_out[((long long)b * a.nq + h) * d + i] = (uint16_t)f2bf(out);

  // In-place KV scatter of the new rows (one block per kv head does it).
  if (a.update_cache && h < a.nkv) {
    const int wp = a.write_pos ? a.write_pos[b] : a.pos[b];
    if (wp >= 0 && wp < a.S_max) {
      const long long off = b * a.cache_b_stride + h * a.cache_h_stride + (long long)wp * d + i;
      a.k_cache[off] = a.kv_new[(((long long)b * 2 + 0) * a.nkv + h) * d + i];
      a.v_cache[off] = a.kv_new[(((long long)b * 2 + 1) * a.nkv + h) * d + i];
    }
  }
}

// ---------------------------------------------------------------------------
hipError_t qk_prep_launch(const AttnArgs& a, int rope_mode, int round_qwen, hipStream_t s) {
  if (a.d != 64 && a.d != 128) return hipErrorInvalidValue;
  const int nh = a.nq + 2 * a.nkv;
  hipLaunchKernelGGL(qk_prep_kernel, dim3((nh + 3) / 4, a.B), dim3(256), 0, s, a, rope_mode,
                     round_qwen);
  return hipGetLastError();
}

template <int D, int GQA>
static hipError_t attn_t(const AttnArgs& a, hipStream_t s) {
  const size_t lds = (size_t)(GQA * D + GQA * a.chunk + (kAttnThreads / (D / 2)) * GQA * D) *
                     sizeof(float);
  hipLaunchKernelGGL((attn_decode_kernel<D, GQA>), dim3(a.n_chunks, a.nkv, a.B),
                     dim3(kAttnThreads), lds, s, a);
  return hipGetLastError();
}

hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t s) {
  const int gqa = a.nq / a.nkv;
  if (a.d == 128) {
    if (gqa == 8) return attn_t<128, 8>(a, s);
    if (gqa == 4) return attn_t<128, 4>(a, s);
    if (gqa == 1) return attn_t<128, 1>(a, s);
    if (gqa == 2) return attn_t<128, 2>(a, s);
    if (gqa == 16) return attn_t<128, 16>(a, s);
  } else if (a.d == 64) {
    if (gqa == 8) return attn_t<64, 8>(a, s);
    if (gqa == 4) return attn_t<64, 4>(a, s);
    if (gqa == 1) return attn_t<64, 1>(a, s);
    if (gqa == 2) return attn_t<64, 2>(a, s);
    if (gqa == 16) return attn_t<64, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t attn_combine_launch(const AttnArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nq, a.B), dim3(a.d), 0, s, a);
  return hipGetLastError();
}

}  // namespace mkd
