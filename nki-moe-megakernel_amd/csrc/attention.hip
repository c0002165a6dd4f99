// Decode attention for one new token per sequence, GQA, split-K over the KV length.
//
// qk_prep   : per (sequence, head) wave -- round the fp32 projections, per-head
//             RMSNorm over d, RoPE (rotate-half, contiguous halves), write q and
//             the new k/v rows (bf16) to a small staging buffer.
// attn_decode: the split-K MFMA kernel in attn_mfma.hip.
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
constexpr int kMaxChunks = 1024;

__global__ void __launch_bounds__(128) attn_combine_kernel(AttnArgs a) {
  __shared__ float wch[kMaxChunks];
  __shared__ float red[2];
  const int h = blockIdx.x, b = blockIdx.y;
  const int i = threadIdx.x;                  // blockDim = d (64 or 128)
  const int lane = i & 63, wv = i >> 6, nw = blockDim.x >> 6;
  const int d = a.d;
  const int nch = (min(max(a.n_prior[b], 0), a.S_max) + 1 + a.chunk - 1) / a.chunk;
  const float* ml = a.part_ml + ((long long)b * a.nq + h) * a.n_chunks * 2;
  // chunk weights exp(m_c - M) in LDS, computed by all threads in parallel
  float M = -INFINITY;
  for (int c = i; c < nch; c += blockDim.x) M = fmaxf(M, ml[2 * c]);
  M = wave_max(M);
  if (lane == 0) red[wv] = M;
  __syncthreads();
  M = red[0];
  for (int q = 1; q < nw; ++q) M = fmaxf(M, red[q]);
  if (a.sink) M = fmaxf(M, a.sink[h]);
  float L = 0.f;
  for (int c = i; c < nch; c += blockDim.x) {
    const float mc = ml[2 * c];
    const float w = (mc == -INFINITY) ? 0.f : expf(mc - M);
    wch[c] = w;
    L += ml[2 * c + 1] * w;
  }
  L = wave_sum(L);
  __syncthreads();
  if (lane == 0) red[wv] = L;
  __syncthreads();
  L = 0.f;
  for (int q = 0; q < nw; ++q) L += red[q];
  if (a.sink) L += expf(a.sink[h] - M);
  const float* po = a.part_o + ((long long)b * a.nq + h) * a.n_chunks * d + i;
  float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
  int c = 0;
  for (; c + 4 <= nch; c += 4) {
    o0 += po[(long long)(c + 0) * d] * wch[c + 0];
    o1 += po[(long long)(c + 1) * d] * wch[c + 1];
    o2 += po[(long long)(c + 2) * d] * wch[c + 2];
    o3 += po[(long long)(c + 3) * d] * wch[c + 3];
  }
  for (; c < nch; ++c) o0 += po[(long long)c * d] * wch[c];
  const float o = (o0 + o1) + (o2 + o3);
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

hipError_t attn_combine_launch(const AttnArgs& a, hipStream_t s) {
  if (a.n_chunks > kMaxChunks || (a.d != 64 && a.d != 128)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nq, a.B), dim3(a.d), 0, s, a);
  return hipGetLastError();
}

}  // namespace mkd
