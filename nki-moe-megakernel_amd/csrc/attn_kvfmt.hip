// Decode attention over the operator's optional KV cache formats
// (attention_block_tkg.py:112 K_cache_transposed, :197-202 its flat layout
// [B, d, S_ctx]; :133-134, :213-218, :749-754 k_scale / v_scale with float8
// e4m3 caches, new rows quantised by _quantize_to_fp8 :1694-1737 and used by
// the attention as stored, attention_tkg.py:749-821).
//
// These formats are served by one split-K kernel of plain VALU math instead of
// the MFMA kernels of attn_mfma.hip: the MFMA score operand needs 8
// consecutive head elements of one position per lane, which a [d, S] K cache
// stores S_max elements apart, and an e4m3 row is decoded element by element
// anyway.  One position per thread: a thread reads its key (a row of a
// [S, d] cache, or d elements that consecutive threads read side by side in a
// [d, S] cache), forms the scores of the kv group's query heads against the
// queries in LDS, the block takes per-head (max, sum) over its chunk, and the
// threads then accumulate P . V over the chunk with each thread owning two
// head elements of a few heads.  The partials go to part_o / part_ml in the
// layout attn_combine_kernel merges, so the sink, the output and the output
// projection are the default path's.
//
// e4m3 codes and their quantiser: fp8.h.
#include "common.h"
#include "fp8.h"
#include "mkd_internal.h"
#include "attn_common.h"

namespace mkd {

namespace {

constexpr int kKvMaxChunk = 256;      // positions per block (attn_chunk_for: 64 / 128 / 256)
constexpr int kKvMaxNew = 8;          // new tokens per sequence

// the stored code of a new k / v element (attention_block_tkg.py:1694-1737)
MKD_DEV uint32_t kv_quant(float x, float scale) { return fp8_quant(x, scale); }

// Element offset of position t, element 0 of kv head g in row r's sequence
// (V, or K when it is not transposed); -1 where a block table holds no block.
MKD_DEV long long kv_row_off(const AttnArgs& a, int r, int g, int t, int D) {
  const int b = seq_of(a, r);
  if (!a.block_table) return b * a.cache_b_stride + g * a.cache_h_stride + (long long)t * D;
  const int blk = a.block_table[(long long)b * a.tbl_stride + t / a.blk_len];
  if ((unsigned)blk >= (unsigned)a.num_blocks) return -1;
  return (((long long)blk * a.blk_len + t % a.blk_len) * a.nkv + g) * D;
}

// 8 elements of a cache row as floats (bf16 bits or e4m3 codes)
template <bool FP8>
MKD_DEV void load8(const void* cache, long long off, float (&x)[8]) {
  if constexpr (FP8) {
    const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(cache) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = e4m3_decode((v.x >> (8 * e)) & 0xffu);
      x[4 + e] = e4m3_decode((v.y >> (8 * e)) & 0xffu);
    }
  } else {
    const u32x4_t v = ld16(static_cast<const uint16_t*>(cache) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf2f(v[e] & 0xffffu);
      x[2 * e + 1] = bf2f(v[e] >> 16);
    }
  }
}

template <bool FP8>
MKD_DEV float load1(const void* cache, long long off) {
  if constexpr (FP8) return e4m3_decode(static_cast<const uint8_t*>(cache)[off]);
  else return bf2f(static_cast<const uint16_t*>(cache)[off]);
}

// two consecutive elements (off even)
template <bool FP8>
MKD_DEV float2 load2(const void* cache, long long off) {
  if constexpr (FP8) {
    const uint32_t v = *reinterpret_cast<const uint16_t*>(static_cast<const uint8_t*>(cache) + off);
    return float2{e4m3_decode(v & 0xffu), e4m3_decode(v >> 8)};
  } else {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(cache) + off);
    return float2{bf2f(v & 0xffffu), bf2f(v >> 16)};
  }
}

}  // namespace

// Block (chunk c, kv head g, query row r), 256 threads.
template <int D, int GQA, bool FP8, bool KT>
__global__ void __launch_bounds__(256) attn_kvfmt_kernel(AttnArgs a) {
  __shared__ float q_s[GQA][D];
  __shared__ float kn_s[kKvMaxNew][D], vn_s[kKvMaxNew][D];
  __shared__ float p_s[GQA][kKvMaxChunk];
  __shared__ long long vo_s[kKvMaxChunk];       // V row offsets of the chunk's cache positions
  __shared__ float m_s[GQA], l_s[GQA];
  const int c = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int CP = a.chunk, chunk0 = c * CP;
  const int NT = new_tokens(a), seq = seq_of(a, r), tk = tok_of(a, r);
  const int n = prior_len(a, r), total = n + NT;
  if (chunk0 >= total) return;                  // whole block: uniform exit
  const int cl = min(CP, total - chunk0);       // live positions of the chunk

  // the query heads of (r, g) and the sequence's new k / v rows (as stored)
  const uint16_t* qsrc = a.prep + ((long long)r * a.nkv + g) * (GQA + 2) * D;
  for (int i = tid; i < GQA * D; i += 256) q_s[i / D][i % D] = bf2f(qsrc[i]);
  for (int i = tid; i < NT * D; i += 256) {
    const int s = i / D, e = i % D;
    const uint16_t* src = a.prep + (((long long)seq * NT + s) * a.nkv + g) * (GQA + 2) * D;
    float kv = bf2f(src[GQA * D + e]), vv = bf2f(src[(GQA + 1) * D + e]);
    if constexpr (FP8) {
      kv = e4m3_decode(kv_quant(kv, a.k_scale[0]));
      vv = e4m3_decode(kv_quant(vv, a.v_scale[0]));
    }
    kn_s[s][e] = kv;
    vn_s[s][e] = vv;
  }
  __syncthreads();

  // ---- scores: one position per thread ----
  for (int tl = tid; tl < cl; tl += 256) {
    const int t = chunk0 + tl;
    float acc[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) acc[h] = 0.f;
    long long vo = -1;
    if (t < n) {
      vo = kv_row_off(a, r, g, t, D);
      if constexpr (KT) {   // flat [.., d, S_max]: consecutive threads read consecutive t
        const long long k0 = seq * a.cache_b_stride + g * a.cache_h_stride + t;
#pragma unroll 8
        for (int e = 0; e < D; ++e) {
          const float kx = load1<FP8>(a.k_cache, k0 + (long long)e * a.S_max);
#pragma unroll
          for (int h = 0; h < GQA; ++h) acc[h] += q_s[h][e] * kx;
        }
      } else if (vo >= 0) {
#pragma unroll 2
        for (int e0 = 0; e0 < D; e0 += 8) {
          float kx[8];
          load8<FP8>(a.k_cache, vo + e0, kx);
#pragma unroll
          for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int h = 0; h < GQA; ++h) acc[h] += q_s[h][e0 + e] * kx[e];
        }
      }
    } else {
      const float* kr = kn_s[t - n];
#pragma unroll 4
      for (int e = 0; e < D; ++e)
#pragma unroll
        for (int h = 0; h < GQA; ++h) acc[h] += q_s[h][e] * kr[e];
    }
    vo_s[tl] = vo;
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
      float sc = a.round_qwen ? rbf(rbf(acc[h]) * a.scale) : acc[h] * a.scale;
      bool ok = true;
      if (a.mask) {
        const int mt = (t < n) ? t : (a.mask_s_ctx - NT + (t - n));
        ok = a.mask[(((long long)mt * (a.B / NT) + seq) * a.nq + g * GQA + h) * NT + tk] != 0;
      }
      p_s[h][tl] = ok ? sc : -INFINITY;
    }
  }
  __syncthreads();

  // ---- per-head max and exp-sum over the chunk: wave w takes heads w, w + 4, .. ----
  for (int h = w; h < GQA; h += 4) {
    float m = -INFINITY;
    for (int tl = lane; tl < cl; tl += 64) m = fmaxf(m, p_s[h][tl]);
    m = wave_max(m);
    float l = 0.f;
    for (int tl = lane; tl < cl; tl += 64) {
      const float p = (m == -INFINITY) ? 0.f : expf(p_s[h][tl] - m);
      p_s[h][tl] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) { m_s[h] = m; l_s[h] = l; }
  }
  __syncthreads();

  // ---- O = P . V: thread (pair j, group q) owns elements 2j, 2j+1 of heads q, q + NG, .. ----
  constexpr int NP = D / 2, NG = 256 / NP, HPG = (GQA + NG - 1) / NG;
  const int j = tid % NP, q = tid / NP;
  float ox[HPG], oy[HPG];
#pragma unroll
  for (int u = 0; u < HPG; ++u) { ox[u] = 0.f; oy[u] = 0.f; }
  if (q < GQA) {
    int tl = 0;
    for (; tl + 8 <= cl; tl += 8) {   // eight rows' loads in flight, then their math
      float2 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int t = chunk0 + tl + i;
        const long long vo = vo_s[tl + i];
        v[i] = t < n ? (vo >= 0 ? load2<FP8>(a.v_cache, vo + 2 * j) : float2{0.f, 0.f})
                     : float2{vn_s[t - n][2 * j], vn_s[t - n][2 * j + 1]};
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int u = 0; u < HPG; ++u) {
          const int h = q + u * NG;
          if (h < GQA) {
            const float p = p_s[h][tl + i];
            ox[u] += p * v[i].x;
            oy[u] += p * v[i].y;
          }
        }
    }
    for (; tl < cl; ++tl) {
      const int t = chunk0 + tl;
      const long long vo = vo_s[tl];
      const float2 v = t < n ? (vo >= 0 ? load2<FP8>(a.v_cache, vo + 2 * j) : float2{0.f, 0.f})
                             : float2{vn_s[t - n][2 * j], vn_s[t - n][2 * j + 1]};
#pragma unroll
      for (int u = 0; u < HPG; ++u) {
        const int h = q + u * NG;
        if (h < GQA) {
          const float p = p_s[h][tl];
          ox[u] += p * v.x;
          oy[u] += p * v.y;
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < HPG; ++u) {
    const int h = q + u * NG;
    if (h < GQA) {
      const int hq = g * GQA + h;
      const long long po = (((long long)r * a.nq + hq) * a.n_chunks + c) * D + 2 * j;
      *reinterpret_cast<float2*>(a.part_o + po) = float2{ox[u], oy[u]};
      if (j == 0)
        *reinterpret_cast<float2*>(a.part_ml + (((long long)r * a.nq + hq) * a.n_chunks + c) * 2) =
            float2{m_s[h], l_s[h]};
    }
  }
}

// Block (kv head g, row r), D threads: row r's prepared k / v into the caches
// at its write row -- bf16 bits or e4m3 codes, K transposed or not.
template <int D, int GQA, bool FP8, bool KT>
__global__ void __launch_bounds__(D) attn_kvfmt_store_kernel(AttnArgs a) {
  const int g = blockIdx.x, r = blockIdx.y, e = threadIdx.x;
  const long long row = kv_write_row(a, r);
  if (row < 0) return;
  const uint16_t* src = a.prep + ((long long)r * a.nkv + g) * (GQA + 2) * D;
  const uint32_t kb = src[GQA * D + e], vb = src[(GQA + 1) * D + e];
  long long ko, vo;
  if (a.block_table) {
    ko = vo = (row * a.nkv + g) * D + e;
  } else {
    const long long base = seq_of(a, r) * a.cache_b_stride + g * a.cache_h_stride;
    vo = base + row * D + e;
    ko = KT ? base + (long long)e * a.S_max + row : vo;
  }
  if constexpr (FP8) {
    static_cast<uint8_t*>(static_cast<void*>(a.k_cache))[ko] = (uint8_t)kv_quant(bf2f(kb), a.k_scale[0]);
    static_cast<uint8_t*>(static_cast<void*>(a.v_cache))[vo] = (uint8_t)kv_quant(bf2f(vb), a.v_scale[0]);
  } else {
    a.k_cache[ko] = (uint16_t)kb;
    a.v_cache[vo] = (uint16_t)vb;
  }
}

namespace {
template <int D, int GQA, bool FP8, bool KT>
hipError_t kvfmt_launch(const AttnArgs& a, bool store, hipStream_t s) {
  if (store) hipLaunchKernelGGL((attn_kvfmt_store_kernel<D, GQA, FP8, KT>), dim3(a.nkv, a.B), dim3(D), 0, s, a);
  else hipLaunchKernelGGL((attn_kvfmt_kernel<D, GQA, FP8, KT>), dim3(a.n_chunks, a.nkv, a.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int D, int GQA>
hipError_t kvfmt_fmt(const AttnArgs& a, bool store, hipStream_t s) {
  if (a.kv_fp8) return a.k_transposed ? kvfmt_launch<D, GQA, true, true>(a, store, s)
                                      : kvfmt_launch<D, GQA, true, false>(a, store, s);
  return a.k_transposed ? kvfmt_launch<D, GQA, false, true>(a, store, s)
                        : kvfmt_launch<D, GQA, false, false>(a, store, s);
}

hipError_t kvfmt_dispatch(const AttnArgs& a, bool store, hipStream_t s) {
  // the kernels' limits: chunk positions, new tokens, heads of a group
  const int nt = a.s_tkg > 1 ? a.s_tkg : 1;
  if (a.chunk <= 0 || a.chunk > kKvMaxChunk || nt > kKvMaxNew || !a.prep || a.window > 0 ||
      (a.kv_fp8 && (!a.k_scale || !a.v_scale)) ||
      a.prefill || (a.k_transposed && a.block_table) || a.nkv <= 0 || a.B % nt)
    return hipErrorInvalidValue;
  const int gqa = a.nq / a.nkv;
  if (a.d == 128) {
    switch (gqa) {
      case 1: return kvfmt_fmt<128, 1>(a, store, s);
      case 2: return kvfmt_fmt<128, 2>(a, store, s);
      case 4: return kvfmt_fmt<128, 4>(a, store, s);
      case 8: return kvfmt_fmt<128, 8>(a, store, s);
      case 16: return kvfmt_fmt<128, 16>(a, store, s);
    }
  } else if (a.d == 64) {
    switch (gqa) {
      case 1: return kvfmt_fmt<64, 1>(a, store, s);
      case 2: return kvfmt_fmt<64, 2>(a, store, s);
      case 4: return kvfmt_fmt<64, 4>(a, store, s);
      case 8: return kvfmt_fmt<64, 8>(a, store, s);
      case 16: return kvfmt_fmt<64, 16>(a, store, s);
    }
  }
  return hipErrorInvalidValue;
}
}  // namespace

hipError_t attn_kvfmt_launch(const AttnArgs& a, int rope_mode, hipStream_t s) {
  if (hipError_t e = attn_prep_launch(a, rope_mode, s)) return e;
  return kvfmt_dispatch(a, false, s);
}

hipError_t attn_kvfmt_store_launch(const AttnArgs& a, hipStream_t s) {
  if (!a.update_cache) return hipSuccess;
  return kvfmt_dispatch(a, true, s);
}

}  // namespace mkd
