// Attention helpers shared by the decode attention kernels (attn_mfma.hip) and
// the persistent layer kernel (layer_mk.hip): per-head q / k / v preparation,
// KV-cache row addressing (flat or block layout) and the prior-length rule.
#pragma once
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

// One wave: head `head` of sequence b (kind 0 query, 1 key, 2 value) from the
// fp32 / bf16 projections to bf16 bits (attention_block_tkg.py:915-1138; Qwen
// rounding attn_fused_nki.py:393-398, 426-446, 494-498, 543-582).  Lane l < D/2
// holds elements l and l + D/2 -- the pair that rotate-half RoPE mixes -- so
// the rotation stays inside the lane; lanes >= D/2 (D = 64) hold zeros.  Split
// into load and finish so a wave can issue the loads of all its heads first.
template <int D, int MP = 8>
struct HeadPrep {
  static constexpr int HD = D / 2;
  // raw loads (converted in finish, so that a wave's loads for all its heads
  // are in flight together: a conversion inside a conditional would make the
  // compiler wait for each load where it is issued).  fp32 projections may come
  // as up to kMaxQkvParts = MP split-K partials (a.qkv_nparts), summed in order
  // (MP = 1: the caller has established a.qkv_nparts <= 1).
  static constexpr int kMaxQkvParts = MP;
  uint32_t xr[2], nr[2];   // nr: the aligned dword holding the bf16 norm weight of element i
  float xp[2][kMaxQkvParts];
  int np;
  float cs[2], sn[2], invf[2];
  int posr;
  bool f32, has_nw, rope_tab;
  long long off0;
  MKD_DEV void load(const AttnArgs& a, int rope_mode, int b, int head, int kind, int lane) {
    f32 = a.qkv != nullptr;
    const char* src = f32 ? reinterpret_cast<const char*>(a.qkv)
                          : reinterpret_cast<const char*>(a.qkv_bf16);
    // pointers that may be absent fall back to the start of the projection
    // buffer (>= 3 * D elements), whose values are then discarded
    const uint16_t* nwp = kind == 0 ? a.q_norm : (kind == 1 ? a.k_norm : nullptr);
    has_nw = nwp != nullptr;
    if (!has_nw) nwp = reinterpret_cast<const uint16_t*>(src);
    rope_tab = kind < 2 && rope_mode == 1;
    const float* cp = rope_tab ? a.cos + (long long)b * D : reinterpret_cast<const float*>(src);
    const float* sp = rope_tab ? a.sin + (long long)b * D : reinterpret_cast<const float*>(src);
    const int l = lane < HD ? lane : 0;
    off0 = (long long)b * a.ld_qkv + head * D + l;
    np = (f32 && a.qkv_nparts > 1 && head * D >= a.qkv_split_row) ? min(a.qkv_nparts, kMaxQkvParts) : 1;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = l + e * HD;
      const long long off = off0 + e * HD;
      // one aligned dword: the fp32 element, or the pair holding the bf16 one
      xr[e] = *reinterpret_cast<const uint32_t*>(src + ((off << (f32 ? 2 : 1)) & ~3LL));
      if (np > 1) {
#pragma unroll
        for (int q = 1; q < kMaxQkvParts; ++q)
          xp[e][q] = a.qkv[(long long)min(q, np - 1) * a.qkv_part_stride + off];
      }
      // the aligned dword holding the bf16 norm weight: a 16-bit load would be
      // zero-extended where it is issued, making the wave wait for it before
      // the next head's loads go out
      nr[e] = *reinterpret_cast<const uint32_t*>(nwp + (i & ~1));
      cs[e] = cp[i];
      sn[e] = sp[i];
    }
    if (kind < 2 && rope_mode == 2) {   // from the position: pos * inv_freq[i mod D/2]
      posr = a.pos[b];
#pragma unroll
      for (int e = 0; e < 2; ++e) invf[e] = a.inv_freq[l];
    }
  }
  float x[2], nw[2];
  MKD_DEV void convert(int rope_mode, int kind, int lane) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const long long off = off0 + e * HD;
      const uint32_t h16 = (off & 1) ? (xr[e] >> 16) : (xr[e] & 0xffffu);
      float v = f32 ? __uint_as_float(xr[e]) : bf2f(h16);
      if (np > 1) {
#pragma unroll
        for (int q = 1; q < kMaxQkvParts; ++q)
          if (q < np) v += xp[e][q];
      }
      x[e] = lane < HD ? v : 0.f;
      const int i = (lane < HD ? lane : 0) + e * HD;
      nw[e] = has_nw ? ((i & 1) ? bf_hi(nr[e]) : bf_lo(nr[e])) : 1.f;
      if (!rope_tab) { cs[e] = 1.f; sn[e] = 0.f; }
      if (kind < 2 && rope_mode == 2) {
        const float ang = (float)posr * invf[e];
        cs[e] = cosf(ang);
        sn[e] = sinf(ang);
      }
    }
  }
  // dst2 (optional): a second copy of the prepared row (a prefill pass's KV
  // cache row, stored here rather than by a launch of its own)
  MKD_DEV void finish(const AttnArgs& a, int rope_mode, int kind, uint16_t* dst, int lane,
                      uint16_t* dst2 = nullptr) {
    convert(rope_mode, kind, lane);
#pragma unroll
    for (int e = 0; e < 2; ++e)
      if (a.round_qwen) x[e] = rbf(x[e]);
    if (kind < 2) {
      if (has_nw) {   // the head's q_norm / k_norm weights are present (load / fill)
        const float ss = wave_sum(x[0] * x[0] + x[1] * x[1]);
        const float rinv = 1.0f / sqrtf(ss * (1.0f / D) + a.qk_eps);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          x[e] = (x[e] * rinv) * nw[e];
          if (a.round_qwen) x[e] = rbf(x[e]);
        }
      }
      if (rope_mode) {
        // element i < D/2 pairs with -x[i + D/2], element i + D/2 with x[i]
        const float rot[2] = {-x[1], x[0]};
#pragma unroll
        for (int e = 0; e < 2; ++e)
          x[e] = a.round_qwen ? rbf(rbf(x[e] * rbf(cs[e])) + rbf(rot[e] * rbf(sn[e])))
                              : x[e] * cs[e] + rot[e] * sn[e];
      }
      // post-RoPE RMSNorm (attention_block_tkg.py:906-910, 1093-1138); its
      // weights are loaded here only when present, so the default path issues
      // no extra loads
      const uint16_t* pw = kind == 0 ? a.q_norm_post : a.k_norm_post;
      if (pw) {
        const int i0 = lane < HD ? lane : 0;
        const float w0 = bf2f(pw[i0]), w1 = bf2f(pw[i0 + HD]);
        const float ss = wave_sum(x[0] * x[0] + x[1] * x[1]);
        const float rinv = 1.0f / sqrtf(ss * (1.0f / D) + a.qk_post_eps);
        x[0] = (x[0] * rinv) * w0;
        x[1] = (x[1] * rinv) * w1;
        if (a.round_qwen) { x[0] = rbf(x[0]); x[1] = rbf(x[1]); }
      }
    }
    if (lane < HD) {
      const uint16_t o0 = (uint16_t)f2bf(x[0]), o1 = (uint16_t)f2bf(x[1]);
      dst[lane] = o0;
      dst[lane + HD] = o1;
      if (dst2) {
        dst2[lane] = o0;
        dst2[lane + HD] = o1;
      }
    }
  }
};

// Sequence of row r and its token slot (several new tokens per sequence, AttnArgs::s_tkg).
MKD_DEV int seq_of(const AttnArgs& a, int r) { return a.s_tkg > 1 ? r / a.s_tkg : r; }
MKD_DEV int tok_of(const AttnArgs& a, int r) { return a.s_tkg > 1 ? r % a.s_tkg : 0; }
MKD_DEV int new_tokens(const AttnArgs& a) { return a.s_tkg > 1 ? a.s_tkg : 1; }

// Position t of kv head g in the cache of row b's sequence (flat or block
// layout); null when the block table holds no valid block there (the row then
// reads as zero).
template <int D>
MKD_DEV const uint16_t* kv_row(const AttnArgs& a, const uint16_t* cache, int r, int g, int t) {
  const int b = seq_of(a, r);
  if (!a.block_table) return cache + b * a.cache_b_stride + g * a.cache_h_stride + (long long)t * D;
  const int blk = a.block_table[(long long)b * a.tbl_stride + t / a.blk_len];
  if ((unsigned)blk >= (unsigned)a.num_blocks) return nullptr;
  return cache + (((long long)blk * a.blk_len + t % a.blk_len) * a.nkv + g) * D;
}

// Prior positions attended by sequence b (the new token sits at index n).
MKD_DEV int prior_clamp(const AttnArgs& a, int raw) {
  int n = max(raw, 0);
  if (a.window > 0) n = min(n, a.window - 1);
  return min(n, a.S_max);
}
MKD_DEV int prior_len(const AttnArgs& a, int r) {
  int n = max(a.n_prior[seq_of(a, r)], 0);
  if (a.window > 0) n = min(n, a.window - 1);
  return min(n, a.S_max);
}

// The raw count by a vector load, for prior_clamp once it is needed: a scalar
// load would be waited for together with every scalar load before it
// (lgkmcnt(0)), so address math issued after it that does not need the count
// would wait for its round trip too.  (The zero offset comes from a VGPR so
// that the uniform address is not turned into a scalar load.)
MKD_DEV int prior_raw_vmem(const AttnArgs& a, int r) {
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  return a.n_prior[seq_of(a, r) + zero];
}

// Cache row that receives row r's new token (-1: skip): token s of a sequence
// goes s rows after the sequence's write position (a global row of a block
// cache).
MKD_DEV long long kv_write_row(const AttnArgs& a, int r) {
  const int b = seq_of(a, r), s = tok_of(a, r);
  if (!a.block_table) {
    int wp = a.write_pos ? a.write_pos[b] : a.pos[b];
    if (a.window > 1 && !a.write_pos) wp = wp >= 0 ? wp % (a.window - 1) : -1;
    if (wp < 0) return -1;
    wp += s;
    return wp < a.S_max ? wp : -1;
  }
  long long row;
  if (a.write_pos) {
    row = a.write_pos[b];
    if (row < 0) return -1;
    row += s;
  } else {
    const int p = a.pos[b];
    if (p < 0 || p >= a.S_max) return -1;
    const int blk = a.block_table[(long long)b * a.tbl_stride + p / a.blk_len];
    if ((unsigned)blk >= (unsigned)a.num_blocks) return -1;
    row = (long long)blk * a.blk_len + p % a.blk_len;
  }
  return (row >= 0 && row < (long long)a.num_blocks * a.blk_len) ? row : -1;
}

}  // namespace mkd
