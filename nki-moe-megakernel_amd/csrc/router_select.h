// Router top-k selection body shared by the router select kernel (moe.hip) and
// the persistent layer kernel (layer_mk.hip).
#pragma once
#include "common.h"
#include "mkd_internal.h"
#include "coherent.h"

namespace mkd {

constexpr int kMaxE = 512;
constexpr int kMaxPerLane = kMaxE / 64;

// ---------------------------------------------------------------------------
// Router select: one block (16 waves) for all T <= 128 tokens; wave w takes
// tokens w, w+16, ...  Logits are the in-order sum of the split-K partials
// (+ bias), all partial loads of a lane issued together.  Selection is
// rank-based: element e gets slot r = #{e' : key[e'] > key[e] or (key[e'] ==
// key[e] and e' < e)} and is chosen when r < K -- descending order, lowest
// index first among equal keys.  The K chosen are found by a radix select over
// the keys' order-preserving codes (32 ballot steps per token, no data-
// dependent branches); only those K are then ranked against each other.  Optionally the
// same block then builds the expert groups: per-expert counts in LDS, one
// wave scans them, the slots are scattered by expert.
// Unsigned code with the order of the float (+0 and -0 share one code, NaN sorts
// above +inf as in torch.topk).
MKD_DEV uint32_t order_code(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b << 1) == 0) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// Number of set bits of `m` at lanes below this one.
MKD_DEV int lanes_below(unsigned long long m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Exclusive prefix sum over the wave: Hillis-Steele inside each row of 16
// lanes with DPP row_shr 1/2/4/8 (a source outside the row reads 0), then the
// row totals (readlane of lanes 15/31/47) are added to the later rows.
template <int CTRL>
MKD_DEV int dpp_shr_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
MKD_DEV int wave_excl_scan(int v, int lane) {
  int x = v;
  x += dpp_shr_i<0x111>(x);
  x += dpp_shr_i<0x112>(x);
  x += dpp_shr_i<0x114>(x);
  x += dpp_shr_i<0x118>(x);
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane >> 4;
  x += (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
  return x - v;
}

// Sum of the split-K partial logits of token t for the lane's experts (+ the
// bias): a whole batch of loads is issued (slots past nparts re-read the last
// partial and are masked out) before summing in fixed order.
// NPM: partial count the loads are unrolled for (a.nparts <= NPM; the partials
// past a.nparts repeat the last one and are not added).
template <int PER, int NPM = 16>
MKD_DEV void load_logits(const RouterArgs& a, int t, int lane, float (&l)[PER]) {
  const int E = a.E;
  uint32_t braw[PER];                   // bias bits, loaded with the partials
  if (a.bias) {
#pragma unroll
    for (int j = 0; j < PER; ++j) braw[j] = a.bias[min(lane + 64 * j, E - 1)];
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) l[j] = 0.f;
  constexpr int PB = (PER <= 2) ? NPM : 4;
#pragma unroll
  for (int p0 = 0; p0 < NPM; p0 += PB) {
    float v[PB][PER];
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int pp = min(p0 + q, a.nparts - 1);
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = min(lane + 64 * j, E - 1);
        v[q][j] = a.parts[pp * a.part_stride + (long long)t * E + e];
      }
    }
#pragma unroll
    for (int q = 0; q < PB; ++q)
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (p0 + q < a.nparts) l[j] += v[q][j];
  }
  if (a.bias) {
#pragma unroll
    for (int j = 0; j < PER; ++j) l[j] += bf2f(braw[j]);
  }
}

// Top-k, weights and expert grouping for the T tokens of one block (16 waves;
// wave w takes tokens w, w+16, ...).  load(t, l) fills the lane's logits l[j] of
// experts lane + 64 j (bias included).
template <int PER, class Load>
MKD_DEV void select_body(const RouterArgs& a, Load&& load) {
  __shared__ uint32_t cu_s[16][8];
  __shared__ int ce_s[16][8], slot_s[16][8];
  __shared__ float ck_s[16][8];
  __shared__ float sel_s[16][8], pw_s[16][8];
  __shared__ float wsel_s[16][8];
  __shared__ int idx_s[128 * 8];
  __shared__ int cnt[kMaxE], off[kMaxE], cursor[kMaxE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int E = a.E, K = a.K, T = a.T;
  const bool sigm = a.mode & 1, pre = a.mode & 2, norm = a.mode & 4, qwen = a.mode & 8;
  for (int e = tid; e < E; e += blockDim.x) { cnt[e] = 0; cursor[e] = 0; }
  for (int t = wv; t < T; t += 16) {
    float l[PER];
    load(t, l);
    // every slot of the token starts invalid so that NaN logits (no consistent
    // ranks) can never route a slot to an out-of-range expert below
    if (lane < K) idx_s[t * K + lane] = -1;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      if (e < E) {
        if (a.logits_out) a.logits_out[(long long)t * E + e] = l[j];
      } else {
        l[j] = -INFINITY;
      }
      mx = fmaxf(mx, l[j]);
    }
    mx = wave_max(mx);
    float sum = 0.f, ex[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      ex[j] = (lane + 64 * j < E) ? expf(l[j] - mx) : 0.f;
      sum += ex[j];
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    // ---- top-K: radix select on order-preserving key codes ----
    // The threshold is the code of the K-th largest key, found bit by bit from
    // the top with wave ballots; keys above it are taken, keys equal to it are
    // taken lowest index first until K.  Slots e >= E get code 0, below every
    // real key.
    float key[PER];
    uint32_t u[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      key[j] = (qwen || !pre) ? l[j] : (sigm ? 1.0f / (1.0f + expf(-l[j])) : ex[j] * inv);
      u[j] = (e < E) ? order_code(key[j]) : 0u;
    }
    uint32_t thr = 0, hmask = 0;
    int kt = K;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t m = hmask | (1u << bit), want = thr | (1u << bit);
      int c = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j) c += __popcll(__ballot((u[j] & m) == want));
      if (c >= kt) thr = want;
      else kt -= c;
      hmask = m;
    }
    // compact the K chosen elements (index order) into the wave's candidate slots
    int cpos[PER];
    int nsel = 0, ties = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const unsigned long long eq = __ballot(u[j] == thr);
      const bool take = u[j] > thr || (u[j] == thr && ties + lanes_below(eq) < kt);
      const unsigned long long tm = __ballot(take);
      cpos[j] = take ? nsel + lanes_below(tm) : -1;
      if (take) {
        cu_s[wv][cpos[j]] = u[j];
        ce_s[wv][cpos[j]] = lane + 64 * j;
        ck_s[wv][cpos[j]] = key[j];
      }
      nsel += __popcll(tm);
      ties += __popcll(eq);
    }
    wave_lds_sync();
    // output slot = rank among the K chosen (key descending, index ascending);
    // each lane also forms its slot's term of the weight normalisation
    if (lane < K) {
      const uint32_t ui = cu_s[wv][lane];
      const int ei = ce_s[wv][lane];
      int r = 0;
      for (int m = 0; m < K; ++m) {
        const uint32_t um = cu_s[wv][m];
        r += (um > ui) | ((um == ui) & (ce_s[wv][m] < ei));
      }
      idx_s[t * K + r] = ei;
      sel_s[wv][r] = ck_s[wv][lane];
      slot_s[wv][lane] = r;
    }
    wave_lds_sync();
    if (lane < K) {
      const float sv = sel_s[wv][lane];
      float pv;
      if (qwen) pv = rbf(expf(sv - mx) * inv);        // softmax value at the logit, bf16
      else if (pre) pv = sv;
      else if (sigm) pv = 1.0f / (1.0f + expf(-sv));
      else pv = expf(sv - sel_s[wv][0]);             // softmax over the top-k (slot 0 = max)
      pw_s[wv][lane] = pv;
    }
    wave_lds_sync();
    if (lane < K) {
      const float pv = pw_s[wv][lane];
      float w = pv;
      if (qwen || (pre && norm) || (!pre && !sigm)) {
        float s = 0.f;                                 // k order
        for (int k = 0; k < K; ++k) s += pw_s[wv][k];
        w = qwen ? rbf(pv * (1.0f / s)) : pv * (1.0f / s);
      }
      wsel_s[wv][lane] = w;
      const int e = idx_s[t * K + lane];
      if (a.idx_out) a.idx_out[t * K + lane] = e;
      if (a.topk_out) a.topk_out[t * K + lane] = w;
      if (a.slot_w) a.slot_w[t * K + lane] = w;
    }
    wave_lds_sync();
    if (a.aff_full) {
      const bool full = pre && !norm && !qwen;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = lane + 64 * j;
        if (e >= E) continue;
        float v;
        if (full) v = sigm ? 1.0f / (1.0f + expf(-l[j])) : ex[j] * inv;
        else v = cpos[j] >= 0 ? wsel_s[wv][slot_s[wv][cpos[j]]] : 0.f;
        a.aff_full[(long long)t * E + e] = v;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (!a.n_groups) return;
  __syncthreads();
  // ---- expert groups: per-expert counts, one wave scans them ----
  for (int p = tid; p < T * K; p += blockDim.x) {
    const int e = idx_s[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (wv == 0) {
    constexpr int PE = kMaxE / 64;
    int c[PE], lsum = 0, llive = 0;
#pragma unroll
    for (int j = 0; j < PE; ++j) {
      const int e = lane * PE + j;
      c[j] = (e < E) ? cnt[e] : 0;
      lsum += c[j];
      llive += c[j] > 0;
    }
    int base = wave_excl_scan(lsum, lane);
    int gbase = wave_excl_scan(llive, lane);
#pragma unroll
    for (int j = 0; j < PE; ++j) {
      const int e = lane * PE + j;
      if (e < E) {
        off[e] = base;
        if (c[j] > 0) {
          a.grp_expert[gbase] = e;
          a.grp_count[gbase] = c[j];
          a.grp_offset[gbase] = base;
          ++gbase;
        }
      }
      base += c[j];
    }
    if (lane == 63) *a.n_groups = gbase;
  }
  __syncthreads();
  for (int p = tid; p < T * K; p += blockDim.x) {
    const int e = idx_s[p];
    if (e < 0 || e >= E) continue;
    const int q = off[e] + atomicAdd(&cursor[e], 1);
    a.pair_token[q] = p / K;
    a.pair_slot[q] = p;
  }
}

// Unsigned wave max (every lane gets the result); the wave must be fully active.
template <int CTRL>
MKD_DEV uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
MKD_DEV uint32_t wave_max_u(uint32_t v) {
  v = max(v, dpp_u<0xB1>(v));
  v = max(v, dpp_u<0x4E>(v));
  v = max(v, dpp_u<0x141>(v));
  v = max(v, dpp_u<0x140>(v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// Top-k, weights and expert groups for a few tokens: T <= the block's waves and
// T * K <= 64 (the decode step at small batch), with the values of select_body
// in every mode (aff_full is not produced).  Wave t takes token t; the K chosen
// come out already in rank order from K rounds of a wave-wide max over the
// order codes (largest code, lowest index among equal codes: select_body's
// order), lane r holding rank r.  After one block barrier wave 0 forms the
// groups from the T * K pairs directly (experts ascending, pairs of an expert in
// token order): pair p's position is #{valid q : e_q < e_p} + #{q < p : e_q ==
// e_p}.  The caller synchronises the block before reading the group tables.
template <int PER, class Load>
MKD_DEV void select_small(const RouterArgs& a, Load&& load) {
  __shared__ int pe_s[64];                 // expert of pair t * K + rank
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int E = a.E, K = a.K, T = a.T;
  const bool sigm = a.mode & 1, pre = a.mode & 2, norm = a.mode & 4, qwen = a.mode & 8;
  if (wv < T) {
    const int t = wv;
    float l[PER];
    load(t, l);
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      if (e < E) {
        if (a.logits_out) a.logits_out[(long long)t * E + e] = l[j];
      } else {
        l[j] = -INFINITY;
      }
      mx = fmaxf(mx, l[j]);
    }
    mx = wave_max(mx);
    float sum = 0.f, ex[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      ex[j] = (lane + 64 * j < E) ? expf(l[j] - mx) : 0.f;
      sum += ex[j];
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    float key[PER];
    uint32_t u[PER];
    bool av[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      key[j] = (qwen || !pre) ? l[j] : (sigm ? 1.0f / (1.0f + expf(-l[j])) : ex[j] * inv);
      u[j] = order_code(key[j]);
      av[j] = lane + 64 * j < E;
    }
    int my_e = -1;
    float my_key = 0.f;
    for (int r = 0; r < K; ++r) {
      uint32_t m = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (av[j]) m = max(m, u[j]);
      m = wave_max_u(m);
      int pick = -1;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const unsigned long long hit = __ballot(av[j] && u[j] == m);
        if (pick < 0 && hit) pick = 64 * j + (int)__builtin_ctzll(hit);
      }
      const int pl = pick & 63, pj = pick >> 6;
      float kv = key[0];
#pragma unroll
      for (int j = 1; j < PER; ++j)
        if (j == pj) kv = key[j];
      kv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, kv), pl));
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (j == pj && lane == pl) av[j] = false;
      if (lane == r) {
        my_e = pick;
        my_key = kv;
      }
    }
    // weights: lane r < K holds rank r
    const float k0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_key), 0));
    float pv;
    if (qwen) pv = rbf(expf(my_key - mx) * inv);   // softmax value at the logit, bf16
    else if (pre) pv = my_key;
    else if (sigm) pv = 1.0f / (1.0f + expf(-my_key));
    else pv = expf(my_key - k0);                    // softmax over the top-k (rank 0 = max)
    float w = pv;
    if (qwen || (pre && norm) || (!pre && !sigm)) {
      float s = 0.f;                                 // k order
      for (int k = 0; k < K; ++k)
        s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), k));
      w = qwen ? rbf(pv * (1.0f / s)) : pv * (1.0f / s);
    }
    if (lane < K) {
      pe_s[t * K + lane] = my_e;
      if (a.idx_out) a.idx_out[t * K + lane] = my_e;
      if (a.topk_out) a.topk_out[t * K + lane] = w;
      if (a.slot_w) a.slot_w[t * K + lane] = w;
    }
  }
  if (!a.n_groups) return;
  __syncthreads();
  if (wv == 0) {
    const int P = T * K;
    const int e = lane < P ? pe_s[lane] : -1;
    const bool valid = e >= 0 && e < E;
    int less = 0, before = 0, cnt = 0;
    for (int q = 0; q < P; ++q) {
      const int eq = __builtin_amdgcn_readlane(e, q);
      const bool vq = eq >= 0 && eq < E;
      less += vq && eq < e;
      before += q < lane && eq == e;
      cnt += eq == e;
    }
    const bool first = valid && before == 0;
    const unsigned long long fm = __ballot(first);
    int g = 0;
    for (int q = 0; q < P; ++q)
      if ((fm >> q) & 1) g += __builtin_amdgcn_readlane(e, q) < e;
    if (valid) {
      a.pair_token[less + before] = lane / K;
      a.pair_slot[less + before] = lane;
    }
    if (first) {
      a.grp_expert[g] = e;
      a.grp_count[g] = cnt;
      a.grp_offset[g] = less;
    }
    if (lane == 0) *a.n_groups = __popcll(fm);
  }
}


// select_small for ONE token, spread over the whole block (blockDim.x >= 4 E,
// a multiple of 64): wave 0 forms the logits, the softmax statistics and the
// keys exactly as select_small does, the keys' order codes go to LDS, and every
// expert's rank -- #{valid e' : code[e'] > code[e] or (code[e'] == code[e] and
// e' < e)}, the order select_small's K rounds of wave-wide max produce -- is
// counted by four threads over a quarter of the experts each, summed with two
// DPP steps.  The expert of rank r < K lands in LDS slot r; wave 0 then forms
// the routing weights as select_small does (same operations, same order).
// With one token every pair is its own group, so the groups are listed in
// rank order: group r = expert of rank r, one row (token 0), pair slot r --
// no sort, and nothing downstream depends on the groups' order.  The caller
// synchronises the block before reading the group tables.
template <class Load>
MKD_DEV void select_one(const RouterArgs& a, Load&& load) {
  constexpr int PER = 2;                   // E <= 128
  __shared__ __attribute__((aligned(16))) uint32_t code_s[128];
  __shared__ float key_s[128];
  __shared__ int sel_s[8];
  __shared__ float stat_s[2];              // max, 1 / sum of exp
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int E = a.E, K = a.K;
  const bool sigm = a.mode & 1, pre = a.mode & 2, norm = a.mode & 4, qwen = a.mode & 8;
  if (wv == 0) {
    float l[PER];
    load(0, l);
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      if (e < E) {
        if (a.logits_out) a.logits_out[e] = l[j];
      } else {
        l[j] = -INFINITY;
      }
      mx = fmaxf(mx, l[j]);
    }
    mx = wave_max(mx);
    float sum = 0.f, ex[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      ex[j] = (lane + 64 * j < E) ? expf(l[j] - mx) : 0.f;
      sum += ex[j];
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float key = (qwen || !pre) ? l[j] : (sigm ? 1.0f / (1.0f + expf(-l[j])) : ex[j] * inv);
      code_s[lane + 64 * j] = (lane + 64 * j < E) ? order_code(key) : 0u;   // padding ranks last
      key_s[lane + 64 * j] = key;
    }
    if (lane == 0) {
      stat_s[0] = mx;
      stat_s[1] = inv;
    }
  }
  __syncthreads();
  {
    // the quarter's 32 codes with eight 16-byte LDS reads issued together.
    // f outranks e when code_f > code_e, or code_f == code_e and f < e: one
    // unsigned compare against code_e - 1 below e and code_e from e on (every
    // finite or infinite key codes to >= 0x7fffff; padding codes are 0) -- a
    // select and a compare per code, no lane-mask logic.
    const int e = tid >> 2, qtr = tid & 3;
    int rank = 0;
    if (e < E) {
      const uint32_t ue = code_s[e];
      const uint32_t ue1 = ue ? ue - 1 : 0u;
      const int d = e - qtr * 32;          // codes i*4+j of the quarter below e: i*4+j < d
      const u32x4_t* cq = reinterpret_cast<const u32x4_t*>(code_s + qtr * 32);
      u32x4_t c[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = cq[i];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t thr = (i * 4 + j < d) ? ue1 : ue;
          rank += c[i][j] > thr ? 1 : 0;
        }
    }
    rank += __builtin_amdgcn_update_dpp(0, rank, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    rank += __builtin_amdgcn_update_dpp(0, rank, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    if (e < E && qtr == 0 && rank < K) sel_s[rank] = e;
  }
  __syncthreads();
  if (wv == 0) {
    const float mx = stat_s[0], inv = stat_s[1];
    const int my_e = lane < K ? sel_s[lane] : 0;
    const float my_key = lane < K ? key_s[my_e] : 0.f;
    const float k0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_key), 0));
    float pv;
    if (qwen) pv = rbf(expf(my_key - mx) * inv);
    else if (pre) pv = my_key;
    else if (sigm) pv = 1.0f / (1.0f + expf(-my_key));
    else pv = expf(my_key - k0);
    float w = pv;
    if (qwen || (pre && norm) || (!pre && !sigm)) {
      float s = 0.f;
      for (int k = 0; k < K; ++k)
        s += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), k));
      w = qwen ? rbf(pv * (1.0f / s)) : pv * (1.0f / s);
    }
    if (lane < K) {
      if (a.idx_out) a.idx_out[lane] = my_e;
      if (a.topk_out) a.topk_out[lane] = w;
      if (a.slot_w) a.slot_w[lane] = w;
      if (a.n_groups) {
        a.grp_expert[lane] = my_e;
        a.grp_count[lane] = 1;
        a.grp_offset[lane] = lane;
        a.pair_token[lane] = 0;
        a.pair_slot[lane] = lane;
      }
    }
    if (lane == 0 && a.n_groups) *a.n_groups = K;
  }
}

// One-token routing split in two for blocks that need their experts before the
// routing weights (flows whose selection key is the logit itself: Qwen's
// logit top-k, or the top-k on logits with a softmax over the top-k).
// select_one_experts: wave 0 loads the logits (kept in its registers, l) and
// stores their order codes and values to LDS; after one block barrier every
// expert's rank is counted as in select_one, and rank r < K goes straight into
// the group tables (group r = expert r of the ranking, one row, pair slot r) --
// no softmax statistics or weights on the way to the weight loads.  The caller
// synchronises the block (LDS) before reading the tables.
struct OneTokenSel {
  uint32_t code[128];
  float key[128];
  int ng, gexp[8], gcnt[8], goff[8], ptok[8], pslot[8];
  float w[8];
};

// `issue` (wave 0) issues the logit loads and `finish` (wave 0) forms l from
// them; between the two every wave passes one plain barrier (no memory fence,
// so wave 0's loads stay in flight) and runs `side` -- where the other waves
// can issue loads of their own that then queue behind the logits.
template <class Issue, class Finish, class Side>
MKD_DEV void select_one_experts(const RouterArgs& a, Issue&& issue, Finish&& finish, Side&& side,
                                OneTokenSel& s, float (&l)[2]) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int E = a.E, K = a.K;
  if (wv == 0) issue();
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  side();
  if (wv == 0) {
    finish(l);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = lane + 64 * j;
      if (e < E) {
        if (a.logits_out) a.logits_out[e] = l[j];
      } else {
        l[j] = -INFINITY;
      }
      s.code[e] = e < E ? order_code(l[j]) : 0u;   // padding ranks last
      s.key[e] = l[j];
    }
  }
  lds_barrier();   // the loads `side` issued stay in flight
  const int e = tid >> 2, qtr = tid & 3;
  int rank = 0;
  if (e < E) {
    const uint32_t ue = s.code[e];
    const uint32_t ue1 = ue ? ue - 1 : 0u;
    const int d = e - qtr * 32;
    const u32x4_t* cq = reinterpret_cast<const u32x4_t*>(s.code + qtr * 32);
    u32x4_t c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = cq[i];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t thr = (i * 4 + j < d) ? ue1 : ue;
        rank += c[i][j] > thr ? 1 : 0;
      }
  }
  rank += __builtin_amdgcn_update_dpp(0, rank, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  rank += __builtin_amdgcn_update_dpp(0, rank, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  if (e < E && qtr == 0 && rank < K) {
    s.gexp[rank] = e;
    s.gcnt[rank] = 1;
    s.goff[rank] = rank;
    s.ptok[rank] = 0;
    s.pslot[rank] = rank;
  }
  if (tid == 0) s.ng = K;
}

// select_one_weights: wave 0, after the caller's barrier that follows
// select_one_experts, forms the routing weights of the K slots (select_one's
// formulas: Qwen softmax value at the expert -> bf16 -> bf16 L1 renormalisation,
// or the softmax over the top-k logits) into s.w, and writes the optional
// global outputs (idx_out, topk_out, slot_w).
MKD_DEV void select_one_weights(const RouterArgs& a, OneTokenSel& s, const float (&l)[2]) {
  const int lane = threadIdx.x & 63;
  const int K = a.K;
  const bool qwen = a.mode & 8;
  float mx = fmaxf(l[0], l[1]);
  mx = wave_max(mx);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) sum += (lane + 64 * j < a.E) ? expf(l[j] - mx) : 0.f;
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  const int my_e = lane < K ? s.gexp[lane] : 0;
  const float my_key = lane < K ? s.key[my_e] : 0.f;
  const float k0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_key), 0));
  const float pv = qwen ? rbf(expf(my_key - mx) * inv) : expf(my_key - k0);
  float t = 0.f;
  for (int k = 0; k < K; ++k)
    t += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv), k));
  const float w = qwen ? rbf(pv * (1.0f / t)) : pv * (1.0f / t);
  if (lane < K) {
    s.w[lane] = w;
    if (a.idx_out) a.idx_out[lane] = my_e;
    if (a.topk_out) a.topk_out[lane] = w;
    if (a.slot_w) a.slot_w[lane] = w;
  }
}

}  // namespace mkd
