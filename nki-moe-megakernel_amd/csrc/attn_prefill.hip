// Prefill attention: the T new tokens of one sequence (a context-encoding pass,
// attention_block_tkg's semantics per token: token b attends the cache rows
// 0 .. n_prior[b] - 1 and then itself, attention_block_tkg.py:1473-1685 with
// the new token's own k / v from its prepared heads) read each K / V row once
// per 16-token query tile, instead of once per token as the split-K decode
// kernel does.
//
// Block (query tile, kv group g, head slice): 16 consecutive tokens x up to 8
// of the group's GQA query heads, one wave per head.  Per 64-position step of the cache a wave forms
// S^T = K Q^T (v_mfma_f32_16x16x32_bf16: A = 16 cache rows, B = the 16 tokens'
// q; lane l holds positions 4(l/16) + i of token l % 16), the online softmax
// per token (running max and sum, the token's own row first), then O += P V
// with 16-position quarters paired on the 32-deep MFMA (A = P, rows the
// tokens; B = V, column l % 16 <-> d = 8 (l % 16) + dt).  The block stages each
// 64-position step of K and V in LDS (double-buffered: the next step's rows are
// loaded while the current one is computed), so a row is read from memory once
// per block rather than once per head.  Rounding follows the decode kernel:
// Qwen scores bf16(bf16(q.k) * scale), P rounded to bf16 for the MFMA, sums in
// fp32; the exponentials use the hardware exp2 (__expf: 184 -> 148 us per
// layer at 2048 tokens).  An optional sink logit joins the normaliser at the
// end.  Four waves per SIMD (two 8-wave blocks per CU, <= 128 VGPRs).
#include "common.h"
#include "mkd_internal.h"
#include "launch_rules.h"
#include "attn_common.h"
#include "coherent.h"

namespace mkd {

constexpr int kPfTok = 16;    // query tokens per block (the MFMA's 16 columns)
constexpr int kPfStep = 64;   // cache positions per step (four 16-row quarters)
constexpr int kPfLd = 136;    // LDS row stride in bf16 (256 B + 16 B: rows land on different banks)

template <int GQA, int HPB = (GQA < 8 ? GQA : 8)>
__global__ void __launch_bounds__(64 * HPB) __attribute__((amdgpu_waves_per_eu(HPB >= 8 ? 4 : 1)))
attn_prefill_kernel(AttnArgs a) {
  constexpr int D = 128, NK = D / 32, NDT = D / 16, NT = 64 * HPB;
  constexpr int CH = kPfStep * D / 8;                 // 16-byte chunks of one K (or V) step
  constexpr int CPT = (CH + NT - 1) / NT;             // of them per thread
  __shared__ __attribute__((aligned(16))) uint16_t k_s[2][kPfStep * kPfLd];
  __shared__ __attribute__((aligned(16))) uint16_t v_s[2][kPfStep * kPfLd];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int tl = lane & 15, q4 = lane >> 4;
  const int nqt = (a.B + kPfTok - 1) / kPfTok;
  // Work units (query tile, kv group, head slice), longest tiles first: unit u
  // is tile nqt - 1 - u / nsets of set u % nsets.  Block L takes unit L, except
  // where the whole grid is resident at two blocks per CU: there block L >= CUs,
  // which shares a CU with block L - CUs, takes unit total - 1 - (L - CUs), so
  // the two tiles on a CU have complementary lengths (2048 tokens: 65.7k ->
  // 70.6k tokens/s for the pass; with two tiles of the same length on every
  // CU, the CUs of the longest tiles set the launch's length).
  const int nsets = gridDim.y * gridDim.z, total = nqt * nsets;
  const int L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const int u = prefill_unit_rule(L, total, a.pf_pair);
  const int t0 = (nqt - 1 - u / nsets) * kPfTok;
  const int set = u % nsets;
  const int g = set % gridDim.y, hg = (set / gridDim.y) * HPB + w, h = g * GQA + hg;   // head in group / overall
  const int tok = t0 + tl;
  const bool live = tok < a.B;
  const int tokc = live ? tok : a.B - 1;                 // in-range address for absent tokens
  const long long hstride = (long long)(GQA + 2) * D;
  const uint16_t* prep_t = a.prep + ((long long)tokc * a.nkv + g) * hstride;

  // ---- the token's q (B operand, natural k order: d = 32 kk + 8 q4 .. + 8)
  // and its own row's score ----
  u32x4_t qf[NK], kown[NK];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    qf[kk] = live ? ld16(prep_t + hg * D + 32 * kk + 8 * q4) : u32x4_t{0u, 0u, 0u, 0u};
    kown[kk] = ld16(prep_t + GQA * D + 32 * kk + 8 * q4);
  }
  const int n_b = live ? prior_len(a, tok) : 0;
  // the tile's largest prior length (every wave forms it: the step loop and
  // its barriers are the same in all of them)
  int nmax = n_b;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) nmax = max(nmax, __shfl_xor(nmax, o, 64));
  nmax = __builtin_amdgcn_readfirstlane(nmax);
  float dot = 0.f;
#pragma unroll
  for (int kk = 0; kk < NK; ++kk)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      dot += bf_lo(qf[kk][e]) * bf_lo(kown[kk][e]) + bf_hi(qf[kk][e]) * bf_hi(kown[kk][e]);
  dot += __shfl_xor(dot, 16, 64);
  dot += __shfl_xor(dot, 32, 64);
  const float sdiag = a.round_qwen ? rbf(rbf(dot) * a.scale) : dot * a.scale;

  // ---- O starts as the own row's v (weight exp(0) = 1): rows are the tokens
  // 4 q4 + i, column tl of d-tile dt is d = 8 tl + dt ----
  f32x4_t o[NDT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ti = min(t0 + 4 * q4 + i, a.B - 1);
    const u32x4_t v = ld16(a.prep + ((long long)ti * a.nkv + g) * hstride + (GQA + 1) * D + 8 * tl);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[2 * e][i] = bf_lo(v[e]);
      o[2 * e + 1][i] = bf_hi(v[e]);
    }
  }
  float m_run = sdiag, l_run = 1.f;

  // ---- the cache rows, kPfStep positions per step, staged in LDS by the
  // whole block (each row read from memory once per block), the next step's
  // rows loaded while the current step is computed ----
  u32x4_t kreg[CPT], vreg[CPT];
  auto load_step = [&](int p0) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * NT;
      const int row = min(p0 + ch / 16, nmax - 1);     // clamped: rows past the tile re-read the last
      const uint16_t* kr = kv_row<D>(a, a.k_cache, 0, g, row);
      const uint16_t* vr = kv_row<D>(a, a.v_cache, 0, g, row);
      kreg[c] = (ch < CH && kr) ? ld16(kr + (ch % 16) * 8) : u32x4_t{0u, 0u, 0u, 0u};
      vreg[c] = (ch < CH && vr) ? ld16(vr + (ch % 16) * 8) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = threadIdx.x + c * NT;
      if (ch < CH) {
        st16(&k_s[buf][(ch / 16) * kPfLd + (ch % 16) * 8], kreg[c]);
        st16(&v_s[buf][(ch / 16) * kPfLd + (ch % 16) * 8], vreg[c]);
      }
    }
  };
  // (A copy of this step without the per-score masking for the steps below
  // every token's prior length, and skipping the O rescale when no maximum
  // moved, cut the VALU count but spilled: 69k -> 58k tokens/s at 2048 tokens.)
  auto compute_step = [&](int p0, int buf) {
    const uint16_t* ks = k_s[buf];
    const uint16_t* vs = v_s[buf];
    float sc[4][4];
    float mt = -INFINITY;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
        acc = mfma16x16x32(ld16(ks + (16 * s + tl) * kPfLd + 32 * kk + 8 * q4), qf[kk], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = a.round_qwen ? rbf(rbf(acc[i]) * a.scale) : acc[i] * a.scale;
        const int pos = p0 + 16 * s + 4 * q4 + i;
        sc[s][i] = pos < n_b ? v : -INFINITY;
        mt = fmaxf(mt, sc[s][i]);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);   // finite: m_run starts at the own row's score
    const float alpha = __expf(m_run - m_new);
    float ls = 0.f;
    uint2 pa[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __expf(sc[s][i] - m_new);     // a masked score (-inf) gives exactly 0
        ls += p[i];
      }
      pa[s] = uint2{pack2bf(p[0], p[1]), pack2bf(p[2], p[3])};
    }
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    l_run = l_run * alpha + ls;
    m_run = m_new;
    // O rows are tokens 4 q4 + i: their factors from the lanes holding them
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * q4 + i, 64);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= al[i];
    // P.V, the quarters in pairs on the 32-deep MFMA: lane group q4's k slots
    // are positions 4 q4 .. 4 q4 + 3 of the even quarter, then of the odd one,
    // in the P operand and in the V operand alike; the B operand's 16-bit
    // halves gathered from two V rows by one byte permute per dword
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) {
      u32x4_t vq[2][4];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) vq[s][j] = ld16(vs + (16 * (2 * sp + s) + 4 * q4 + j) * kPfLd + 8 * tl);
      const u32x4_t pp = {pa[2 * sp].x, pa[2 * sp].y, pa[2 * sp + 1].x, pa[2 * sp + 1].y};
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int e = dt >> 1;
        // low halves: bytes 0-1 of the first row, 0-1 of the second (selector
        // 0x05040100); high halves: bytes 2-3 of each (0x07060302)
        const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
        uint2 bo[2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
          bo[s] = uint2{__builtin_amdgcn_perm(vq[s][1][e], vq[s][0][e], sel),
                        __builtin_amdgcn_perm(vq[s][3][e], vq[s][2][e], sel)};
        o[dt] = mfma16x16x32(pp, u32x4_t{bo[0].x, bo[0].y, bo[1].x, bo[1].y}, o[dt]);
      }
    }
  };
  if (nmax > 0) {
    load_step(0);
    store_step(0);
    lds_barrier();
    int buf = 0;
    for (int p0 = 0; p0 < nmax; p0 += kPfStep) {
      const bool more = p0 + kPfStep < nmax;        // block-uniform
      if (more) load_step(p0 + kPfStep);
      compute_step(p0, buf);
      if (more) store_step(buf ^ 1);
      lds_barrier();                                 // the next buffer written, this one read
      buf ^= 1;
    }
  }
  // ---- sink logit, normalisation, bf16 rows ----
  if (a.sink) {
    const float sk = a.sink[h];
    const float m2 = fmaxf(m_run, sk);
    const float r = expf(m_run - m2);
    l_run = l_run * r + expf(sk - m2);
    float rr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rr[i] = __shfl(r, 4 * q4 + i, 64);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= rr[i];
  }
  const float inv = 1.f / l_run;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float f = __shfl(inv, 4 * q4 + i, 64);
    const int ti = t0 + 4 * q4 + i;
    if (ti >= a.B) continue;
    u32x4_t out;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = pack2bf(o[2 * e][i] * f, o[2 * e + 1][i] * f);
    st16(a.attn_out + ((long long)ti * a.nq + h) * D + 8 * tl, out);
  }
}

bool attn_prefill_ok(const AttnArgs& a) {
  const int gqa = a.nkv > 0 ? a.nq / a.nkv : 0;
  return a.prefill && a.prep && a.d == 128 && gqa * a.nkv == a.nq &&
         (gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8 || gqa == 16) && !a.mask && a.window == 0 &&
         a.s_tkg <= 1 && !a.kv_fp8 && !a.k_transposed && a.B >= 1 && a.update_cache;
}

hipError_t attn_prefill_launch(const AttnArgs& a, int rope_mode, hipStream_t s) {
  if (!attn_prefill_ok(a)) return hipErrorInvalidValue;
  if (hipError_t e = attn_prep_write_launch(a, rope_mode, s)) return e;
  const int gqa = a.nq / a.nkv, hpb = gqa < 8 ? gqa : 8;
  const dim3 grid((a.B + kPfTok - 1) / kPfTok, a.nkv, gqa / hpb);
  // tile pairing for the 8-wave blocks (two per CU: 128 VGPRs, 68 KiB of LDS
  // each) when the whole grid is resident: workgroups go round-robin to the
  // XCDs and fill each XCD's CUs in order, so block L + CUs lands beside block L
  AttnArgs b = a;
  const long long total = (long long)grid.x * grid.y * grid.z;
  const int cus = device_cus();
  b.pf_pair = prefill_pair_rule(total, cus, hpb);
  switch (gqa) {
    case 1: return timed_launch(attn_prefill_kernel<1>, grid, dim3(64), 0, s, b);
    case 2: return timed_launch(attn_prefill_kernel<2>, grid, dim3(128), 0, s, b);
    case 4: return timed_launch(attn_prefill_kernel<4>, grid, dim3(256), 0, s, b);
    case 8: return timed_launch(attn_prefill_kernel<8>, grid, dim3(512), 0, s, b);
    case 16: return timed_launch(attn_prefill_kernel<16>, grid, dim3(512), 0, s, b);
  }
  return hipErrorInvalidValue;
}

}  // namespace mkd
