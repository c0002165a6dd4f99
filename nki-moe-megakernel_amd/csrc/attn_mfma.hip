// Split-K GQA decode attention on MFMA (gfx950).
//
// Grid (chunk, kv_head, sequence); block = 4 waves; wave w owns TPW tiles of 16
// consecutive KV positions.  Per 16-position tile:
//   S = K_tile . q^T   v_mfma_f32_16x16x32_bf16, A = 16 K rows read straight
//                      from HBM (each lane 4 x 16 B of one row), B = the gqa
//                      query heads of this kv head (16 columns, >= gqa zero).
//                      D lane l holds S[pos 4*(l/16)+i][head l%16].
//   softmax numerator  p = exp(s - m_head) with the wave's per-head max.
//   O += P . V        v_mfma_f32_16x16x16_bf16: the S layout above IS the
//                      A layout of this MFMA (row = head l%16, k = positions
//                      4*(l/16)+i), so P never leaves registers.  B = V tile
//                      [16 pos][16 d], staged through LDS (rows padded to
//                      D+8 elements: conflict-free 2-byte transposed reads).
// The 4 wave partials are merged in LDS; the block writes (max, sum,
// unnormalised O) per (sequence, head, chunk) for attn_combine_kernel.
// Positions: t < n_prior[b] read the cache, t == n_prior[b] is the new token
// (staged by qk_prep), t > n_prior[b] are masked.  With round_qwen the score
// is bf16(bf16(q.k) * scale) as in the reference's fused kernel.
#include "common.h"
#include "mkd_internal.h"

namespace mkd {

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4v;

MKD_DEV f32x4_t mfma16x16x16(uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4v, a),
                                                   __builtin_bit_cast(bf16x4v, b), c, 0, 0, 0);
}

template <int D, int GQA, int TPW>
__global__ void __launch_bounds__(256) attn_mfma_kernel(AttnArgs a) {
  constexpr int VS = D + 8;                   // padded LDS row stride (elements)
  constexpr int NK = D / 32;                  // QK MFMAs per tile (k = 32)
  constexpr int NDT = D / 16;                 // PV d-tiles
  __shared__ uint16_t v_s[4][16 * VS];        // one V tile per wave
  __shared__ float m_s[4][16], l_s[4][16];
  __shared__ float o_s[4][GQA][D];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int n = min(max(a.n_prior[b], 0), a.S_max);
  const int total = n + 1;
  const int chunk0 = c * (4 * TPW * 16);
  if (chunk0 >= total) return;                // whole block: uniform exit

  const uint16_t* kbase = a.k_cache + b * a.cache_b_stride + g * a.cache_h_stride;
  const uint16_t* vbase = a.v_cache + b * a.cache_b_stride + g * a.cache_h_stride;
  const uint16_t* knew = a.kv_new + (((long long)b * 2 + 0) * a.nkv + g) * D;
  const uint16_t* vnew = a.kv_new + (((long long)b * 2 + 1) * a.nkv + g) * D;

  // q fragments (B operand): lane l -> head l%16, d = (l/16)*(D/4) + kk*8 .. +8
  const int hcol = lane & 15;
  const int dq = (lane >> 4) * (D / 4);
  u32x4_t qf[NK];
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    if (hcol < GQA)
      qf[kk] = ld16(a.q_out + ((long long)b * a.nq + g * GQA + hcol) * D + dq + kk * 8);
    else
      qf[kk] = u32x4_t{0, 0, 0, 0};
  }

  // ---- scores for the wave's tiles ----
  float s[TPW][4];
  const int wbase = chunk0 + w * TPW * 16;
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int t = wbase + tt * 16 + (lane & 15);  // A row owned by this lane
    const uint16_t* kr = (t < n) ? kbase + (long long)t * D : knew;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      u32x4_t kf = (t <= n) ? ld16(kr + dq + kk * 8) : u32x4_t{0, 0, 0, 0};
      acc = mfma16x16x32(kf, qf[kk], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tp = wbase + tt * 16 + (lane >> 4) * 4 + i;   // position of acc[i]
      float sc = a.round_qwen ? rbf(rbf(acc[i]) * a.scale) : acc[i] * a.scale;
      bool ok = tp < total && hcol < GQA;
      if (ok && a.mask) {
        const int mt = (tp < n) ? tp : (a.mask_s_ctx - 1);
        ok = a.mask[((long long)mt * a.B + b) * a.nq + g * GQA + hcol] != 0;
      }
      s[tt][i] = ok ? sc : -INFINITY;
    }
  }
  // per-head max over the wave's positions (lanes sharing l%16)
  float m = -INFINITY;
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, s[tt][i]);
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float lsum = 0.f;
  uint2 pa[TPW];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = (m == -INFINITY) ? 0.f : expf(s[tt][i] - m);
      lsum += p[i];
    }
    pa[tt] = uint2{pack2bf(p[0], p[1]), pack2bf(p[2], p[3])};
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // ---- O = P V ----
  f32x4_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint16_t* vt = v_s[w];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    // stage V rows of the tile: lane -> row l%16, D/4 elements at (l/16)*(D/4)
    const int t = wbase + tt * 16 + (lane & 15);
    const uint16_t* vr = (t < n) ? vbase + (long long)t * D : vnew;
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      const u32x4_t v = (t <= n) ? ld16(vr + dq + j * 8) : u32x4_t{0, 0, 0, 0};
      *reinterpret_cast<u32x4_t*>(vt + (lane & 15) * VS + dq + j * 8) = v;
    }
    wave_lds_sync();                          // V tile visible to the whole wave
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int col = dt * 16 + (lane & 15);
      const int r0 = (lane >> 4) * 4;
      const uint32_t e0 = vt[(r0 + 0) * VS + col], e1 = vt[(r0 + 1) * VS + col];
      const uint32_t e2 = vt[(r0 + 2) * VS + col], e3 = vt[(r0 + 3) * VS + col];
      o[dt] = mfma16x16x16(pa[tt], uint2{e0 | (e1 << 16), e2 | (e3 << 16)}, o[dt]);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the 4 waves ----
  if (lane < 16) { m_s[w][lane] = m; l_s[w][lane] = lsum; }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = (lane >> 4) * 4 + i;
      if (h < GQA) o_s[w][h][dt * 16 + (lane & 15)] = o[dt][i];
    }
  __syncthreads();
  for (int idx = threadIdx.x; idx < GQA * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < 4; ++q) M = fmaxf(M, m_s[q][h]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float f = (m_s[q][h] == -INFINITY) ? 0.f : expf(m_s[q][h] - M);
      L += l_s[q][h] * f;
      O += o_s[q][h][d] * f;
    }
    const int hq = g * GQA + h;
    a.part_o[(((long long)b * a.nq + hq) * a.n_chunks + c) * D + d] = O;
    if (d == 0) {
      float* ml = a.part_ml + (((long long)b * a.nq + hq) * a.n_chunks + c) * 2;
      ml[0] = M;
      ml[1] = L;
    }
  }
}

template <int D, int GQA, int TPW>
static hipError_t launch_attn(const AttnArgs& a, hipStream_t s) {
  return timed_launch(attn_mfma_kernel<D, GQA, TPW>, dim3(a.n_chunks, a.nkv, a.B), dim3(256), 0, s,
                      a);
}

template <int D, int GQA>
static hipError_t launch_tpw(const AttnArgs& a, hipStream_t s) {
  const int chunk = a.chunk;
  if (chunk == 64) return launch_attn<D, GQA, 1>(a, s);
  if (chunk == 128) return launch_attn<D, GQA, 2>(a, s);
  if (chunk == 256) return launch_attn<D, GQA, 4>(a, s);
  return hipErrorInvalidValue;
}

int attn_chunk_for(int B, int nkv, int S_max) {
  // positions per block: enough blocks to cover the CUs several times over
  for (int chunk : {256, 128}) {
    const long long blocks = (long long)B * nkv * ((S_max + 1 + chunk - 1) / chunk);
    if (blocks >= 1024) return chunk;
  }
  return 64;
}

hipError_t attn_decode_launch(const AttnArgs& a, hipStream_t s) {
  const int gqa = a.nq / a.nkv;
  if (a.d == 128) {
    switch (gqa) {
      case 1: return launch_tpw<128, 1>(a, s);
      case 2: return launch_tpw<128, 2>(a, s);
      case 4: return launch_tpw<128, 4>(a, s);
      case 8: return launch_tpw<128, 8>(a, s);
      case 16: return launch_tpw<128, 16>(a, s);
    }
  } else if (a.d == 64) {
    switch (gqa) {
      case 1: return launch_tpw<64, 1>(a, s);
      case 2: return launch_tpw<64, 2>(a, s);
      case 4: return launch_tpw<64, 4>(a, s);
      case 8: return launch_tpw<64, 8>(a, s);
      case 16: return launch_tpw<64, 16>(a, s);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace mkd
