// Cross-wave reduction and epilogue shared by the weight-streaming GEMMs
// (bf16 frag layout in gemm.hip, MX formats in mx.hip).
//
// Every wave holds RB x TN 16x16 fp32 tiles (MFMA D layout: lane l has rows
// 4*(l/16)+i, token column l%16) for its K slice.  The partial tiles are summed
// through LDS in wave order (deterministic), then one epilogue per token tile
// writes the block's output columns:
//   EPI_F32         fp32 store (split-K partial kblk at y + kblk*part_stride)
//   EPI_BF16        bf16 store
//   EPI_RESID_BF16  bf16(residual + bf16(acc))
//   EPI_SWIGLU_BF16 gate rows in tile 0, up rows in tile RB-1 -> bf16(act(g)*u)
//   EPI_SCALE_F32   fp32 acc * pair_scale[row]
#pragma once
#include "common.h"
#include "mkd_internal.h"
#include "coherent.h"
#include "poll_word.h"

namespace mkd {

// g * sigmoid(z) = g / (1 + e^-z) with the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: about 1 ulp each, so a few fp32 ulps in all -- far
// below the bf16 rounding that follows); e^-z -> inf gives g * 0, e^-z -> 0
// gives g.  The accurate expf and IEEE division cost ~40 instructions per
// element, which dominated the epilogue of the MFMA-regime expert GEMM.
MKD_DEV float gated_sigmoid(float g, float z) {
  const float e = __builtin_amdgcn_exp2f(-z * 1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// One gated activation value from the gate and up projections (fp32, bias
// already added).  Qwen rounding: g, u -> bf16, silu(g) -> bf16, product;
// otherwise clamps, then act(g) * u with act (kAct*) = silu, swish(alpha),
// GELU (erf) or GELU's tanh approximation.
MKD_DEV float swiglu_value(const GemmArgs& a, float gv, float uv) {
  if (a.round_qwen) {
    const float g = rbf(gv), u = rbf(uv);
    return rbf(gated_sigmoid(g, g)) * u;
  }
  const float g = fmaxf(fminf(gv, a.gate_hi), a.gate_lo);
  const float u = fmaxf(fminf(uv, a.up_hi), a.up_lo);
  if (a.act == kActGelu) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f)) * u;
  if (a.act == kActGeluTanh)
    return 0.5f * g * (1.0f + tanhf(0.79788456080286536f * (g + 0.044715f * g * g * g))) * u;
  const float z = a.act == kActSwish ? a.alpha * g : g;
  return gated_sigmoid(g, z) * u;
}

template <int RB, int TN, int EPI, bool COH = false>
MKD_DEV void gemm_finish(const GemmArgs& a, f32x4_t (&acc)[RB][TN], int lane, int wave, int rbase,
                         int group, int t0, int base, const int (&xrow)[TN], int kblk) {
  // ---- cross-wave reduction (fixed order) ----
  extern __shared__ float red[];        // [nsplit][RB*TN*4][64]
  constexpr int NR = RB * TN * 4;
  const int nsplit = blockDim.x >> 6;
  if (nsplit > 1) {
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[(wave * NR + (r * TN + tn) * 4 + i) * 64 + lane] = acc[r][tn][i];
    __syncthreads();
  }

  // Each wave finalises the (tn) tiles with tn % nsplit == wave.
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    if (tn % nsplit != wave) continue;
    float v[RB][4];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (nsplit > 1) {
          float s = 0.f;
          for (int q = 0; q < nsplit; ++q) s += red[(q * NR + (r * TN + tn) * 4 + i) * 64 + lane];
          v[r][i] = s;
        } else {
          v[r][i] = acc[r][tn][i];
        }
      }
    if (xrow[tn] < 0) continue;
    const int c = t0 + tn * 16 + (lane & 15);
    const int orow = a.grp_expert ? (a.pair_out_row ? a.pair_out_row[base + c] : base + c)
                                  : c;
    const int n0 = rbase * 16 + (lane >> 4) * 4;   // logical output column of v[.][0]
    const int ncol = RB == 2 ? a.N / 2 : a.N;       // logical output width
    const int nv = min(4, ncol - n0);               // valid columns of this lane
    if (nv <= 0) continue;
    const bool vec = (nv == 4) && ((a.ldy & 3) == 0);
    if (a.bias && kblk == 0) {   // split-K: the bias goes into partial 0 only
      const uint16_t* bp = a.bias + (a.grp_expert ? (long long)a.grp_expert[group] * a.bias_group_stride : 0);
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (i < nv) v[r][i] += bf2f(bp[(r ? ncol : 0) + n0 + i]);
    }
    float o[4];
    if (EPI == EPI_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = v[0][i];
    } else if (EPI == EPI_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = v[0][i];
    } else if (EPI == EPI_RESID_BF16) {
      // o = bf16(acc); out = bf16(res + o)   (projection then bf16 residual add)
      const uint16_t* rp = a.residual + (long long)orow * a.ldy + n0;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (i < nv) ? bf2f(rp[i]) + rbf(v[0][i]) : 0.f;
    } else if (EPI == EPI_SWIGLU_BF16) {
      // gate rows in v[0], up rows in v[1]; the product is stored as bf16
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = swiglu_value(a, v[0][i], v[RB - 1][i]);
    } else if (EPI == EPI_SCALE_F32) {
      const float sc = a.pair_scale ? a.pair_scale[orow] : 1.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = v[0][i] * sc;
    }
    if (EPI == EPI_F32 || EPI == EPI_SCALE_F32) {
      float* y = reinterpret_cast<float*>(a.y) + kblk * a.part_stride + (long long)orow * a.ldy + n0;
      if (vec) {
        *reinterpret_cast<f32x4_t*>(y) = f32x4_t{o[0], o[1], o[2], o[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) if (i < nv) y[i] = o[i];
      }
    } else {
      uint16_t* y = reinterpret_cast<uint16_t*>(a.y) + (long long)orow * a.ldy + n0;
      if (COH) {   // read back by other blocks of this launch, which may poll these
        // words for the empty marker: a NaN whose bits equal it is stored as the quiet NaN
        const __amdgpu_buffer_rsrc_t yr = coh_rsrc(a.y);
        const int off = (int)(((long long)orow * a.ldy + n0) * 2);
        if (vec) {
          coh_st8(yr, off, poll_safe_bf16x2(pack2bf(o[0], o[1])), poll_safe_bf16x2(pack2bf(o[2], o[3])));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (i < nv) coh_st2(yr, off + 2 * i, (uint16_t)poll_safe_bf16x2(f2bf(o[i])));
        }
      } else if (vec) {
        *reinterpret_cast<uint2*>(y) = uint2{pack2bf(o[0], o[1]), pack2bf(o[2], o[3])};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) if (i < nv) y[i] = (uint16_t)f2bf(o[i]);
      }
    }
  }
}

}  // namespace mkd
