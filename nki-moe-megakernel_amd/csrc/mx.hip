// MX (OCP Microscaling v1.0) expert path for gfx950: MXFP8 / MXFP4 weights,
// MXFP8 activations, v_mfma_scale_f32_16x16x128_f8f6f4.
//
// Quantisation (mx_quantize_kernel): blocks of 32 consecutive elements along K
// share one E8M0 scale X = 2^(floor(log2 amax) - emax_elem) (byte = exponent
// + 127, clamped to [0, 254]; an all-zero block gets byte 0); each element is
// v / X rounded to nearest-even in the element format and saturated to its
// largest finite magnitude (E4M3 448, E2M1 6).  This is the OCP rule; the
// reference's nisa.quantize_mx (selective_expert_mx_impl.py:143-149,
// down_projection_mx_shard_H.py:74-79) is a Neuron instruction whose rounding
// is not in its sources.
//
// MX frag layout.  One scaled MFMA takes a 16 x 128 A tile; lane l = 16*q + r
// supplies row r and, for 8-bit elements, k in [16q, 16q+16) and
// [64+16q, 64+16q+16) (two 16-byte halves), for 4-bit elements k in
// [32q, 32q+32) (one 16-byte run, low nibble first); the scale byte a lane
// supplies is the E8M0 of row r, k-block q (k in [32q, 32q+32)).  The B
// operand (16 token columns x 128 k) uses the same per-lane layout.  Packed:
//   codes [G][NB][KB][2 halves][64 lanes][16 B] (e4m3) | [G][NB][KB][64 lanes][16 B] (e2m1)
//   KB = K_pad/128; an e4m3 fragment's two 16-byte halves per lane lie 1 KiB
//   apart, so each of its two loads reads 1 KiB contiguous (with the halves
//   adjacent per lane, each load touched twice the cache lines it used and the
//   address unit ran ~80 % busy)
//   scales[G][NB][ceil(KB/4)][64 lanes][4 B]  byte i = fragment 4*kb4 + i
// Rows past N and k past K are zero codes with scale byte 0.  K_pad (mx_kpad)
// is K rounded up to 128, or to 512 when that leaves no even split of the
// fragments over <= 8 waves.
//
// The GEMM is the weight-streaming scheme of gemm.hip with 128-k fragments:
// waves split K, partial tiles meet in LDS (fixed order), shared epilogues
// (gemm_epi.h).  Activations arrive pre-quantised (MXFP8, row-major codes,
// one scale byte per 32).
#include "common.h"
#include "gemm_epi.h"
#include "mkd_internal.h"
#include "mx_codec.h"

namespace mkd {

typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8_t;

// ---------------------------------------------------------------------------
// Quantisation: one thread per 32-element block.  codes row stride: K_pad bytes
// (e4m3) or K_pad/2 bytes (e2m1, two per byte, low nibble first); scales row
// stride K_pad/32.  Blocks at k >= K are written as zeros.
// ---------------------------------------------------------------------------
template <int FMT, bool XF32>
__global__ void mx_quantize_kernel(const void* __restrict__ x, int rows, int K, int ldx,
                                   uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                   int K_pad) {
  const int nblk = K_pad / 32;
  const long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x;
  if (idx >= (long long)rows * nblk) return;
  const int r = (int)(idx / nblk), b = (int)(idx % nblk);
  float v[32];
  if (b * 32 < K) {
    if (XF32) {
      const float* p = static_cast<const float*>(x) + (long long)r * ldx + b * 32;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f32x4_t t = *reinterpret_cast<const f32x4_t*>(p + 4 * j);
        v[4 * j] = t[0]; v[4 * j + 1] = t[1]; v[4 * j + 2] = t[2]; v[4 * j + 3] = t[3];
      }
    } else {
      const uint16_t* p = static_cast<const uint16_t*>(x) + (long long)r * ldx + b * 32;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t t = ld16(p + 8 * j);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          v[8 * j + 2 * h] = bf_lo(t[h]);
          v[8 * j + 2 * h + 1] = bf_hi(t[h]);
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = 0.f;
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const uint32_t sb = mx_scale_byte<FMT>(amax);
  const int sh = 127 - (int)sb;
  if (FMT == MX_E4M3) {
    u32x4_t o[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t d = 0;
#pragma unroll
      for (int h = 0; h < 4; ++h) d |= mx_encode<FMT>(ldexpf(v[4 * j + h], sh)) << (8 * h);
      o[j >> 2][j & 3] = d;
    }
    uint8_t* c = codes + (long long)r * K_pad + b * 32;
    st16(c, o[0]);
    st16(c + 16, o[1]);
  } else {
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t d = 0;
#pragma unroll
      for (int h = 0; h < 8; ++h) d |= mx_encode<FMT>(ldexpf(v[8 * j + h], sh)) << (4 * h);
      o[j] = d;
    }
    st16(codes + (long long)r * (K_pad / 2) + b * 16, o);
  }
  scales[(long long)r * nblk + b] = (uint8_t)sb;
}

// ---------------------------------------------------------------------------
// Packing into MX frag layout.  Source codes [G][N][K] (e4m3, one byte each) or
// [G][N][K/2] (e2m1 pairs), k contiguous, strides in bytes; source scales
// [G][N][K/32].  interleave_half as in pack_frag_kernel (gate/up row blocks).
// ---------------------------------------------------------------------------
template <int FMT>
__global__ void mx_pack_kernel(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
                               uint8_t* __restrict__ dst, uint8_t* __restrict__ dst_s, int G, int N,
                               int K, int KB, long long gs, long long rs, long long sgs,
                               long long srs, int interleave_half) {
  constexpr int BPL = MxSpec<FMT>::BPL;
  const int KB4 = (KB + 3) / 4, NB = (N + 15) / 16;
  const long long total = (long long)G * NB * KB * 64;
  for (long long idx = blockIdx.x * (long long)blockDim.x + threadIdx.x; idx < total;
       idx += (long long)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    long long t = idx >> 6;
    const int kb = (int)(t % KB); t /= KB;
    const int nb = (int)(t % NB);
    const int g = (int)(t / NB);
    int row_block = nb;
    if (interleave_half > 0) {
      const int pair = nb >> 1;
      row_block = (nb & 1) ? (interleave_half / 16 + pair) : pair;
    }
    const int n = row_block * 16 + (lane & 15), q = lane >> 4;
    uint8_t out[BPL];
#pragma unroll
    for (int j = 0; j < BPL; ++j) out[j] = 0;
    if (n < N) {
      const uint8_t* src = codes + g * gs + n * rs;
      if (FMT == MX_E4M3) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int k0 = kb * 128 + h * 64 + 16 * q;   // 16-aligned, K % 32 == 0
          if (k0 < K)
#pragma unroll
            for (int j = 0; j < 16; ++j) out[16 * h + j] = src[k0 + j];
        }
      } else {
        const int k0 = kb * 128 + 32 * q;
        if (k0 < K)
#pragma unroll
          for (int j = 0; j < 16; ++j) out[j] = src[k0 / 2 + j];
      }
    }
    uint8_t* d = dst + (((long long)g * NB + nb) * KB + kb) * 64 * BPL + lane * 16;
#pragma unroll
    for (int j = 0; j < BPL; ++j) d[(j / 16) * 1024 + (j % 16)] = out[j];
    if ((kb & 3) == 0) {
      uint32_t sv = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int blk = (kb + i) * 4 + q;                // 32-wide block index along K
        if (n < N && kb + i < KB && blk * 32 < K)
          sv |= (uint32_t)scales[g * sgs + n * srs + blk] << (8 * i);
      }
      *reinterpret_cast<uint32_t*>(dst_s + ((((long long)g * NB + nb) * KB4 + (kb >> 2)) * 64 + lane) * 4) = sv;
    }
  }
}

// ---------------------------------------------------------------------------
// The MX GEMM (16 token columns per block, TN = 1).
// ---------------------------------------------------------------------------
// A fragment registers: 8 dwords for 8-bit elements, 4 for 4-bit ones (the
// MFMA reads only the low 4 dwords of a 4-bit operand).
// p: the lane's 16 bytes of the fragment's first half (the second half 1 KiB on)
template <int FMT>
struct WFrag {
  u32x4_t lo, hi;
  MKD_DEV void load(const uint8_t* p) {
    lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p + 1024));
  }
  MKD_DEV i32x8_t op() const {
    return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                   (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  }
};
template <>
struct WFrag<MX_E2M1> {
  u32x4_t lo;
  MKD_DEV void load(const uint8_t* p) {
    lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  }
  MKD_DEV i32x8_t op() const {
    return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], 0, 0, 0, 0};
  }
};

// B fragment: token row codes (e4m3) for fragment kb, this lane's two halves.
MKD_DEV i32x8_t load_xfrag(const uint8_t* xr, int kb, int q) {
  const u32x4_t lo = ld16(xr + kb * 128 + 16 * q);
  const u32x4_t hi = ld16(xr + kb * 128 + 64 + 16 * q);
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                 (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// B fragments of every row block: the weight codes and scales go out first,
// then the x codes and scales of the lane's token row (formed only now: in
// grouped mode the row comes from a routing table whose load may still be in
// flight), and only then the MFMAs.  Lanes of absent tokens (xrow < 0) read
// row 0 -- their output column is never written.  AL: the batch's B fragments
// start at a multiple of B (B divides 4), so they share one scale dword per
// row block, and with B == 2 their two x-scale dwords are one 8-byte load --
// the kernels issue ~20 % fewer loads per weight byte (the texture-address unit
// was ~80 % busy at bs = 32).
template <int RB, int FMT, int B, bool AL = false>
MKD_DEV void mx_batch(const uint8_t* const (&wrow)[RB], const uint8_t* const (&srow)[RB],
                      int xrow, const GemmArgs& a, int kb0, int f, int q, f32x4_t (&acc)[RB][1]) {
  constexpr int BPL = MxSpec<FMT>::BPL;
  static_assert(!AL || 4 % B == 0, "aligned batches lie within a group of 4 fragments");
  WFrag<FMT> wf[RB][B];
  uint32_t ws[RB][B];
  if constexpr (AL) {
    const int kbf = kb0 + f;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int u = 0; u < B; ++u) wf[r][u].load(wrow[r] + (long long)(f + u) * 64 * BPL);
      const uint32_t sd = *reinterpret_cast<const uint32_t*>(srow[r] + (kbf >> 2) * 256);
#pragma unroll
      for (int u = 0; u < B; ++u) ws[r][u] = sd >> (8 * ((kbf + u) & 3));
    }
  } else {
#pragma unroll
    for (int u = 0; u < B; ++u)
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int kb = kb0 + f + u;
        wf[r][u].load(wrow[r] + (long long)(f + u) * 64 * BPL);
        ws[r][u] = *reinterpret_cast<const uint32_t*>(srow[r] + (kb >> 2) * 256) >> (8 * (kb & 3));
      }
  }
  __builtin_amdgcn_sched_barrier(0);
  int xr_i = xrow;
  asm volatile("" : "+v"(xr_i));         // formed here, not hoisted out of the k loop
  const long long row = xr_i >= 0 ? xr_i : 0;
  const uint8_t* xr = reinterpret_cast<const uint8_t*>(a.x) + row * a.ldx;
  const uint8_t* xs = a.x_scale + row * a.ldxs;
  i32x8_t xf[B];
  uint32_t xsc[B];
#pragma unroll
  for (int u = 0; u < B; ++u) xf[u] = load_xfrag(xr, kb0 + f + u, q);
  if constexpr (AL && B == 2) {   // 8-byte aligned: ldxs and 4 * (kb0 + f) are multiples of 8
    const uint2 xd = *reinterpret_cast<const uint2*>(xs + (kb0 + f) * 4);
    xsc[0] = xd.x >> (8 * q);
    xsc[1] = xd.y >> (8 * q);
  } else {
#pragma unroll
    for (int u = 0; u < B; ++u) xsc[u] = *reinterpret_cast<const uint32_t*>(xs + (kb0 + f + u) * 4) >> (8 * q);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < B; ++u)
#pragma unroll
    for (int r = 0; r < RB; ++r)
      acc[r][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
          wf[r][u].op(), xf[u], acc[r][0], MxSpec<FMT>::HW, MxSpec<MX_E4M3>::HW, 0,
          (int)(ws[r][u] & 0xffu), 0, (int)(xsc[u] & 0xffu));
}

// Fragments per batch of one wave's loads for R streamed row tiles: as many as
// fit 64 VGPRs (R x U weight fragments with their scale words, U x-code
// fragments), rounded down to 8 / 4 / 2 / 1.  Small batches keep the kernel
// near 100 VGPRs, i.e. 4 waves per SIMD: measured at bs=32 (MXFP8 gate/up
// 84.6 -> 69.5 us, down 52.6 -> 38.5 us against 128-VGPR batches), the number
// of waves in flight matters more than the bytes each has in flight.
template <int FMT, int R>
constexpr int mx_batch_frags() {
  constexpr int per = 8 + (MxSpec<FMT>::BPL / 4 + 1) * R;
  constexpr int u = 64 / per;
  return u >= 8 ? 8 : u >= 4 ? 4 : u >= 2 ? 2 : 1;
}

// RT output tiles (16*RB rows each) per block: every wave streams the
// fragments of all RT tiles of its K slice, so a block moves RT times the bytes
// of a one-tile block for the same reduction and launch cost.
template <int RB, int FMT, int EPI, int RT>
__global__ void __launch_bounds__(512) gemm_mx_kernel(GemmArgs a) {
  constexpr int BPL = MxSpec<FMT>::BPL;
  constexpr int R = RB * RT;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile0 = blockIdx.x * RT;
  const int n_tiles = (a.N + 16 * RB - 1) / (16 * RB);
  const int group = blockIdx.y;
  const int kg = a.kgrid > 1 ? a.kgrid : 1;
  const int kblk = blockIdx.z % kg;

  int count, base;
  const uint8_t* w = reinterpret_cast<const uint8_t*>(a.w);
  const uint8_t* wsc = a.w_scale;
  if (a.grp_expert) {
    // table entries read with the group count: one memory round trip
    const int ng = *a.n_groups;
    count = a.grp_count[group];
    base = a.grp_offset[group];
    const int ex = a.grp_expert[group];
    asm volatile("" ::"s"(ng), "s"(count), "s"(base), "s"(ex));   // no sinking past the exit
    if (group >= ng) return;
    w += (long long)ex * a.w_group_stride;
    wsc += (long long)ex * a.w_scale_group_stride;
  } else {
    count = a.T;
    base = 0;
  }
  // a.t_loop: the block walks every token tile of its group
  for (int ttile = blockIdx.z / kg;; ++ttile) {
  const int t0 = ttile * 16;
  if (t0 >= count) return;
  if (ttile > (int)blockIdx.z / kg) __syncthreads();   // the previous tile's reduction buffer is free
  int xrow[1];
  {
    const int c = t0 + (lane & 15);
    xrow[0] = c < count ? (a.pair_row ? a.pair_row[base + c] : base + c) : -1;
  }

  const int KB = a.K / 128, KB4 = (KB + 3) / 4;
  const int NF = a.KW / 128;
  const int kb0 = (kblk * (int)(blockDim.x >> 6) + wave) * NF;
  const int q = lane >> 4;

  f32x4_t acc[R][1];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // row tile t of the block, row block r of the tile -> stream row R*t + r;
  // tiles past the last (a ragged final block) re-read the last one and are
  // not stored
  const uint8_t* wrow[R];
  const uint8_t* srow[R];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const long long rb = (long long)min(tile0 + t, n_tiles - 1) * RB + r;
      wrow[t * RB + r] = w + (rb * KB + kb0) * 64 * BPL + lane * 16;
      srow[t * RB + r] = wsc + (rb * KB4 * 64 + lane) * 4;
    }
  constexpr int U = mx_batch_frags<FMT, R>();
  // every batch starts at a multiple of its size when the wave's slice does
  // (kb0 = a multiple of NF; batches of U, then 4 / 2 / 1, each starting at a
  // multiple of the sizes before it), and U <= 4 divides 4: shared scale words
  // (the x-scale pair needs ldxs % 8 == 0 too)
  constexpr bool UAL = U <= 4;
  if (UAL && NF % U == 0 && a.ldxs % 8 == 0) {
    int f = 0;
    for (; f + U <= NF; f += U) mx_batch<R, FMT, U, UAL>(wrow, srow, xrow[0], a, kb0, f, q, acc);
    if constexpr (U > 2)
      if (f + 2 <= NF) { mx_batch<R, FMT, 2, UAL>(wrow, srow, xrow[0], a, kb0, f, q, acc); f += 2; }
    if constexpr (U > 1)
      if (f < NF) mx_batch<R, FMT, 1, UAL>(wrow, srow, xrow[0], a, kb0, f, q, acc);
  } else {
    int f = 0;
    for (; f + U <= NF; f += U) mx_batch<R, FMT, U>(wrow, srow, xrow[0], a, kb0, f, q, acc);
    if constexpr (U > 4)
      if (f + 4 <= NF) { mx_batch<R, FMT, 4>(wrow, srow, xrow[0], a, kb0, f, q, acc); f += 4; }
    if constexpr (U > 2)
      if (f + 2 <= NF) { mx_batch<R, FMT, 2>(wrow, srow, xrow[0], a, kb0, f, q, acc); f += 2; }
    if constexpr (U > 1)
      if (f < NF) mx_batch<R, FMT, 1>(wrow, srow, xrow[0], a, kb0, f, q, acc);
  }

#pragma unroll
  for (int t = 0; t < RT; ++t) {
    if (tile0 + t >= n_tiles) break;          // block-uniform
    if (t > 0) __syncthreads();               // the previous tile's reduction buffer is free
    f32x4_t at[RB][1];
#pragma unroll
    for (int r = 0; r < RB; ++r) at[r][0] = acc[t * RB + r][0];
    gemm_finish<RB, 1, EPI>(a, at, lane, wave, tile0 + t, group, t0, base, xrow, kblk);
  }
  if (!a.t_loop) return;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
hipError_t mx_quantize_launch(const void* x, bool x_f32, int rows, int K, int ldx, int fmt,
                              uint8_t* codes, uint8_t* scales, int K_pad, hipStream_t s) {
  if (rows <= 0 || K <= 0 || K % 32 || K_pad < K || K_pad % 128) return hipErrorInvalidValue;
  const long long n = (long long)rows * (K_pad / 32);
  const int threads = 256;
  const unsigned blocks = (unsigned)((n + threads - 1) / threads);
#define MKD_Q(F, X) hipLaunchKernelGGL((mx_quantize_kernel<F, X>), dim3(blocks), dim3(threads), 0, s, x, rows, K, ldx, codes, scales, K_pad)
  if (fmt == MX_E4M3) { if (x_f32) MKD_Q(MX_E4M3, true); else MKD_Q(MX_E4M3, false); }
  else if (fmt == MX_E2M1) { if (x_f32) MKD_Q(MX_E2M1, true); else MKD_Q(MX_E2M1, false); }
  else return hipErrorInvalidValue;
#undef MKD_Q
  return hipGetLastError();
}

long long mx_packed_code_bytes(int G, int N, int K, int fmt) {
  const long long KB = mx_kpad(K) / 128, NB = (N + 15) / 16;
  return (long long)G * NB * KB * 64 * (fmt == MX_E4M3 ? 32 : 16);
}

long long mx_packed_scale_bytes(int G, int N, int K) {
  const long long KB = mx_kpad(K) / 128, NB = (N + 15) / 16;
  return (long long)G * NB * ((KB + 3) / 4) * 64 * 4;
}

hipError_t mx_pack_launch(const uint8_t* codes, const uint8_t* scales, uint8_t* dst,
                          uint8_t* dst_scales, int G, int N, int K, long long g_stride,
                          long long row_stride, long long s_g_stride, long long s_row_stride,
                          int fmt, int interleave_half, hipStream_t s) {
  if (G <= 0 || N <= 0 || K <= 0 || K % 32) return hipErrorInvalidValue;
  // every scale dword is written by the first fragment of its 4-fragment group
  const int KB = mx_kpad(K) / 128;
  const long long total = (long long)G * ((N + 15) / 16) * KB * 64;
  const int threads = 256;
  long long blocks = (total + threads - 1) / threads;
  if (blocks > 65535LL * 16) blocks = 65535LL * 16;
#define MKD_P(F) hipLaunchKernelGGL(mx_pack_kernel<F>, dim3((unsigned)blocks), dim3(threads), 0, s, codes, scales, dst, dst_scales, G, N, K, KB, g_stride, row_stride, s_g_stride, s_row_stride, interleave_half)
  if (fmt == MX_E4M3) MKD_P(MX_E4M3);
  else if (fmt == MX_E2M1) MKD_P(MX_E2M1);
  else return hipErrorInvalidValue;
#undef MKD_P
  return hipGetLastError();
}

int choose_kw_mx(int K_pad) {
  // per-wave K slice (multiple of 128) splitting K_pad over <= 8 waves: 4 or 8
  // waves per block first, so that whole blocks fill a CU's 16 wave slots
  // (measured: MXFP4 gate/up at K_pad 3072, 6-wave blocks 83.8 us, 4-wave
  // blocks 58.1 us), then slices of 2^i fragments (whole batches)
  for (int nw : {4, 8})
    if (K_pad % (128 * nw) == 0) return K_pad / nw;
  for (int kw : {512, 256, 1024, 128, 384, 768, 1536, 2048})
    if (K_pad % kw == 0 && K_pad / kw <= 8) return kw;
  return -1;
}

int mx_kpad(int K) {
  const int p = (K + 127) / 128 * 128;
  return choose_kw_mx(p) > 0 ? p : (K + 511) / 512 * 512;
}

template <int RB, int FMT, int EPI, int RT>
static hipError_t launch_mx(const GemmArgs& a, int n_tiles, int groups, int ttiles, hipStream_t s) {
  const int nsplit = a.K / a.KW;
  if (a.KW <= 0 || a.KW % 128 || nsplit < 1 || nsplit > 8 || nsplit * a.KW != a.K)
    return hipErrorInvalidValue;
  dim3 grid((n_tiles + RT - 1) / RT, groups, ttiles);
  dim3 block(64 * nsplit);
  const size_t lds = nsplit > 1 ? (size_t)nsplit * RB * 4 * 64 * sizeof(float) : 0;
  return timed_launch(gemm_mx_kernel<RB, FMT, EPI, RT>, grid, block, lds, s, a);
}

// Output tiles per block.  Measured at bs=32: one tile everywhere except the
// MXFP4 down projection (a 1 KiB fragment per row tile), where four tiles per
// block took 42.8 -> 39.3 us (GPT-OSS shape); for MXFP8 and for gate/up, more
// tiles per block cost occupancy and were slower.
int mx_tiles_per_block(int RB, int fmt, int n_tiles, int groups) {
  constexpr long long kMxMinBlocks = 1024;
  if (RB == 1 && fmt == MX_E2M1 && (long long)((n_tiles + 3) / 4) * groups >= kMxMinBlocks) return 4;
  return 1;
}

hipError_t gemm_mx_launch(GemmArgs a, int fmt, int epi, int groups_max, int max_tokens_per_group,
                          hipStream_t s) {
  if (a.kgrid > 1) return hipErrorInvalidValue;
  const int RB = (epi == EPI_SWIGLU_BF16) ? 2 : 1;
  const int n_tiles = (a.N + 16 * RB - 1) / (16 * RB);
  int ttiles = (max_tokens_per_group + 15) / 16;
  const int groups = a.grp_expert ? groups_max : 1;
  if (a.grp_expert && ttiles > 1) {   // grouped: one tile per block, walking the group (a.t_loop)
    a.t_loop = 1;
    ttiles = 1;
  }
  const int rt = mx_tiles_per_block(RB, fmt, n_tiles, groups);
#define MKD_M(RB_, F_, E_)                                                                 \
  if (RB == RB_ && fmt == F_ && epi == E_) {                                               \
    if constexpr (RB_ == 1)                                                                \
      if (rt == 4) return launch_mx<RB_, F_, E_, 4>(a, n_tiles, groups, ttiles, s);        \
    return launch_mx<RB_, F_, E_, 1>(a, n_tiles, groups, ttiles, s);                       \
  }
  MKD_M(2, MX_E4M3, EPI_SWIGLU_BF16) MKD_M(2, MX_E2M1, EPI_SWIGLU_BF16)
  MKD_M(1, MX_E4M3, EPI_SCALE_F32) MKD_M(1, MX_E2M1, EPI_SCALE_F32)
  MKD_M(1, MX_E4M3, EPI_F32) MKD_M(1, MX_E2M1, EPI_F32)
#undef MKD_M
  return hipErrorInvalidValue;
}

}  // namespace mkd
