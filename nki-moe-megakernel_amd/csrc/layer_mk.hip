// Persistent decoder layer for small decode batches (B <= 4, Qwen3 flow):
// one launch per layer runs every stage of the layer of the reference's
// megakernel step (qwen_with_megakernel.py:414-531; the stage kernels
// rmsnorm_tkg.py, attention_block_tkg.py, router_topk.py, moe_tkg.py) on one
// block per CU, the stages separated by grid barriers instead of kernel
// boundaries:
//
//   P  every block: x -> rinv -> hn = bf16((x * rinv) * ln_in)       (LDS)
//   Q  QKV projection, split over all blocks                          -> partials
//   T  attention: units (sequence, kv head, 128-position chunk): the
//      q / k / v heads of the new token from the QKV partials (q / k
//      RMSNorm, RoPE, Qwen rounding), QK^T and PV on MFMA, the 8 waves'
//      partials merged; the chunk holding the new position writes the new
//      K / V rows into the cache                                      -> (m, l, O) per chunk
//   C  combine: one wave per (sequence, q head)                       -> attn_out (bf16)
//   O  output projection                                              -> partials
//   R  every block: r = bf16(x + bf16(o)), y = (r * ln_post) * rinv
//      (fp32, bf16 copy for the experts); router logits GEMV          -> partials
//   S  every block: top-k + expert groups (the router select body), so
//      every block knows the experts without another barrier
//   G  expert gate / up projections over the live expert groups      -> partials
//   D  every block forms act = silu(g) * u (Qwen rounding) for the groups
//      of its range, then the down projections                       -> partials
//   F  block slice of the hidden rows: x = bf16(r + bf16(sum_k w_k y_k))
//
// Stage-to-stage data crosses blocks through device-coherent buffer accesses
// (cache-policy bit sc1 on every store and load of the exchanged data), so a
// barrier needs no cache write-back or invalidate: each wave waits for its own
// stores (s_waitcnt vmcnt(0)), then one thread per block arrives on one of
// eight group counters (blockIdx % 8; the last arrival of a group bumps a top
// counter, the last group arrival releases eight per-group flags) and spins on
// its group's flag with a bounded spin (timeout -> error word, later barriers
// stop waiting, so the grid always drains).  Measured on MI355X: ~2 us per
// barrier with the exchange, against ~4.5 us for the agent-scope
// release / acquire fences alone.
//
// Split-K GEMV stages: the F = groups x row_blocks x k_blocks weight fragments
// (1 KiB frag-packed tiles, 16 rows x 32 k) are cut into nbp contiguous,
// equal ranges (one per block; nbp <= #CUs so that a 16-row unit spans at most
// 4 blocks), each cut again over the 8 waves.  A wave streams its fragments in
// batches of 8 (software pipelined; the first batch of the next stage is
// issued between a barrier's arrival and its wait), accumulating one MFMA
// tile per unit; the block sums its waves' tiles through LDS in wave order
// and writes one fp32 partial per unit; consumers add a unit's (<= 4)
// partials in block order.  Deterministic throughout.
#include "common.h"
#include "mkd_internal.h"
#include "attn_common.h"
#include "router_select.h"
#include "gemm_epi.h"

namespace mkd {

#ifndef MKD_LK_U
#define MKD_LK_U 8
#endif
namespace {
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kU = MKD_LK_U;            // fragments per load batch
constexpr int kMaxS = 4;               // partials per unit
constexpr int kCols = kLkMaxB;         // token columns stored per partial
constexpr int kChunk = 16 * kWaves;    // attention positions per unit
constexpr int kRowChunks = kLkMaxRowElems / (8 * kThreads);   // 8-element row chunks per thread
constexpr int kSc1 = 16;               // buffer cache-policy bit sc1 (device coherent)
constexpr unsigned kSpinLimit = 1u << 19;
typedef unsigned u32x4e __attribute__((ext_vector_type(4)));
}  // namespace

// Stage timestamps for tuning builds (-DMKD_LK_TRACE): thread 0 of every block
// records the wall clock at each stage boundary of the last launch.
#ifdef MKD_LK_TRACE
__device__ unsigned long long lk_trace[1024 * 32];
#define LK_STAMP(i) \
  do { if (threadIdx.x == 0) lk_trace[blockIdx.x * 32 + (i)] = wall_clock64(); } while (0)
extern "C" int mkd_debug_layer_trace(unsigned long long* host, int n) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(lk_trace), sizeof(unsigned long long) * n);
}
#else
#define LK_STAMP(i) do { } while (0)
#endif

// ---------------------------------------------------------------------------
// device-coherent accesses
MKD_DEV __amdgpu_buffer_rsrc_t dev_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, 0x7fffffff, 0x00020000);
}
MKD_DEV float dev_ldf(__amdgpu_buffer_rsrc_t r, int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kSc1));
}
MKD_DEV f32x4_t dev_ld4f(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
}
MKD_DEV u32x4_t dev_ld16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
}
MKD_DEV void dev_st16(__amdgpu_buffer_rsrc_t r, int off, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4e, v), r, off, 0, kSc1);
}
MKD_DEV void dev_st16u(__amdgpu_buffer_rsrc_t r, int off, u32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4e, v), r, off, 0, kSc1);
}
MKD_DEV void dev_st4(__amdgpu_buffer_rsrc_t r, int off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kSc1);
}
MKD_DEV void dev_st2(__amdgpu_buffer_rsrc_t r, int off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kSc1);
}
// Reads of stage outputs (partials, attention chunks, attn_out): device
// coherent, like the barrier flags -- every stage buffer is rewritten by the
// next layer within the same launch, so an L2 copy of one of its lines could be
// stale.
constexpr int kXch = kSc1;
MKD_DEV float xch_ldf(__amdgpu_buffer_rsrc_t r, int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kXch));
}
MKD_DEV f32x4_t xch_ld4f(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kXch));
}
MKD_DEV u32x4_t xch_ld16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kXch));
}
MKD_DEV u32x4_t ld_stream(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// ---------------------------------------------------------------------------
// grid barrier: block b stores the barrier's generation number into its own
// flag word bar[b] (after its stores have completed); waiters read all the
// flag words -- one 16-byte device-coherent load per lane covers 4 blocks,
// one instruction per poll for up to 256 blocks -- until every block's flag
// has reached the generation.  No atomics, so no same-address serialisation.
// bar[kLkMaxNB] is the error word (a spin that timed out).
MKD_DEV unsigned ag_load(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MKD_DEV void ag_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

MKD_DEV void grid_arrive(const LayerArgs& L, int k) {
  __builtin_amdgcn_s_waitcnt(0xF70);   // vmcnt(0): this wave's stores have completed
  __syncthreads();
  if (k == 3) LK_STAMP(22);
  if (threadIdx.x == 0) ag_store(L.bar + blockIdx.x, (unsigned)k + 1u);
  if (k == 3) LK_STAMP(23);
}

MKD_DEV void grid_wait(const LayerArgs& L, int k) {
  if (threadIdx.x < 64) {
    const unsigned gen = (unsigned)k + 1u;
    const int nb = gridDim.x, lane = threadIdx.x;
    const __amdgpu_buffer_rsrc_t r = dev_rsrc(L.bar);
    unsigned* err = L.bar + kLkMaxNB;
    if (ag_load(err) == 0u) {
      for (int c0 = 0; c0 < nb; c0 += 256) {     // 256 flags per poll instruction
        unsigned it = 0;
        while (true) {
          const int f = c0 + lane * 4;
          const u32x4_t v = dev_ld16(r, min(f, kLkMaxNB - 4) * 4);
          bool ok = true;
#pragma unroll
          for (int j = 0; j < 4; ++j) ok &= (f + j >= nb) || v[j] >= gen;
          if (__all(ok)) break;
          if (++it > kSpinLimit) {
            if (lane == 0) ag_store(err, 1u);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
    }
  }
  if (k == 3) LK_STAMP(24);
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Division by a block-uniform divisor 1 <= d < 2^20 for n < 2^31: q =
// (mulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d)
// + 1 (Granlund-Montgomery, "Division by invariant integers using
// multiplication", 1994).  m is formed in double precision: the numerator
// (< 2^52) is exact, and for d < 2^20 the quotient lies at least one ulp from
// an integer, so the rounded quotient floors to the exact one
// (tests/test_fdiv_magic.py checks every d < 2^20 against integer arithmetic)
// -- far cheaper than an emulated 64-bit integer division.
struct FDiv {
  uint32_t m, s, d;
};
MKD_DEV FDiv fdiv_make(uint32_t d) {
  const uint32_t s = d <= 1 ? 0u : 32u - (uint32_t)__builtin_clz(d - 1);
  const double num = 4294967296.0 * (double)((1u << s) - d);
  return FDiv{(uint32_t)floor(num / (double)d) + 1u, s, d};
}
MKD_DEV uint32_t fdiv(uint32_t n, const FDiv& f) { return (__umulhi(n, f.m) + n) >> f.s; }

// split-K partition: block b takes fragments [b fpb, min(F, (b + 1) fpb)),
// fpb = max(ceil(F / #CUs), ceil(KB / 3)) so that a unit of KB fragments
// spans at most 4 blocks; waves split the block range evenly.
struct GemvCtx {
  int F, fpb, nbp, KB, NRB, ng;
  int lo, hi;      // block range
  int wlo, whi;    // wave range
  int w0;          // first streaming wave (waves below it take no fragments)
  int span;        // fragments that must stay within 4 blocks (KB, or ng * KB)
  FDiv dfpb, dKB, dNRB, dFG, dNG, dspan;
};

// Range of wave q: the block range split evenly over waves w0 .. 7.
MKD_DEV void wave_range(const GemvCtx& c, int q, int& wlo, int& whi) {
  const int n = c.hi - c.lo, ns = kWaves - c.w0;
  const int qq = q - c.w0;
  wlo = qq < 0 ? c.lo : c.lo + n * qq / ns;
  whi = qq < 0 ? c.lo : c.lo + n * (qq + 1) / ns;
}

// w0 = 1 for a stage whose first batch is issued between a barrier's arrival
// and its wait: wave 0 (which spins on the barrier) then has no loads in
// flight, since a wave's vector loads complete in issue order.
// rbm: the down stage's order -- units (row block, group), groups fastest --
// with a row block's ng * KB fragments spread over at most 4 blocks.
MKD_DEV GemvCtx gemv_ctx(const LkGemv& p, int ngroups, int NB, int blk, int w, int w0,
                         bool rbm = false) {
  // inputs laundered through an opaque asm: the set-up is recomputed where it
  // is used rather than hoisted out of the layer loop and held in registers
  int KB = p.KB, NRB = p.NRB;
  asm volatile("" : "+s"(KB), "+s"(NRB), "+s"(ngroups), "+s"(NB));
  GemvCtx c;
  c.w0 = w0;
  c.KB = KB;
  c.NRB = NRB;
  c.ng = ngroups;
  c.F = ngroups * NRB * KB;
  c.span = rbm ? ngroups * KB : KB;
  c.fpb = lk_fpb(c.F, c.span, NB);
  c.nbp = (c.F + c.fpb - 1) / c.fpb;
  c.lo = (int)min((long long)c.F, (long long)blk * c.fpb);
  c.hi = min(c.F, c.lo + c.fpb);
  wave_range(c, w, c.wlo, c.whi);
  c.dfpb = fdiv_make(c.fpb);
  c.dKB = fdiv_make(KB);
  c.dNRB = fdiv_make(NRB);
  c.dFG = fdiv_make(NRB * KB);
  c.dNG = fdiv_make(ngroups);
  c.dspan = fdiv_make(c.span);
  return c;
}

// Weight fragments f0 .. f0 + kU - 1 of the wave's range (past its end: the
// first fragment of the matrix, discarded).  gexp: expert of group (null: dense).
template <bool RBM>
MKD_DEV void gemv_load(const LkGemv& p, const int* gexp, const GemvCtx& c, int f0,
                       u32x4_t (&buf)[kU], int lane) {
  if constexpr (!RBM) {
    const int FG = p.NRB * p.KB;
    int g = (int)fdiv((uint32_t)f0, c.dFG), rem = f0 - g * FG;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint16_t* src = p.w + lane * 8;
      if (f0 + u < c.whi) {
        const long long e = gexp ? gexp[g] : 0;
        src = p.w + e * p.gstride + ((long long)rem * 64 + lane) * 8;
      }
      buf[u] = ld_stream(src);
      if (++rem == FG) { rem = 0; ++g; }
    }
  } else {
    const int uu = (int)fdiv((uint32_t)f0, c.dKB);
    int kb = f0 - uu * p.KB;
    int rb = (int)fdiv((uint32_t)uu, c.dNG);
    int g = uu - rb * c.ng;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint16_t* src = p.w + lane * 8;
      if (f0 + u < c.whi)
        src = p.w + (long long)gexp[g] * p.gstride + ((long long)(rb * p.KB + kb) * 64 + lane) * 8;
      buf[u] = ld_stream(src);
      if (++kb == p.KB) {
        kb = 0;
        if (++g == c.ng) { g = 0; ++rb; }
      }
    }
  }
}

// B operand sources of the GEMV stages (lane: column l%16, k = kb*32 + 8*(l/16))
enum { XM_DENSE = 0, XM_F32 = 1, XM_GROUP = 2, XM_ACT = 3 };
struct XSrc {
  const uint16_t* rows;   // bf16 rows in LDS (DENSE, GROUP, ACT)
  const float* rows32;    // fp32 rows in LDS (F32)
  int ld;                 // row stride (elements)
  int ncol;               // dense columns
  const int* gcnt;        // GROUP / ACT: tokens of each group
  const int* goff;        // GROUP: first pair of each group
  const int* ptok;        // GROUP: token of each pair
};

// Row of the lane's column for group g (null: no such column -> zeros).
template <int XM>
MKD_DEV const void* x_row(const XSrc& x, int g, int lane) {
  const int col = lane & 15;
  if constexpr (XM == XM_DENSE) {
    return col < x.ncol ? x.rows + col * x.ld : nullptr;
  } else if constexpr (XM == XM_F32) {
    return col < x.ncol ? x.rows32 + col * x.ld : nullptr;
  } else if constexpr (XM == XM_GROUP) {
    return col < x.gcnt[g] ? x.rows + x.ptok[x.goff[g] + col] * x.ld : nullptr;
  } else {   // ACT: one row per pair position goff[g] + col
    return col < x.gcnt[g] ? x.rows + (x.goff[g] + col) * x.ld : nullptr;
  }
}

// B operand fragment at k of a row (bf16; fp32 rows as bf16 hi + lo).
template <int XM>
MKD_DEV void x_frag(const void* row, int k, u32x4_t& hi, u32x4_t& lo) {
  hi = u32x4_t{0, 0, 0, 0};
  lo = u32x4_t{0, 0, 0, 0};
  if (!row) return;
  if constexpr (XM == XM_F32) {
    const float* r = static_cast<const float*>(row) + k;
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(r);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(r + 4);
    const float y[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t h0 = f2bf(y[2 * j]), h1 = f2bf(y[2 * j + 1]);
      hi[j] = h0 | (h1 << 16);
      lo[j] = f2bf(y[2 * j] - bf2f(h0)) | (f2bf(y[2 * j + 1] - bf2f(h1)) << 16);
    }
  } else {
    hi = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(row) + k);
  }
}

// The wave's fragments: MFMA tiles per unit into red[w][slot] (slot = unit -
// the wave's first unit).  buf holds the first batch (already issued).
template <int XM, bool RBM = false>
MKD_DEV void gemv_run(const LkGemv& p, const int* gexp, const GemvCtx& c, u32x4_t (&buf)[kU],
                      const XSrc& x, f32x4_t* red, int lane, int w) {
  if (c.whi <= c.wlo) return;
  const int KB = p.KB, NRB = RBM ? c.ng : p.NRB;   // RBM: the group cycles fastest
  const int ufirst = (int)fdiv((uint32_t)c.wlo, c.dKB);
  int uu = ufirst, kb = c.wlo - ufirst * KB;
  int g, urem;
  if constexpr (RBM) {
    urem = (int)fdiv((uint32_t)uu, c.dNG);   // row block
    g = uu - urem * c.ng;
  } else {
    g = (int)fdiv((uint32_t)uu, c.dNRB);
    urem = uu - g * NRB;
  }
  const void* row = x_row<XM>(x, g, lane);
  const int koff = (lane >> 4) * 8;
  int cur = uu;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int f0 = c.wlo; f0 < c.whi; f0 += kU) {
    u32x4_t nxt[kU];
    const bool more = f0 + kU < c.whi;
    if (more) gemv_load<RBM>(p, gexp, c, f0 + kU, nxt, lane);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (f0 + u >= c.whi) break;
      if (uu != cur) {
        red[(w * p.LW + (cur - ufirst)) * 64 + lane] = acc;
        acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
        cur = uu;
      }
      u32x4_t hi, lo;
      x_frag<XM>(row, kb * 32 + koff, hi, lo);
      acc = mfma16x16x32(buf[u], hi, acc);
      if constexpr (XM == XM_F32) acc = mfma16x16x32(buf[u], lo, acc);
      if (++kb == KB) {
        kb = 0;
        ++uu;
        if constexpr (RBM) {
          if (++g == c.ng) { g = 0; ++urem; }
          if (f0 + u + 1 < c.whi) row = x_row<XM>(x, g, lane);
        } else if (++urem == NRB) {
          urem = 0;
          ++g;
          if (f0 + u + 1 < c.whi) row = x_row<XM>(x, g, lane);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < kU; ++u) buf[u] = nxt[u];
    }
  }
  red[(w * p.LW + (cur - ufirst)) * 64 + lane] = acc;
}

// Block partial per unit: the waves' tiles in wave order; lanes of live
// columns store rows 4*(l/16).. of column l%16.  gcnt: columns per group
// (null: ncol for every unit).
MKD_DEV void gemv_finish(const LkGemv& p, const GemvCtx& c, const f32x4_t* red, const int* gcnt,
                         int ncol, int blk, int lane, int w) {
  __syncthreads();
  if (c.hi > c.lo) {
    const int ub0 = (int)fdiv((uint32_t)c.lo, c.dKB), ub1 = (int)fdiv((uint32_t)(c.hi - 1), c.dKB);
    const __amdgpu_buffer_rsrc_t r = dev_rsrc(p.part);
    for (int lu = w; lu <= ub1 - ub0; lu += kWaves) {
      const int u = ub0 + lu;
      f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < kWaves; ++q) {
        int qlo, qhi;
        wave_range(c, q, qlo, qhi);
        if (qhi <= qlo) continue;
        const int q0 = (int)fdiv((uint32_t)qlo, c.dKB), q1 = (int)fdiv((uint32_t)(qhi - 1), c.dKB);
        if (q0 <= u && u <= q1) s += red[(q * p.LW + (u - q0)) * 64 + lane];
      }
      const int cols = gcnt ? gcnt[fdiv((uint32_t)u, c.dNRB)] : ncol;
      const int col = lane & 15;
      if (col < cols)
        dev_st16(r, ((((blk * p.LB + lu) * kCols + col) * 16) + (lane >> 4) * 4) * 4, s);
    }
  }
  __syncthreads();
}

// Down stage (units (row block rb, group g), groups fastest): per row block of
// the block range, the waves' tiles of each of its units are summed in wave
// order, each column scaled by its (token, slot) routing weight and added to
// that token's rows, units in group order -> one partial per (block, row block,
// token): rows of the weighted expert sum sum_k w_k y_k (moe_tkg.py:151-170).
struct LkSel;
MKD_DEV void gemv_finish_dn(const LkGemv& p, const GemvCtx& c, const f32x4_t* red, LkSel* sel,
                            int B, int blk, int lane, int w);

// Sum of unit u's block partials at column col, rows r0..r0+3 (or row r0):
// the unit's first block b0 holds it at its local index u - first unit of b0,
// every later block (up to 3) as its local unit 0.
MKD_DEV void part_loc(const LkGemv& p, const GemvCtx& c, int u, int& b0, int& b1, int& lu0) {
  const uint32_t f0 = (uint32_t)(u * p.KB);
  b0 = (int)fdiv(f0, c.dfpb);
  b1 = (int)fdiv(f0 + p.KB - 1, c.dfpb);
  lu0 = u - (int)fdiv((uint32_t)(b0 * c.fpb), c.dKB);
}
MKD_DEV f32x4_t part_sum4(const LkGemv& p, const GemvCtx& c, int u, int col, int r0) {
  int b0, b1, lu0;
  part_loc(p, c, u, b0, b1, lu0);
  const __amdgpu_buffer_rsrc_t r = dev_rsrc(p.part);
  f32x4_t v[kMaxS];
#pragma unroll
  for (int s = 0; s < kMaxS; ++s) {
    const int bb = min(b0 + s, b1);
    const int lu = bb == b0 ? lu0 : 0;
    v[s] = xch_ld4f(r, (((bb * p.LB + lu) * kCols + col) * 16 + r0) * 4);
  }
  f32x4_t sum = v[0];
#pragma unroll
  for (int s = 1; s < kMaxS; ++s)
    if (b0 + s <= b1) sum += v[s];
  return sum;
}
MKD_DEV float part_sum1(const LkGemv& p, const GemvCtx& c, int u, int col, int r) {
  int b0, b1, lu0;
  part_loc(p, c, u, b0, b1, lu0);
  const __amdgpu_buffer_rsrc_t rs = dev_rsrc(p.part);
  float v[kMaxS];
#pragma unroll
  for (int s = 0; s < kMaxS; ++s) {
    const int bb = min(b0 + s, b1);
    const int lu = bb == b0 ? lu0 : 0;
    v[s] = xch_ldf(rs, (((bb * p.LB + lu) * kCols + col) * 16 + r) * 4);
  }
  float sum = v[0];
#pragma unroll
  for (int s = 1; s < kMaxS; ++s)
    if (b0 + s <= b1) sum += v[s];
  return sum;
}

// ---------------------------------------------------------------------------
// selection results shared by the stages after S (LDS)
struct LkSel {
  int ng;
  int gexp[kLkMaxB * 8], gcnt[kLkMaxB * 8], goff[kLkMaxB * 8];
  int ptok[kLkMaxB * 8], pslot[kLkMaxB * 8];
  int pg[kLkMaxB * 8], pj[kLkMaxB * 8];
  float slot_w[kLkMaxB * 8];
  float red[kWaves * kLkMaxB];
  float dacc[kWaves][kLkMaxB * 16];   // down stage: per-wave (token, row) sums
  int pgrp[kLkMaxB * 8];              // group of each pair position
};

static_assert(sizeof(LkSel) <= kLkSelBytes, "selection results exceed their LDS carve");

MKD_DEV void gemv_finish_dn(const LkGemv& p, const GemvCtx& c, const f32x4_t* red, LkSel* sel,
                            int B, int blk, int lane, int w) {
  __syncthreads();
  if (c.hi > c.lo) {
    const int ng = c.ng;
    const int ub0 = (int)fdiv((uint32_t)c.lo, c.dKB), ub1 = (int)fdiv((uint32_t)(c.hi - 1), c.dKB);
    const int rb0 = (int)fdiv((uint32_t)ub0, c.dNG), rb1 = (int)fdiv((uint32_t)ub1, c.dNG);
    const __amdgpu_buffer_rsrc_t r = dev_rsrc(p.part);
    float* acc = sel->dacc[w];
    for (int ri = w; ri <= rb1 - rb0; ri += kWaves) {
      const int rb = rb0 + ri;
      acc[lane] = 0.f;                       // kLkMaxB * 16 == 64 entries
      wave_lds_sync();
      const int u0 = max(ub0, rb * ng), u1 = min(ub1, rb * ng + ng - 1);
      for (int u = u0; u <= u1; ++u) {
        f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
          int qlo, qhi;
          wave_range(c, q, qlo, qhi);
          if (qhi <= qlo) continue;
          const int q0 = (int)fdiv((uint32_t)qlo, c.dKB), q1 = (int)fdiv((uint32_t)(qhi - 1), c.dKB);
          if (q0 <= u && u <= q1) s += red[(q * p.LW + (u - q0)) * 64 + lane];
        }
        const int g = u - rb * ng, j = lane & 15;
        if (j < sel->gcnt[g]) {
          const int pq = sel->goff[g] + j;
          const int t = sel->ptok[pq];
          const float wt = sel->slot_w[sel->pslot[pq]];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t * 16 + (lane >> 4) * 4 + i] += s[i] * wt;
        }
        wave_lds_sync();
      }
      if (lane < B * 4) {
        const int t = lane >> 2, r0 = (lane & 3) * 4;
        dev_st16(r, (((blk * p.LB + ri) * kCols + t) * 16 + r0) * 4,
                 f32x4_t{acc[t * 16 + r0], acc[t * 16 + r0 + 1], acc[t * 16 + r0 + 2], acc[t * 16 + r0 + 3]});
      }
      wave_lds_sync();
    }
  }
  __syncthreads();
}

// Per-token sums of squares of the block's 512 threads: ss[t] per thread in,
// full sums out (fixed order).
MKD_DEV void block_sums(float (&ss)[kLkMaxB], int B, LkSel* sel, int lane, int w) {
#pragma unroll
  for (int t = 0; t < kLkMaxB; ++t) {
    if (t >= B) break;
    const float v = wave_sum(ss[t]);
    if (lane == 0) sel->red[w * kLkMaxB + t] = v;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < kLkMaxB; ++t) {
    if (t >= B) break;
    float s = 0.f;
    for (int q = 0; q < kWaves; ++q) s += sel->red[q * kLkMaxB + t];
    ss[t] = s;
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// attention stage: unit (sequence b, kv head g, chunk c of kChunk positions)
// Prior positions of sequence b and cache row addressing: the rules of
// prior_len / kv_row (attn_common.h) for caches without a window, on the
// launch arguments directly.
MKD_DEV int lk_prior_len(const LayerArgs& L, int b) { return min(max(L.pos[b], 0), L.S_max); }
template <int D>
MKD_DEV const uint16_t* lk_kv_row(const LayerArgs& L, const uint16_t* cache, int b, int g, int t) {
  if (!L.block_table) return cache + b * L.cache_b_stride + g * L.cache_h_stride + (long long)t * D;
  const int bk = L.block_table[(long long)b * L.tbl_stride + t / L.blk_len];
  if ((unsigned)bk >= (unsigned)L.num_blocks) return nullptr;
  return cache + (((long long)bk * L.blk_len + t % L.blk_len) * L.nkv + g) * D;
}
template <int D>
struct AttnRows {
  u32x4_t k[D / 32];          // K row of the wave's tile (A operand)
  uint32_t v[4][D / 32];      // four V row segments (PV B operand)
};

template <int D>
MKD_DEV void attn_load(const LayerArgs& L, const LkLayer& ly, int b, int g, int c, int lane, int w,
                       AttnRows<D>& R) {
  constexpr int NK = D / 32, VW = D / 32;
  const int n = lk_prior_len(L, b);
  const int tile0 = c * kChunk + w * 16;
  const int dq = (lane >> 4) * (D / 4), vc = (lane & 15) * (D / 16);
  const int tk = tile0 + (lane & 15);
  const uint16_t* kr = tk < n ? lk_kv_row<D>(L, ly.k_cache, b, g, tk) : nullptr;
  const uint16_t* vp[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = tile0 + (lane >> 4) * 4 + j;
    vp[j] = t < n ? lk_kv_row<D>(L, ly.v_cache, b, g, t) : nullptr;
  }
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) R.k[kk] = kr ? ld16(kr + dq + kk * 8) : u32x4_t{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (VW == 4) {
      const u32x4_t v = vp[j] ? ld16(vp[j] + vc) : u32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) R.v[j][e] = v[e];
    } else {
      const uint2 v = vp[j] ? *reinterpret_cast<const uint2*>(vp[j] + vc) : uint2{0, 0};
      R.v[j][0] = v.x;
      R.v[j][1] = v.y;
    }
  }
}

template <int D>
MKD_DEV void attn_unit(const LayerArgs& L, const LkLayer& ly, const AttnArgs& aa, const GemvCtx& cq,
                       int b, int g, int c, AttnRows<D>& R, char* lds, int lane, int w) {
  constexpr int NK = D / 32, NDT = D / 16, VW = D / 32, HD = D / 2;
  const int gqa = L.gqa;
  uint16_t* q_s = reinterpret_cast<uint16_t*>(lds);                 // [16][D]
  uint16_t* kn_s = q_s + 16 * D;                                    // [D]
  uint16_t* vn_s = kn_s + D;                                        // [D]
  float* m_s = reinterpret_cast<float*>(vn_s + D);                  // [8][16]
  float* l_s = m_s + kWaves * 16;                                   // [8][16]
  float* o_s = l_s + kWaves * 16;                                   // [8][gqa][D]
  const int n = lk_prior_len(L, b), total = n + 1;
  const int tile0 = c * kChunk + w * 16;

  // ---- the new token's heads: wave w takes heads w, w + 8, w + 16 of
  // [q heads of g | k of g | v of g] (gqa + 2 <= 18) from the QKV partials ----
  {
    constexpr int NR = 3;
    HeadPrep<D> hp[NR];
    int kinds[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int h = w + kWaves * r;
      kinds[r] = -1;
      if (h >= gqa + 2) continue;
      const int kind = h < gqa ? 0 : h - gqa + 1;
      const int head = h < gqa ? g * gqa + h : (kind == 1 ? L.nq + g : L.nq + L.nkv + g);
      kinds[r] = kind;
      const uint16_t* nw = kind == 0 ? ly.q_norm : (kind == 1 ? ly.k_norm : nullptr);
      HeadPrep<D>& q = hp[r];
      q.f32 = true;
      q.off0 = 0;
      q.has_nw = nw != nullptr;
      q.rope_tab = kind < 2;
      const int l = lane < HD ? lane : 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int i = l + e * HD;
        const int row = head * D + i;
        q.xr[e] = __float_as_uint(part_sum1(L.q, cq, row >> 4, b, row & 15));
        q.nr[e] = nw ? *reinterpret_cast<const uint32_t*>(nw + (i & ~1)) : 0;   // HeadPrep's dword
        q.cs[e] = L.cos[b * D + i];
        q.sn[e] = L.sin[b * D + i];
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (kinds[r] < 0) continue;
      const int h = w + kWaves * r;
      uint16_t* dst = h < gqa ? q_s + h * D : (kinds[r] == 1 ? kn_s : vn_s);
      hp[r].finish(aa, 1, kinds[r], dst, lane);
    }
  }
  __syncthreads();
  LK_STAMP(18);

  // ---- scores S = K q^T for the wave's 16 positions ----
  const int hcol = lane & 15;
  const int dq = (lane >> 4) * (D / 4), vc = (lane & 15) * (D / 16);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < NK; ++kk) {
    const u32x4_t qf = hcol < gqa ? *reinterpret_cast<const u32x4_t*>(q_s + hcol * D + dq + kk * 8)
                                  : u32x4_t{0, 0, 0, 0};
    u32x4_t kf = R.k[kk];
    if (tile0 + (lane & 15) == n) kf = *reinterpret_cast<const u32x4_t*>(kn_s + dq + kk * 8);
    acc = mfma16x16x32(kf, qf, acc);
  }
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tp = tile0 + (lane >> 4) * 4 + i;
    const float sc = rbf(rbf(acc[i]) * L.scale);    // Qwen rounding of the score
    s[i] = (tp < total && hcol < gqa) ? sc : -INFINITY;
  }
  float m = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float p[4], lsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = (m == -INFINITY) ? 0.f : expf(s[i] - m);
    lsum += p[i];
  }
  const uint2 pa = uint2{pack2bf(p[0], p[1]), pack2bf(p[2], p[3])};
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);

  // ---- O = P V (V rows: d labels permuted so each lane holds D/16
  // contiguous elements of its four position rows).  One 16-position tile per
  // wave, so the 16-deep MFMA: the 32-deep one would take a second tile's
  // positions for its other k half ----
  uint32_t v[4][VW];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool isnew = tile0 + (lane >> 4) * 4 + j == n;
#pragma unroll
    for (int e = 0; e < VW; ++e)
      v[j][e] = isnew ? *reinterpret_cast<const uint32_t*>(vn_s + vc + 2 * e) : R.v[j][e];
  }
  f32x4_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int e = dt >> 1;
    const uint2 bop = (dt & 1)
        ? uint2{(v[0][e] >> 16) | (v[1][e] & 0xffff0000u), (v[2][e] >> 16) | (v[3][e] & 0xffff0000u)}
        : uint2{(v[0][e] & 0xffffu) | (v[1][e] << 16), (v[2][e] & 0xffffu) | (v[3][e] << 16)};
    o[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
        __builtin_bit_cast(bf16x4_t, pa), __builtin_bit_cast(bf16x4_t, bop),
        f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  }

  // ---- merge the 8 waves: (max, sum, unnormalised O) per head ----
  if (lane < 16) {
    m_s[w * 16 + lane] = m;
    l_s[w * 16 + lane] = lsum;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = (lane >> 4) * 4 + i;
    if (h < gqa)
#pragma unroll
      for (int q = 0; q < NDT / 4; ++q)
        *reinterpret_cast<f32x4_t*>(o_s + (w * gqa + h) * D + vc + 4 * q) =
            f32x4_t{o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]};
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rpo = dev_rsrc(L.attn_po), rml = dev_rsrc(L.attn_ml);
  for (int idx = threadIdx.x; idx < gqa * D; idx += kThreads) {
    const int h = idx / D, d = idx - h * D;
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) M = fmaxf(M, m_s[q * 16 + h]);
    float Lt = 0.f, O = 0.f;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      const float f = (m_s[q * 16 + h] == -INFINITY) ? 0.f : expf(m_s[q * 16 + h] - M);
      Lt += l_s[q * 16 + h] * f;
      O += o_s[(q * gqa + h) * D + d] * f;
    }
    const long long slot = ((long long)b * L.nq + g * gqa + h) * L.nch_max + c;
    dev_st4(rpo, (int)((slot * D + d) * 4), __float_as_uint(O));
    if (d == 0) {
      dev_st4(rml, (int)(slot * 8), __float_as_uint(M));
      dev_st4(rml, (int)(slot * 8 + 4), __float_as_uint(Lt));
    }
  }
  // the chunk holding the new position writes its K / V rows into the cache
  // (no block of this launch reads that row): row pos[b] of a flat cache, or
  // the block-table slot of pos[b] (kv_write_row's rule without a window)
  if (n >= c * kChunk && n < (c + 1) * kChunk && threadIdx.x < D) {
    long long row = -1;
    const int p = L.pos[b];
    if (p >= 0 && p < L.S_max) {
      if (!L.block_table) {
        row = p;
      } else {
        const int bk = L.block_table[(long long)b * L.tbl_stride + p / L.blk_len];
        if ((unsigned)bk < (unsigned)L.num_blocks) row = (long long)bk * L.blk_len + p % L.blk_len;
      }
    }
    if (row >= 0) {
      const int d = threadIdx.x;
      const long long off = L.block_table ? (row * L.nkv + g) * D + d
                                          : b * L.cache_b_stride + g * L.cache_h_stride + row * D + d;
      ly.k_cache[off] = kn_s[d];
      ly.v_cache[off] = vn_s[d];
    }
  }
  __syncthreads();
}

// Combine of the chunks of (sequence b, q head h), one block: wave w takes
// chunks w, w + 8, ... in batches of 4 (one memory round trip for up to 32
// chunks) with online rescaling; the 8 wave results merge in LDS in wave
// order; bf16 output.
template <int D>
MKD_DEV void combine_block(const LayerArgs& L, int b, int h, char* lds, int lane, int w) {
  constexpr int EL = D / 64, U = 4;
  float* m_s = reinterpret_cast<float*>(lds);     // [8]
  float* l_s = m_s + kWaves;                      // [8]
  float* a_s = l_s + kWaves;                      // [8][D]
  const int n = lk_prior_len(L, b);
  const int nch = (n + 1 + kChunk - 1) / kChunk;
  const long long base = ((long long)b * L.nq + h) * L.nch_max;
  const __amdgpu_buffer_rsrc_t rpo = dev_rsrc(L.attn_po), rml = dev_rsrc(L.attn_ml);
  float m = -INFINITY, Ls = 0.f, acc[EL];
#pragma unroll
  for (int e = 0; e < EL; ++e) acc[e] = 0.f;
  for (int k0 = w; k0 < nch; k0 += kWaves * U) {
    float mk[U], lk[U], pv[U][EL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + kWaves * u;
      const int kc = k < nch ? k : k0;
      mk[u] = xch_ldf(rml, (int)((base + kc) * 8));
      lk[u] = xch_ldf(rml, (int)((base + kc) * 8 + 4));
#pragma unroll
      for (int e = 0; e < EL; ++e) pv[u][e] = xch_ldf(rpo, (int)(((base + kc) * D + lane * EL + e) * 4));
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k0 + kWaves * u >= nch) mk[u] = -INFINITY;
    float bm = m;
#pragma unroll
    for (int u = 0; u < U; ++u) bm = fmaxf(bm, mk[u]);
    if (bm == -INFINITY) continue;
    const float r = (m == -INFINITY) ? 0.f : expf(m - bm);
    Ls *= r;
#pragma unroll
    for (int e = 0; e < EL; ++e) acc[e] *= r;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float wk = mk[u] == -INFINITY ? 0.f : expf(mk[u] - bm);
      Ls += lk[u] * wk;
#pragma unroll
      for (int e = 0; e < EL; ++e) acc[e] += pv[u][e] * wk;
    }
    m = bm;
  }
#pragma unroll
  for (int e = 0; e < EL; ++e) a_s[w * D + lane * EL + e] = acc[e];
  if (lane == 0) {
    m_s[w] = m;
    l_s[w] = Ls;
  }
  __syncthreads();
  if (threadIdx.x < D) {
    const int d = threadIdx.x;
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) M = fmaxf(M, m_s[q]);
    float Lt = 0.f, o = 0.f;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) {
      const float f = (m_s[q] == -INFINITY) ? 0.f : expf(m_s[q] - M);
      Lt += l_s[q] * f;
      o += a_s[q * D + d] * f;
    }
    dev_st2(dev_rsrc(L.attn_out), (int)((((long long)b * L.nq + h) * D + d) * 2),
            (uint16_t)f2bf(Lt > 0.f ? o / Lt : 0.f));
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
template <int D, int PER>
__global__ void __launch_bounds__(kThreads) layer_kernel(LayerArgs L) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = blockIdx.x, NB = gridDim.x;
  const int B = L.B, H = L.H, QD = L.nq * D;
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds + L.lds_a);       // [B][H] x, then r, then next x
  char* rb = lds + L.lds_b;
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds + L.lds_c);
  LkSel* sel = reinterpret_cast<LkSel*>(lds + L.lds_s);

  LK_STAMP(0);
  AttnArgs aa;                 // what the head preparation reads: rounding, q/k norm eps
  memset(&aa, 0, sizeof(aa));
  aa.qk_eps = L.qk_eps;
  aa.round_qwen = 1;

  // attention units (sequence t, kv head, chunk), sequence-major
  int ucount[kLkMaxB];
  int nunits = 0;
#pragma unroll
  for (int t = 0; t < kLkMaxB; ++t) {
    ucount[t] = t < B ? (lk_prior_len(L, t) + 1 + kChunk - 1) / kChunk * L.nkv : 0;
    nunits += ucount[t];
  }
  auto unit_of = [&](int uid, int& ub, int& ug, int& uc) {
    int r = uid;
    ub = 0;
#pragma unroll
    for (int t = 0; t < kLkMaxB - 1; ++t)
      if (ub == t && r >= ucount[t]) {
        r -= ucount[t];
        ub = t + 1;
      }
    ug = r % L.nkv;
    uc = r / L.nkv;
  };

  // ---- the input rows into LDS; the first QKV batch of layer 0 ----
  u32x4_t buf[kU];
  {
    const GemvCtx cq = gemv_ctx(L.q, 1, NB, blk, w, 1);
    LkGemv q0 = L.q;
    q0.w = L.layers[0].w_qkv;
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c) {
      const int i = (c * kThreads + threadIdx.x) * 8;
      if (i < B * H) *reinterpret_cast<u32x4_t*>(xs + i) = ld16(L.x + i);
    }
    gemv_load<false>(q0, nullptr, cq, cq.wlo, buf, lane);
  }
  __syncthreads();

  for (int l = 0; l < L.num_layers; ++l) {
    // opaque copies: keeps the per-stage partition set-up inside the loop
    // instead of hoisted (and held in registers across every stage)
    int lw = w, lb = blk, tid = threadIdx.x, ln = lane;
    asm volatile("" : "+s"(lw), "+s"(lb), "+v"(tid), "+v"(ln));
    const LkLayer ly = L.layers[l];
    const int kb = l * kLkBarriers;          // this layer's first barrier
    LkGemv gq = L.q, go = L.o, gr = L.r, ggu = L.gu, gdn = L.dn;
    gq.w = ly.w_qkv;
    go.w = ly.w_o;
    gr.w = ly.router;
    ggu.w = ly.gate_up;
    gdn.w = ly.down;

    // ---- P: pre-attention norm from the rows in LDS ----
    uint16_t* hn = reinterpret_cast<uint16_t*>(rb);                   // [B][H]
    {
      u32x4_t gm[kRowChunks];
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i < B * H) gm[c] = ld16(ly.ln_in + (i % H));
      }
      float ss[kLkMaxB] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i < B * H) {
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xs + i);
          const int t = i / H;
          float a = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) a += bf_lo(xv[j]) * bf_lo(xv[j]) + bf_hi(xv[j]) * bf_hi(xv[j]);
#pragma unroll
          for (int q = 0; q < kLkMaxB; ++q)
            if (q == t) ss[q] += a;
        }
      }
      block_sums(ss, B, sel, ln, w);
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i < B * H) {
          const int t = i / H;
          float rinv = 0.f;
#pragma unroll
          for (int q = 0; q < kLkMaxB; ++q)
            if (q == t) rinv = 1.0f / sqrtf(ss[q] * L.inv_h + L.eps);
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xs + i);
          u32x4_t o;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            o[j] = pack2bf((bf_lo(xv[j]) * rinv) * bf_lo(gm[c][j]), (bf_hi(xv[j]) * rinv) * bf_hi(gm[c][j]));
          *reinterpret_cast<u32x4_t*>(hn + i) = o;
        }
      }
    }
    __syncthreads();
    LK_STAMP(1);

    // ---- Q: QKV projection ----
    const GemvCtx cq = gemv_ctx(L.q, 1, NB, lb, lw, 1);
    {
      XSrc x = {};
      x.rows = hn;
      x.ld = H;
      x.ncol = B;
      gemv_run<XM_DENSE>(gq, nullptr, cq, buf, x, red, ln, w);
      gemv_finish(gq, cq, red, nullptr, B, blk, ln, w);
    }

    // ---- T: attention units (the first unit's cache rows across the barrier,
    // not by wave 0, which polls the barrier flags) ----
    AttnRows<D> rows;
    LK_STAMP(2);
    grid_arrive(L, kb + 0);
    if (blk < nunits && w != 0) {
      int ub, ug, uc;
      unit_of(blk, ub, ug, uc);
      attn_load<D>(L, ly, ub, ug, uc, ln, w, rows);
    }
    grid_wait(L, kb + 0);
    LK_STAMP(3);
    for (int uid = blk; uid < nunits; uid += NB) {
      int ub, ug, uc;
      unit_of(uid, ub, ug, uc);
      if (uid != blk || w == 0) attn_load<D>(L, ly, ub, ug, uc, ln, w, rows);
      attn_unit<D>(L, ly, aa, cq, ub, ug, uc, rows, reinterpret_cast<char*>(red), ln, w);
    }
    LK_STAMP(4);
    grid_arrive(L, kb + 1);
    grid_wait(L, kb + 1);
    LK_STAMP(5);

    // ---- C: combine, one block per (sequence, q head) ----
    for (int u = blk; u < B * L.nq; u += NB)
      combine_block<D>(L, u / L.nq, u - (u / L.nq) * L.nq, reinterpret_cast<char*>(red), ln, w);
    LK_STAMP(6);
    const GemvCtx co = gemv_ctx(L.o, 1, NB, lb, lw, 1);
    grid_arrive(L, kb + 2);
    gemv_load<false>(go, nullptr, co, co.wlo, buf, ln);
    grid_wait(L, kb + 2);
    LK_STAMP(7);

    // ---- O: output projection ----
    {
      uint16_t* ao = reinterpret_cast<uint16_t*>(rb);                 // [B][nq * D]
      const __amdgpu_buffer_rsrc_t ra = dev_rsrc(L.attn_out);
      for (int i = tid * 8; i < B * QD; i += kThreads * 8)
        *reinterpret_cast<u32x4_t*>(ao + i) = xch_ld16(ra, i * 2);
      __syncthreads();
      XSrc x = {};
      x.rows = ao;
      x.ld = QD;
      x.ncol = B;
      gemv_run<XM_DENSE>(go, nullptr, co, buf, x, red, ln, w);
      gemv_finish(go, co, red, nullptr, B, blk, ln, w);
    }
    LK_STAMP(8);
    const GemvCtx cr = gemv_ctx(L.r, 1, NB, lb, lw, 1);
    grid_arrive(L, kb + 3);
    gemv_load<false>(gr, nullptr, cr, cr.wlo, buf, ln);
    grid_wait(L, kb + 3);
    LK_STAMP(9);

    // ---- R: residual + post-attention norm (r kept in LDS), router logits ----
    uint16_t* hn2 = reinterpret_cast<uint16_t*>(rb);                  // [B][H] bf16
    float* y32 = reinterpret_cast<float*>(rb + (size_t)B * H * 2);    // [B][H] fp32
    {
      f32x4_t o0[kRowChunks], o1[kRowChunks];
      u32x4_t gm[kRowChunks];
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i < B * H) {
          const int t = i / H, h = i - t * H;
          gm[c] = ld16(ly.ln_post + h);
          o0[c] = part_sum4(go, co, h >> 4, t, h & 15);
          o1[c] = part_sum4(go, co, h >> 4, t, (h & 15) + 4);
        }
      }
      float ss[kLkMaxB] = {0.f, 0.f, 0.f, 0.f};
      u32x4_t rvs[kRowChunks];
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i < B * H) {
          const int t = i / H;
          const float ov[8] = {o0[c][0], o0[c][1], o0[c][2], o0[c][3], o1[c][0], o1[c][1], o1[c][2], o1[c][3]};
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xs + i);
          float a = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float r0 = rbf(bf_lo(xv[j]) + rbf(ov[2 * j]));
            const float r1 = rbf(bf_hi(xv[j]) + rbf(ov[2 * j + 1]));
            a += r0 * r0 + r1 * r1;
            rvs[c][j] = pack2bf(r0, r1);
          }
          *reinterpret_cast<u32x4_t*>(xs + i) = rvs[c];
          if (L.route_log && blk == 0)
            st16(L.route_log + (long long)l * L.log_stride + L.log_r + (long long)i * 2, rvs[c]);
#pragma unroll
          for (int q = 0; q < kLkMaxB; ++q)
            if (q == t) ss[q] += a;
        }
      }
      block_sums(ss, B, sel, ln, w);
#pragma unroll
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i < B * H) {
          const int t = i / H;
          float rinv = 0.f;
#pragma unroll
          for (int q = 0; q < kLkMaxB; ++q)
            if (q == t) rinv = 1.0f / sqrtf(ss[q] * L.inv_h + L.eps);
          float y[8];
          u32x4_t yb;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            y[2 * j] = (bf_lo(rvs[c][j]) * bf_lo(gm[c][j])) * rinv;
            y[2 * j + 1] = (bf_hi(rvs[c][j]) * bf_hi(gm[c][j])) * rinv;
            yb[j] = pack2bf(y[2 * j], y[2 * j + 1]);
          }
          *reinterpret_cast<u32x4_t*>(hn2 + i) = yb;
          *reinterpret_cast<f32x4_t*>(y32 + i) = f32x4_t{y[0], y[1], y[2], y[3]};
          *reinterpret_cast<f32x4_t*>(y32 + i + 4) = f32x4_t{y[4], y[5], y[6], y[7]};
        }
      }
    }
    __syncthreads();
    LK_STAMP(19);
    {
      XSrc x = {};
      x.rows32 = y32;
      x.ld = H;
      x.ncol = B;
      gemv_run<XM_F32>(gr, nullptr, cr, buf, x, red, ln, w);
      gemv_finish(gr, cr, red, nullptr, B, blk, ln, w);
    }
    LK_STAMP(10);
    grid_arrive(L, kb + 4);
    grid_wait(L, kb + 4);
    LK_STAMP(11);

    // ---- S: top-k and expert groups in every block ----
    {
      RouterArgs ra;
      memset(&ra, 0, sizeof(ra));
      ra.T = B;
      ra.E = L.E;
      ra.K = L.K;
      ra.mode = L.router_mode;
      ra.slot_w = sel->slot_w;
      ra.n_groups = &sel->ng;
      ra.grp_expert = sel->gexp;
      ra.grp_count = sel->gcnt;
      ra.grp_offset = sel->goff;
      ra.pair_token = sel->ptok;
      ra.pair_slot = sel->pslot;
      if (L.route_log && blk == 0) {       // the routing record of this layer
        char* rec = L.route_log + (long long)l * L.log_stride;
        ra.idx_out = reinterpret_cast<int*>(rec);
        ra.topk_out = reinterpret_cast<float*>(rec + L.log_w);
        ra.logits_out = reinterpret_cast<float*>(rec + L.log_logits);
      }
      select_small<PER>(ra, [&](int t, float (&lg)[PER]) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const int e = min(ln + 64 * j, L.E - 1);
          lg[j] = part_sum1(gr, cr, e >> 4, t, e & 15);
        }
      });
    }
    __syncthreads();
    LK_STAMP(20);
    const int ng = sel->ng;
    if (threadIdx.x < ng)
      for (int j = 0; j < sel->gcnt[threadIdx.x]; ++j) sel->pgrp[sel->goff[threadIdx.x] + j] = threadIdx.x;
    __syncthreads();
    const int npairs = ng > 0 ? sel->goff[ng - 1] + sel->gcnt[ng - 1] : 0;
    LK_STAMP(12);

    // ---- G: expert gate / up projections ----
    const GemvCtx cg = gemv_ctx(ggu, ng, NB, lb, lw, 0);
    gemv_load<false>(ggu, sel->gexp, cg, cg.wlo, buf, ln);
    {
      XSrc x = {};
      x.rows = hn2;
      x.ld = H;
      x.gcnt = sel->gcnt;
      x.goff = sel->goff;
      x.ptok = sel->ptok;
      gemv_run<XM_GROUP>(ggu, sel->gexp, cg, buf, x, red, ln, w);
      gemv_finish(ggu, cg, red, sel->gcnt, 0, blk, ln, w);
    }
    const GemvCtx cd = gemv_ctx(gdn, ng, NB, lb, lw, 1, true);
    LK_STAMP(13);
    grid_arrive(L, kb + 5);
    gemv_load<true>(gdn, sel->gexp, cd, cd.wlo, buf, ln);
    grid_wait(L, kb + 5);
    LK_STAMP(14);

    // ---- D: activations of the groups in the block's range, then the down
    // projections (row-block-major) with the routing-weighted sum over experts ----
    {
      uint16_t* act = reinterpret_cast<uint16_t*>(rb);               // [pair position][I]
      const int I = L.I;
      // the groups of the block's units: all of them, or nu consecutive ones
      // (cyclically) from the first unit's group
      int g0 = 0, nu = 0;
      if (cd.hi > cd.lo) {
        const int ub0 = (int)fdiv((uint32_t)cd.lo, cd.dKB), ub1 = (int)fdiv((uint32_t)(cd.hi - 1), cd.dKB);
        nu = ub1 - ub0 + 1;
        g0 = ub0 - (int)fdiv((uint32_t)ub0, cd.dNG) * ng;
      }
      GemmArgs ga;
      memset(&ga, 0, sizeof(ga));
      ga.round_qwen = 1;
      const int per_p = I / 4;
      for (int it = tid; it < npairs * per_p; it += kThreads) {
        const int q = it / per_p, i = (it - q * per_p) * 4;
        const int gg = sel->pgrp[q];
        if (nu < ng && (gg - g0 + ng) % ng >= nu) continue;
        const int j = q - sel->goff[gg];
        const int ub = gg * ggu.NRB + 2 * (i >> 4);
        const f32x4_t gv = part_sum4(ggu, cg, ub, j, i & 15);
        const f32x4_t uv = part_sum4(ggu, cg, ub + 1, j, i & 15);
        uint2 o;
        o.x = pack2bf(swiglu_value(ga, gv[0], uv[0]), swiglu_value(ga, gv[1], uv[1]));
        o.y = pack2bf(swiglu_value(ga, gv[2], uv[2]), swiglu_value(ga, gv[3], uv[3]));
        *reinterpret_cast<uint2*>(act + q * I + i) = o;
      }
      __syncthreads();
      LK_STAMP(21);
      XSrc x = {};
      x.rows = act;
      x.ld = I;
      x.gcnt = sel->gcnt;
      x.goff = sel->goff;
      gemv_run<XM_ACT, true>(gdn, sel->gexp, cd, buf, x, red, ln, w);
      gemv_finish_dn(gdn, cd, red, sel, B, blk, ln, w);
    }
    LK_STAMP(15);
    grid_arrive(L, kb + 6);
    if (l + 1 < L.num_layers) {              // the next layer's first QKV batch
      LkGemv q1 = L.q;
      q1.w = L.layers[l + 1].w_qkv;
      gemv_load<false>(q1, nullptr, cq, cq.wlo, buf, ln);
    }
    grid_wait(L, kb + 6);
    LK_STAMP(16);

    // ---- F: every block, all rows: x = bf16(r + bf16(sum of the row block's
    // partials)), the next layer's input, kept in LDS ----
    {
      const int span = cd.span;
#pragma unroll 1
      for (int c = 0; c < kRowChunks; ++c) {
        const int i = (c * kThreads + tid) * 8;
        if (i >= B * H) break;
        const int t = i / H, h = i - t * H;
        const int rbk = h >> 4, r0 = h & 15;
        const uint32_t f0 = (uint32_t)(rbk * span);
        const int b0 = (int)fdiv(f0, cd.dfpb), b1 = (int)fdiv(f0 + span - 1, cd.dfpb);
        const int lr0 = rbk - (int)fdiv((uint32_t)(b0 * cd.fpb), cd.dspan);
        const __amdgpu_buffer_rsrc_t rp = dev_rsrc(gdn.part);
        f32x4_t v0[kMaxS], v1[kMaxS];
#pragma unroll
        for (int sidx = 0; sidx < kMaxS; ++sidx) {
          const int bb = min(b0 + sidx, b1);
          const int lr = bb == b0 ? lr0 : 0;
          const int off = (((bb * gdn.LB + lr) * kCols + t) * 16 + r0) * 4;
          v0[sidx] = xch_ld4f(rp, off);
          v1[sidx] = xch_ld4f(rp, off + 16);
        }
        f32x4_t s0 = v0[0], s1 = v1[0];
#pragma unroll
        for (int sidx = 1; sidx < kMaxS; ++sidx)
          if (b0 + sidx <= b1) {
            s0 += v0[sidx];
            s1 += v1[sidx];
          }
        const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        const u32x4_t rv = *reinterpret_cast<const u32x4_t*>(xs + i);
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = pack2bf(rbf(bf_lo(rv[j]) + rbf(sv[2 * j])), rbf(bf_hi(rv[j]) + rbf(sv[2 * j + 1])));
        *reinterpret_cast<u32x4_t*>(xs + i) = o;
      }
    }
    __syncthreads();
    LK_STAMP(17);
  }

  // ---- the block's slice of the final rows ----
  {
    const int n8 = B * H / 8;
    for (int c = (int)((long long)n8 * blk / NB) + threadIdx.x; c < (int)((long long)n8 * (blk + 1) / NB);
         c += kThreads)
      *reinterpret_cast<u32x4_t*>(L.x + c * 8) = *reinterpret_cast<const u32x4_t*>(xs + c * 8);
  }
}

// ---------------------------------------------------------------------------
__global__ void layer_reset_kernel(unsigned* bar) {
  for (int i = threadIdx.x; i < kLkBarWords; i += blockDim.x) bar[i] = 0u;
}

hipError_t layer_reset_launch(unsigned* bar, hipStream_t s) {
  hipLaunchKernelGGL(layer_reset_kernel, dim3(1), dim3(256), 0, s, bar);
  return hipGetLastError();
}

template <int D, int PER>
static hipError_t launch_dp(const LayerArgs& a, hipStream_t s) {
  static int lds_set = 0;
  if (a.lds_total > lds_set) {
    if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&layer_kernel<D, PER>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, a.lds_total))
      return e;
    lds_set = a.lds_total;
  }
  return timed_launch(layer_kernel<D, PER>, dim3(a.NB), dim3(kThreads), (size_t)a.lds_total, s, a);
}

hipError_t layer_kernel_launch(const LayerArgs& a, hipStream_t s) {
  const int per = (a.E + 63) / 64;
  if (a.d == 128) return per <= 2 ? launch_dp<128, 2>(a, s) : launch_dp<128, 8>(a, s);
  if (a.d == 64) return per <= 2 ? launch_dp<64, 2>(a, s) : launch_dp<64, 8>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace mkd
