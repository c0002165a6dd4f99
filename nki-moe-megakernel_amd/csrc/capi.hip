// extern "C" entry points of libmkd.so (declared in include/mkd.h).
//
// This layer validates shapes and pointers on the host, carves the caller's
// workspace, and enqueues the kernels on the caller's stream.  It never
// allocates device memory and never synchronises.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"
#include "mkd_internal.h"
#include "../../include/mkd.h"

using namespace mkd;

LaunchTiming mkd::g_launch_timing;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// MKD_SYNC_CHECK=1 in the environment: synchronise after every launch so a
// failing kernel is named at its own call site (debugging aid; never on by default).
bool sync_check() {
  static const int on = [] {
    const char* e = getenv("MKD_SYNC_CHECK");
    return (e && e[0] == '1') ? 1 : 0;
  }();
  return on;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MKD_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  if (sync_check()) {
    e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) return fail(MKD_ERR_HIP, "%s (synchronised): %s", what, hipGetErrorString(e));
  }
  return MKD_OK;
}

// A HIP error left pending by an earlier, unrelated call would otherwise be
// reported by the first launch check of the next entry point; clear it at entry
// and name it if debugging.
int stale_check(const char* fn) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess && sync_check())
    return fail(MKD_ERR_HIP, "%s: HIP error pending before entry: %s", fn, hipGetErrorString(e));
  return MKD_OK;
}

// ---- measurement hook state (mkd_profile_events) ----
struct ProfState {
  int cls = -1;
  int n = 0;
  int next = 0;
  hipEvent_t start[512];
  hipEvent_t stop[512];
} g_prof;

// The events of a slot are recorded by the bracketed kernel's own dispatch
// (g_launch_timing), so they time the kernel alone.  Nothing is armed while the
// stream is being captured (a graph keeps no timing events).  A bracket whose
// launches never consumed the pair gives its slot back and turns the hook off,
// so mkd_profile_count() reports fewer launches than the caller expected.
int prof_begin(int cls, hipStream_t s) {
  if (g_prof.cls != cls || g_prof.next >= g_prof.n) return -1;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return -1;
  }
  const int i = g_prof.next++;
  g_launch_timing.start = g_prof.start[i];
  g_launch_timing.stop = g_prof.stop[i];
  return i;
}
void prof_end(int slot, hipStream_t) {
  if (slot < 0) return;
  if (g_launch_timing.start) {                // not consumed by any launch
    g_launch_timing = LaunchTiming{};
    --g_prof.next;
    g_prof.cls = -1;
  }
}

#define MKD_REQUIRE(cond, code, ...) \
  do {                               \
    if (!(cond)) return fail(code, __VA_ARGS__); \
  } while (0)

#define MKD_TRY(expr, what)                   \
  do {                                        \
    int rc_ = hip_check((expr), what);        \
    if (rc_) return rc_;                      \
  } while (0)

// Bump allocator over the caller's workspace (256-byte aligned slices).
struct Carver {
  char* base;
  size_t cap, used = 0;
  bool ok = true;
  template <class T>
  T* take(size_t count) {
    const size_t bytes = (count * sizeof(T) + 255) & ~size_t(255);
    if (used + bytes > cap) { ok = false; used += bytes; return nullptr; }
    T* p = reinterpret_cast<T*>(base + used);
    used += bytes;
    return p;
  }
};

int token_tiles(int T) { return T <= 16 ? 1 : (T <= 32 ? 2 : 4); }

GemmArgs dense_args(const void* w, const void* x, int ldx, int N, int K, int T, void* y, int ldy) {
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.w = reinterpret_cast<const uint16_t*>(w);
  a.x = x;
  a.ldx = ldx;
  a.N = N;
  a.K = K;
  a.KW = choose_kw(K, 512, (N + 15) / 16);
  a.T = T;
  a.y = y;
  a.ldy = ldy;
  a.gate_hi = INFINITY; a.gate_lo = -INFINITY; a.up_hi = INFINITY; a.up_lo = -INFINITY;
  return a;
}

// Rows of a packed matrix: the logical count rounded up to a 16-row block.
long long padded_rows(int N) { return ((long long)N + 15) / 16 * 16; }

// rb == 2 (fused gate/up) needs each half to be whole 16-row blocks.
int check_gemm_dims(int N, int K, int rb) {
  MKD_REQUIRE(N > 0 && (rb == 1 || N % (16 * rb) == 0), MKD_ERR_INVALID,
              "fused gate/up width %d must be a multiple of %d", N, 16 * rb);
  MKD_REQUIRE(K > 0 && K % 32 == 0, MKD_ERR_INVALID, "contraction %d must be a multiple of 32", K);
  MKD_REQUIRE(choose_kw(K) > 0, MKD_ERR_UNSUPPORTED,
              "contraction %d has no split into <= 16 waves of a multiple of 32 (max 8192)", K);
  return MKD_OK;
}

// MX weights: whole 16-row blocks (32 for fused gate/up), K % 32 == 0, and a
// padded contraction that splits over <= 8 waves.
int check_mx_dims(int N, int K, int rb) {
  MKD_REQUIRE(N > 0 && N % (16 * rb) == 0, MKD_ERR_INVALID,
              "MX weight rows %d must be a multiple of %d", N, 16 * rb);
  MKD_REQUIRE(K > 0 && K % 32 == 0, MKD_ERR_INVALID, "MX contraction %d must be a multiple of 32", K);
  MKD_REQUIRE(choose_kw_mx(mx_kpad(K)) > 0, MKD_ERR_UNSUPPORTED, "MX contraction %d is too large", K);
  return MKD_OK;
}

// The LDS-tiled GEMM addresses one expert's (or the dense) weight block and its
// activation rows through 32-bit buffer offsets: both must stay below 2^31 bytes.
bool tile_offsets_ok(long long x_rows, long long ldx, long long N, long long K) {
  constexpr long long kLim = 1LL << 31;
  return x_rows * ldx * 2 < kLim && padded_rows((int)N) * K * 2 < kLim;
}

// Dense launch: the tiled MFMA GEMM for many tokens, else one launch of 16..64-token
// column tiles.
int dense_gemm(GemmArgs a, int epi, bool xf32, hipStream_t s) {
  const int T = a.T;
  // many tokens (prefill passes): the LDS-tiled MFMA GEMM, fp32 out (+ bias)
  if (T >= 256 && epi == EPI_F32 && !xf32 && (a.kgrid <= 1 || gemm_tile_kgrid_ok(a.K, a.kgrid)) &&
      !a.residual && !a.grp_expert &&
      gemm_tile_supported(a.N, a.K, EPI_SCALE_F32) && tile_offsets_ok(T, a.ldx, a.N, a.K)) {
    a.pair_scale = nullptr;
    MKD_TRY(gemm_tile_launch(a, EPI_SCALE_F32, 1, T, s), "tiled gemm");
    return MKD_OK;
  }
  // more than one 64-token column of tiles: one launch over all of them (grid z
  // holds the token tiles x the K split)
  if (T > 64) {
    MKD_TRY(gemm_launch(a, epi, xf32, 4, 1, T, s), "gemm launch");
    return MKD_OK;
  }
  for (int t0 = 0; t0 < T; t0 += 64) {
    GemmArgs b = a;
    const int tt = T - t0 < 64 ? T - t0 : 64;
    b.T = tt;
    b.x = static_cast<const char*>(a.x) + (size_t)t0 * a.ldx * (xf32 ? 4 : 2);
    const int ysz = (epi == EPI_F32 || epi == EPI_SCALE_F32) ? 4 : 2;
    b.y = static_cast<char*>(a.y) + (size_t)t0 * a.ldy * ysz;
    if (a.residual) b.residual = a.residual + (size_t)t0 * a.ldy;
    MKD_TRY(gemm_launch(b, epi, xf32, token_tiles(tt), 1, tt, s), "gemm launch");
  }
  return MKD_OK;
}

// Router GEMM split over K across blocks so that even E = 128 (8 row blocks)
// occupies ~128 blocks; the select kernel sums the partials in order.
int router_kgrid(int E, int H) {
  const int tiles = (E + 15) / 16;
  int kg = 1;
  while (kg < 16 && tiles * kg < 128) kg *= 2;
  while (kg > 1 && choose_kw_split(H, kg) <= 0) kg /= 2;
  return kg;
}

// logits (split-K partials into `parts`) -> select (+ groups when r.n_groups).
int router_stage(const void* x, bool xf32, int H, const void* w_packed, float* parts, RouterArgs r,
                 hipStream_t s, bool multi = false) {
  const int kg = router_kgrid(r.E, H);
  GemmArgs a = dense_args(w_packed, x, H, r.E, H, r.T, parts, r.E);
  a.kgrid = kg;
  a.KW = kg > 1 ? choose_kw_split(H, kg) : choose_kw(H);
  a.part_stride = (long long)r.T * r.E;
  MKD_REQUIRE(a.KW > 0, MKD_ERR_UNSUPPORTED, "router: no K split for H=%d", H);
  // 17..128 tokens: the rows' K slices staged in LDS (gemm_mid), the same number
  // of K-split partials when the split matches
  if (gemm_mid_kgrid(r.E, H, r.T, 16) == kg) {
    MKD_TRY(gemm_mid_launch(a, kg, xf32, s), "router gemm (mid)");
  } else if (r.T > 128 && gemm_mid_chunked_ok(H, kg)) {
    // a prefill pass: the same, over chunks of 128 tokens, each chunk's activation
    // slice staged once per block instead of re-read for every 16-row block
    MKD_TRY(gemm_mid_launch(a, kg, xf32, s), "router gemm (mid, token chunks)");
  } else if (int rc = dense_gemm(a, EPI_F32, xf32, s)) {
    return rc;
  }
  r.parts = parts;
  r.nparts = kg;
  r.part_stride = a.part_stride;
  if (multi) {
    MKD_TRY(router_select_multi_launch(r, s), "router select (multi-block)");
  } else if (r.n_groups && r.T > 16 && r.idx_out) {
    // more tokens than one block's waves: one token per wave over several
    // blocks, then the expert groups from the indices (one block serialising
    // the tokens took 24 us at 64 tokens)
    RouterArgs q = r;
    q.n_groups = nullptr;
    MKD_TRY(router_select_multi_launch(q, s), "router select (multi-block)");
    MKD_TRY(moe_route_launch(r.idx_out, r.T, r.K, r.E, r.n_groups, r.grp_expert, r.grp_count,
                             r.grp_offset, r.pair_token, r.pair_slot, s), "router groups");
  } else {
    MKD_TRY(router_select_launch(r, s), "router select");
  }
  return MKD_OK;
}

struct MoeWs {
  int *n_groups, *grp_expert, *grp_count, *grp_offset, *pair_token, *pair_slot, *idx;
  int* route_off;               // per-chunk slot offsets of the split routing
  float *slot_w, *ybuf;
  uint16_t* hbuf;
  uint8_t *xq, *xs, *hq, *hs;   // MXFP8 codes / scales of the hidden rows and of hbuf
};

int mx_pad(int k) { return mx_kpad(k); }

MoeWs carve_moe(Carver& c, int T, int H, int E, int I, int K) {
  MoeWs w;
  w.n_groups = c.take<int>(1);
  w.grp_expert = c.take<int>(E);
  w.grp_count = c.take<int>(E);
  w.grp_offset = c.take<int>(E);
  w.pair_token = c.take<int>((size_t)T * K);
  w.pair_slot = c.take<int>((size_t)T * K);
  w.idx = c.take<int>((size_t)T * K);
  w.route_off = c.take<int>(kRouteChunkCounts);
  w.slot_w = c.take<float>((size_t)T * K);
  w.hbuf = c.take<uint16_t>((size_t)T * K * I);
  w.ybuf = c.take<float>((size_t)T * K * H);
  w.xq = c.take<uint8_t>((size_t)T * mx_pad(H));
  w.xs = c.take<uint8_t>((size_t)T * mx_pad(H) / 32);
  w.hq = c.take<uint8_t>((size_t)T * K * mx_pad(I));
  w.hs = c.take<uint8_t>((size_t)T * K * mx_pad(I) / 32);
  return w;
}

__global__ void gather_slot_weights(const float* aff, const int* idx, int T, int E, int K,
                                    float* slot_w) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= T * K) return;
  const int e = idx[p];
  slot_w[p] = (aff && e >= 0 && e < E) ? aff[(long long)(p / K) * E + e] : (aff ? 0.0f : 1.0f);
}

__global__ void copy_slot_weights(const float* src, int n, float* dst) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p < n) dst[p] = src[p];
}

// Per-wave K slice of the frag gate/up GEMM (two row blocks per wave).
int gate_up_kw(int H, int I, int gmax) { return choose_kw(H, 256, (long long)(I / 16) * gmax); }

// The expert FFN on an already-routed batch: routing tables -> gate/up -> down -> finalize.
// With `sel` (a few tokens, bf16 frag experts) the routing is formed inside the
// gate/up launch from the router's partial logits instead.
int moe_core(const uint16_t* hidden, const void* gate_up, const void* down, const int* idx,
             const float* slot_w, const uint16_t* gu_bias, const uint16_t* dn_bias,
             const uint16_t* resid, uint16_t* out, float* out_f32, int T, int H, int E, int I,
             int K, int act, float alpha, float ghi, float glo, float uhi, float ulo, int round_qwen,
             MoeWs& w, hipStream_t s, bool do_finalize = true, int wfmt = 0,
             const void* gu_scales = nullptr, const void* dn_scales = nullptr, bool tiled = false,
             const RouterArgs* sel = nullptr, unsigned* fused_flags = nullptr,
             unsigned* fused_err = nullptr, uint16_t* poll_h = nullptr,
             const uint16_t* hn_r = nullptr, const uint16_t* hn_gamma = nullptr,
             bool x_mx_ready = false) {
  if (sel && (idx || wfmt || tiled)) return MKD_ERR_INVALID;
  if (fused_flags && !sel) return MKD_ERR_INVALID;
  if (idx)  // otherwise the router stage already built the expert groups
    MKD_TRY(moe_route_launch(idx, T, K, E, w.n_groups, w.grp_expert, w.grp_count, w.grp_offset,
                             w.pair_token, w.pair_slot, s, w.route_off), "moe_route");
  const int gmax = E < T * K ? E : T * K;
  if (wfmt == MKD_FP8_E4M3) {
    // e4m3 experts (FP8 ROW / STATIC): bf16 activations, per-column dequantisation
    W8GroupArgs a;
    memset(&a, 0, sizeof(a));
    a.g.n_groups = w.n_groups; a.g.grp_expert = w.grp_expert; a.g.grp_count = w.grp_count;
    a.g.grp_offset = w.grp_offset;
    a.act.act = act; a.act.alpha = alpha; a.act.gate_hi = ghi; a.act.gate_lo = glo;
    a.act.up_hi = uhi; a.act.up_lo = ulo;
    a.w = static_cast<const uint8_t*>(gate_up);
    a.w_group_stride = 2LL * I * H;
    a.x = hidden; a.ldx = H; a.N = 2 * I; a.K = H;
    a.x_row = w.pair_token; a.out_row = w.pair_slot;
    a.col_scale = static_cast<const float*>(gu_scales);
    a.bias = gu_bias;
    a.h = w.hbuf; a.ldy = I;
    {
      const int ps = prof_begin(MKD_KCLASS_MOE_GATE_UP, s);
      MKD_TRY(gemm_w8_grouped_launch(a, W8_SWIGLU, gmax, s), "moe gate_up (fp8)");
      prof_end(ps, s);
    }
    a.w = static_cast<const uint8_t*>(down);
    a.w_group_stride = (long long)H * I;
    a.x = w.hbuf; a.ldx = I; a.N = H; a.K = I;
    a.x_row = w.pair_slot;
    a.col_scale = static_cast<const float*>(dn_scales);
    a.bias = dn_bias;
    a.pair_scale = slot_w;
    a.h = nullptr; a.y = w.ybuf; a.ldy = H;
    {
      const int ps = prof_begin(MKD_KCLASS_MOE_DOWN, s);
      MKD_TRY(gemm_w8_grouped_launch(a, W8_SCALE, gmax, s), "moe down (fp8)");
      prof_end(ps, s);
    }
    if (do_finalize)
      MKD_TRY(moe_finalize_launch(w.ybuf, T, K, H, resid, out, out_f32, s), "moe finalize");
    return MKD_OK;
  }
  if (wfmt) {
    // MX experts: hidden -> MXFP8, gate/up (scaled MFMA) + SwiGLU -> bf16 h,
    // h -> MXFP8, down (scaled MFMA) * slot affinity.
    const int Hp = mx_pad(H), Ip = mx_pad(I);
    if (!x_mx_ready)   // else the norm that produced `hidden` wrote its MXFP8 form too
      MKD_TRY(mx_quantize_launch(hidden, false, T, H, H, MX_E4M3, w.xq, w.xs, Hp, s), "moe quantize hidden");
    {
      GemmArgs a = dense_args(gate_up, w.xq, Hp, 2 * I, Hp, T, w.hbuf, I);
      a.KW = choose_kw_mx(Hp);
      a.w_group_stride = mx_packed_code_bytes(1, 2 * I, H, wfmt);
      a.w_scale = static_cast<const uint8_t*>(gu_scales);
      a.w_scale_group_stride = mx_packed_scale_bytes(1, 2 * I, H);
      a.x_scale = w.xs; a.ldxs = Hp / 32;
      a.grp_expert = w.grp_expert; a.grp_count = w.grp_count; a.grp_offset = w.grp_offset;
      a.n_groups = w.n_groups; a.pair_row = w.pair_token; a.pair_out_row = w.pair_slot;
      a.bias = gu_bias; a.bias_group_stride = 2LL * I;
      a.act = act; a.alpha = alpha; a.gate_hi = ghi; a.gate_lo = glo; a.up_hi = uhi; a.up_lo = ulo;
      a.round_qwen = 0;
      const int ps = prof_begin(MKD_KCLASS_MOE_GATE_UP, s);
      MKD_TRY(gemm_mx_launch(a, wfmt, EPI_SWIGLU_BF16, gmax, T, s), "moe gate_up (mx)");
      prof_end(ps, s);
    }
    MKD_TRY(mx_quantize_launch(w.hbuf, false, T * K, I, I, MX_E4M3, w.hq, w.hs, Ip, s),
            "moe quantize intermediate");
    {
      GemmArgs a = dense_args(down, w.hq, Ip, H, Ip, T, w.ybuf, H);
      a.KW = choose_kw_mx(Ip);
      a.w_group_stride = mx_packed_code_bytes(1, H, I, wfmt);
      a.w_scale = static_cast<const uint8_t*>(dn_scales);
      a.w_scale_group_stride = mx_packed_scale_bytes(1, H, I);
      a.x_scale = w.hs; a.ldxs = Ip / 32;
      a.grp_expert = w.grp_expert; a.grp_count = w.grp_count; a.grp_offset = w.grp_offset;
      a.n_groups = w.n_groups; a.pair_row = w.pair_slot; a.pair_out_row = w.pair_slot;
      a.pair_scale = slot_w;
      a.bias = dn_bias; a.bias_group_stride = H;
      const int ps = prof_begin(MKD_KCLASS_MOE_DOWN, s);
      MKD_TRY(gemm_mx_launch(a, wfmt, EPI_SCALE_F32, gmax, T, s), "moe down (mx)");
      prof_end(ps, s);
    }
    if (do_finalize)
      MKD_TRY(moe_finalize_launch(w.ybuf, T, K, H, resid, out, out_f32, s), "moe finalize");
    return MKD_OK;
  }
  if (tiled) {
    // Many tokens per expert: LDS-tiled grouped GEMMs (256 x 256 tiles), one
    // token tile per 256 tokens of the largest possible group (T).
    {
      GemmArgs a = dense_args(gate_up, hidden, H, 2 * I, H, T, w.hbuf, I);
      a.w_group_stride = (long long)2 * I * H;
      a.grp_expert = w.grp_expert; a.grp_count = w.grp_count; a.grp_offset = w.grp_offset;
      a.n_groups = w.n_groups; a.pair_row = w.pair_token; a.pair_out_row = w.pair_slot;
      a.bias = gu_bias; a.bias_group_stride = 2LL * I;
      a.act = act; a.alpha = alpha; a.gate_hi = ghi; a.gate_lo = glo; a.up_hi = uhi; a.up_lo = ulo;
      a.round_qwen = round_qwen;
      const int ps = prof_begin(MKD_KCLASS_MOE_GATE_UP, s);
      MKD_TRY(gemm_tile_launch(a, EPI_SWIGLU_BF16, gmax, (long long)T * K, s), "moe gate_up (tiled)");
      prof_end(ps, s);
    }
    {
      GemmArgs a = dense_args(down, w.hbuf, I, H, I, T, w.ybuf, H);
      a.w_group_stride = padded_rows(H) * I;
      a.grp_expert = w.grp_expert; a.grp_count = w.grp_count; a.grp_offset = w.grp_offset;
      a.n_groups = w.n_groups; a.pair_row = w.pair_slot; a.pair_out_row = w.pair_slot;
      a.pair_scale = slot_w;
      a.bias = dn_bias; a.bias_group_stride = H;
      const int ps = prof_begin(MKD_KCLASS_MOE_DOWN, s);
      MKD_TRY(gemm_tile_launch(a, EPI_SCALE_F32, gmax, (long long)T * K, s), "moe down (tiled)");
      prof_end(ps, s);
    }
    if (do_finalize)
      MKD_TRY(moe_finalize_launch(w.ybuf, T, K, H, resid, out, out_f32, s), "moe finalize");
    return MKD_OK;
  }
  // Routed experts see few tokens each (T*K/E on average), so one 16-token
  // MFMA column tile per block; groups with more tokens use extra z-tiles.
  const int tn = 1;
  if (fused_flags) {
    // a few tokens: router top-k, gate/up and down in one launch (the down
    // blocks wait for their group's gate/up blocks inside the launch)
    MoeFusedArgs f = {};
    f.gu = dense_args(gate_up, hidden, H, 2 * I, H, T, w.hbuf, I);
    f.gu.KW = H / 8;
    f.gu.w_group_stride = (long long)2 * I * H;
    f.gu.bias = gu_bias; f.gu.bias_group_stride = 2LL * I;
    f.gu.act = act; f.gu.alpha = alpha; f.gu.gate_hi = ghi; f.gu.gate_lo = glo;
    f.gu.up_hi = uhi; f.gu.up_lo = ulo;
    f.gu.round_qwen = round_qwen;
    f.gu.grp_expert = w.grp_expert;      // replaced by the block's own tables
    f.dn = dense_args(down, w.hbuf, I, H, I, T, w.ybuf, H);
    f.dn.w_group_stride = padded_rows(H) * I;
    f.dn.bias = dn_bias; f.dn.bias_group_stride = H;
    f.r = *sel;
    f.flags = fused_flags; f.err = fused_err;
    f.poll_h = T == 1 ? poll_h : nullptr;
    if (sel->ss_parts) {   // the experts' input is formed in the launch (K-sliced router form)
      f.hn_r = hn_r;
      f.hn_gamma = hn_gamma;
      f.hn_out = const_cast<uint16_t*>(hidden);
    }
    const int ps = prof_begin(MKD_KCLASS_MOE_GATE_UP, s);
    MKD_TRY(moe_fused_launch(f, gmax, s), "moe router select + gate_up + down");
    prof_end(ps, s);
    if (do_finalize)
      MKD_TRY(moe_finalize_launch(w.ybuf, T, K, H, resid, out, out_f32, s), "moe finalize");
    return MKD_OK;
  }
  {  // gate/up + activation
    GemmArgs a = dense_args(gate_up, hidden, H, 2 * I, H, T, w.hbuf, I);
    a.KW = gate_up_kw(H, I, gmax);
    a.w_group_stride = (long long)2 * I * H;
    a.grp_expert = w.grp_expert; a.grp_count = w.grp_count; a.grp_offset = w.grp_offset;
    a.n_groups = w.n_groups; a.pair_row = w.pair_token; a.pair_out_row = w.pair_slot;
    a.bias = gu_bias; a.bias_group_stride = 2LL * I;
    a.act = act; a.alpha = alpha; a.gate_hi = ghi; a.gate_lo = glo; a.up_hi = uhi; a.up_lo = ulo;
    a.round_qwen = round_qwen;
    const int ps = prof_begin(MKD_KCLASS_MOE_GATE_UP, s);
    if (sel)   // the router top-k and the expert groups are formed in the gate/up blocks
      MKD_TRY(gemm_sel_launch(a, *sel, gmax, s), "moe router select + gate_up");
    else
      MKD_TRY(gemm_launch(a, EPI_SWIGLU_BF16, false, tn, gmax, T, s), "moe gate_up");
    prof_end(ps, s);
  }
  {  // down, scaled by the slot affinity
    GemmArgs a = dense_args(down, w.hbuf, I, H, I, T, w.ybuf, H);
    a.KW = choose_kw(I, 512, (long long)((H + 15) / 16) * gmax);
    a.w_group_stride = padded_rows(H) * I;
    a.grp_expert = w.grp_expert; a.grp_count = w.grp_count; a.grp_offset = w.grp_offset;
    a.n_groups = w.n_groups; a.pair_row = w.pair_slot; a.pair_out_row = w.pair_slot;
    a.pair_scale = slot_w;
    a.bias = dn_bias; a.bias_group_stride = H;
    const int ps = prof_begin(MKD_KCLASS_MOE_DOWN, s);
    MKD_TRY(gemm_launch(a, EPI_SCALE_F32, false, tn, gmax, T, s), "moe down");
    prof_end(ps, s);
  }
  if (do_finalize)
    MKD_TRY(moe_finalize_launch(w.ybuf, T, K, H, resid, out, out_f32, s), "moe finalize");
  return MKD_OK;
}

}  // namespace

extern "C" {

int mkd_version(void) { return 1; }
const char* mkd_last_error(void) { return g_err; }

int mkd_rmsnorm_tkg(const void* input, int input_dtype, const void* gamma, void* output,
                    int output_dtype, int rows, int hidden, int hidden_actual, float eps,
                    void* stream) {
  if (int rc = stale_check("mkd_rmsnorm_tkg")) return rc;
  MKD_REQUIRE(input && gamma && output, MKD_ERR_NULL, "rmsnorm_tkg: null pointer");
  MKD_REQUIRE(rows > 0, MKD_ERR_INVALID, "rmsnorm_tkg: rows must be > 0, got %d", rows);
  MKD_REQUIRE(hidden > 0 && hidden % 8 == 0 && hidden <= 8192, MKD_ERR_INVALID,
              "rmsnorm_tkg: hidden %d must be a multiple of 8 and <= 8192", hidden);
  MKD_REQUIRE(input_dtype == MKD_DT_BF16 || input_dtype == MKD_DT_F32, MKD_ERR_INVALID, "rmsnorm_tkg: bad input dtype");
  MKD_REQUIRE(output_dtype == MKD_DT_BF16 || output_dtype == MKD_DT_F32, MKD_ERR_INVALID, "rmsnorm_tkg: bad output dtype");
  const int ha = hidden_actual > 0 ? hidden_actual : hidden;
  MKD_REQUIRE(ha <= hidden, MKD_ERR_INVALID, "rmsnorm_tkg: hidden_actual %d > hidden %d", ha, hidden);
  hipStream_t s = static_cast<hipStream_t>(stream);
  MKD_TRY(rmsnorm_launch(input, input_dtype == MKD_DT_F32, static_cast<const uint16_t*>(gamma),
                         output_dtype == MKD_DT_BF16 ? static_cast<uint16_t*>(output) : nullptr,
                         output_dtype == MKD_DT_F32 ? static_cast<float*>(output) : nullptr, rows,
                         hidden, hidden, ha, eps, 0, s), "rmsnorm launch");
  return MKD_OK;
}

size_t mkd_packed_bytes(int groups, int n, int k) {
  return (size_t)groups * (size_t)padded_rows(n) * (size_t)k * 2;
}

int mkd_pack_weights(const void* src, void* dst, int groups, int n, int k, long long g_stride,
                     long long row_stride, long long col_stride, int interleave_half,
                     void* stream) {
  if (int rc = stale_check("mkd_pack_weights")) return rc;
  MKD_REQUIRE(src && dst, MKD_ERR_NULL, "pack_weights: null pointer");
  MKD_REQUIRE(groups > 0 && n > 0 && k > 0, MKD_ERR_INVALID, "pack_weights: empty shape");
  if (int rc = check_gemm_dims(n, k, interleave_half > 0 ? 2 : 1)) return rc;
  MKD_REQUIRE(interleave_half == 0 || (interleave_half * 2 == n && interleave_half % 16 == 0),
              MKD_ERR_INVALID, "pack_weights: interleave_half %d must be n/2 and a multiple of 16", interleave_half);
  MKD_TRY(pack_frag_launch(static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), groups,
                           n, k, g_stride, row_stride, col_stride, interleave_half,
                           static_cast<hipStream_t>(stream)), "pack launch");
  return MKD_OK;
}

int mkd_linear(const void* x, int x_dtype, int ldx, int rows, const void* w_packed, int n, int k,
               const void* bias, void* y, int y_dtype, int ldy, const void* residual,
               void* stream) {
  if (int rc = stale_check("mkd_linear")) return rc;
  MKD_REQUIRE(x && w_packed && y, MKD_ERR_NULL, "linear: null pointer");
  MKD_REQUIRE(rows > 0 && rows <= kMaxPrefillT, MKD_ERR_INVALID, "linear: rows %d must be in [1, %d]", rows,
              kMaxPrefillT);
  if (int rc = check_gemm_dims(n, k, 1)) return rc;
  MKD_REQUIRE(ldx >= k && ldy >= n, MKD_ERR_INVALID, "linear: leading dims too small");
  MKD_REQUIRE(ldx % 8 == 0 && ldy % 4 == 0, MKD_ERR_INVALID, "linear: leading dims must be 16-byte aligned");
  MKD_REQUIRE(!residual || y_dtype == MKD_DT_BF16, MKD_ERR_INVALID, "linear: residual needs bf16 output");
  GemmArgs a = dense_args(w_packed, x, ldx, n, k, rows, y, ldy);
  a.bias = static_cast<const uint16_t*>(bias);
  a.residual = static_cast<const uint16_t*>(residual);
  const int epi = residual ? EPI_RESID_BF16 : (y_dtype == MKD_DT_F32 ? EPI_F32 : EPI_BF16);
  return dense_gemm(a, epi, x_dtype == MKD_DT_F32, static_cast<hipStream_t>(stream));
}

size_t mkd_router_workspace_bytes(int T, int H, int E) {
  return (size_t)router_kgrid(E, H) * T * E * sizeof(float) + 256;
}

int mkd_router_topk(const void* x, int x_dtype, int T, int H, const void* w_packed, int E,
                    const void* w_bias, float* router_logits, float* expert_affinities,
                    int* expert_index, float* topk_affinities, int k, int mode, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (int rc = stale_check("mkd_router_topk")) return rc;
  MKD_REQUIRE(x && w_packed && router_logits && expert_index && workspace, MKD_ERR_NULL,
              "router_topk: null pointer");
  MKD_REQUIRE(T > 0 && T <= kMaxPrefillT, MKD_ERR_INVALID, "router_topk: T %d must be in [1, %d]", T,
              kMaxPrefillT);
  MKD_REQUIRE(E > 0 && E <= 512, MKD_ERR_INVALID, "router_topk: E %d must be in [1, 512]", E);
  MKD_REQUIRE(k >= 1 && k <= 8 && k <= E, MKD_ERR_INVALID, "router_topk: k %d must be in [1, 8]", k);
  if (int rc = check_gemm_dims(E, H, 1)) return rc;
  const bool pre = mode & MKD_ROUTER_PRE_NORM, norm = mode & MKD_ROUTER_NORM_TOPK;
  MKD_REQUIRE(!(norm && !pre), MKD_ERR_INVALID, "router_topk: norm_topk_prob requires router_pre_norm");
  MKD_REQUIRE(workspace_bytes >= mkd_router_workspace_bytes(T, H, E), MKD_ERR_WORKSPACE,
              "router_topk: workspace %zu < %zu bytes", workspace_bytes, mkd_router_workspace_bytes(T, H, E));
  RouterArgs r;
  memset(&r, 0, sizeof(r));
  r.bias = static_cast<const uint16_t*>(w_bias);
  r.T = T; r.E = E; r.K = k; r.mode = mode;
  r.logits_out = router_logits; r.aff_full = expert_affinities; r.idx_out = expert_index;
  r.topk_out = topk_affinities;
  // above 128 tokens the selection runs on 16 tokens per block
  return router_stage(x, x_dtype == MKD_DT_F32, H, w_packed, static_cast<float*>(workspace), r,
                      static_cast<hipStream_t>(stream), T > 128);
}

// ---- router_topk without a caller workspace (mkd_router_topk_static) ----
// The split-K partial logits live in this file-scope device array instead.
// Each GPU the library runs on holds its own copy (2 MiB + 256 B: router_kgrid
// keeps K-slices x experts below 4096, so 128 tokens need less) until the process
// ends; host code must use the per-device address from hipGetSymbolAddress,
// never the array's name.  Every call on one GPU shares that GPU's copy, so
// calls that overlap in time on one GPU race.  Every partial the router GEMM
// writes covers all T x E outputs of its K slice, so nothing needs clearing.
constexpr size_t kRouterScratchFloats = ((size_t)1 << 19) + 64;   // 4096 x 128 partials + 256 B
static __device__ __align__(256) float scratch[kRouterScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device.
int router_scratch(float** out) {
  int dev = -1;
  MKD_TRY(hipGetDevice(&dev), "router_topk_static: hipGetDevice");
  MKD_REQUIRE(dev >= 0 && dev < kMaxDevices, MKD_ERR_UNSUPPORTED,
              "router_topk_static: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    MKD_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "router_topk_static: hipGetSymbolAddress");
    MKD_REQUIRE(p, MKD_ERR_HIP, "router_topk_static: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<float*>(g_scratch_ptr[dev]);
  return MKD_OK;
}
}  // namespace

int mkd_router_topk_static(const void* x, int x_dtype, int T, int H, const void* w_packed, int E,
                           const void* w_bias, float* router_logits, float* expert_affinities,
                           int* expert_index, float* topk_affinities, int k, int mode, void* stream) {
  if (int rc = stale_check("mkd_router_topk_static")) return rc;
  MKD_REQUIRE(T > 0 && T <= 128, MKD_ERR_INVALID, "router_topk_static: T %d must be in [1, 128]", T);
  MKD_REQUIRE(E > 0 && E <= 512, MKD_ERR_INVALID, "router_topk_static: E %d must be in [1, 512]", E);
  MKD_REQUIRE(H > 0, MKD_ERR_INVALID, "router_topk_static: H %d must be > 0", H);
  const size_t need = mkd_router_workspace_bytes(T, H, E);
  MKD_REQUIRE(need <= sizeof(scratch), MKD_ERR_UNSUPPORTED,
              "router_topk_static: T=%d H=%d E=%d needs %zu bytes of scratch, above the %zu-byte maximum",
              T, H, E, need, sizeof(scratch));
  float* parts = nullptr;
  if (int rc = router_scratch(&parts)) return rc;
  return mkd_router_topk(x, x_dtype, T, H, w_packed, E, w_bias, router_logits, expert_affinities,
                         expert_index, topk_affinities, k, mode, parts, sizeof(scratch), stream);
}

size_t mkd_moe_workspace_bytes(int T, int H, int E, int I, int K) {
  Carver c{nullptr, 0};
  carve_moe(c, T, H, E, I, K);
  return c.used;
}

}  // extern "C"

namespace {
int moe_entry(const mkd_moe_args* p, void* workspace, size_t workspace_bytes, void* stream,
              bool tiled) {
  MKD_REQUIRE(p, MKD_ERR_NULL, "moe_tkg: null args");
  MKD_REQUIRE(p->hidden && p->gate_up_packed && p->down_packed && p->expert_index && p->output,
              MKD_ERR_NULL, "moe_tkg: null pointer");
  if (tiled) {
    MKD_REQUIRE(p->T > 0 && p->T <= 65535 && (long long)p->T * p->K <= (1 << 23), MKD_ERR_INVALID,
                "moe_prefill: T %d must be in [1, 65535] with T*K <= 2^23", p->T);
    MKD_REQUIRE(p->weight_format == 0, MKD_ERR_UNSUPPORTED, "moe_prefill: bf16 expert weights only");
    MKD_REQUIRE(gemm_tile_supported(2 * p->I, p->H, EPI_SWIGLU_BF16) &&
                    gemm_tile_supported(p->H, p->I, EPI_SCALE_F32),
                MKD_ERR_UNSUPPORTED, "moe_prefill: H (%d) and I (%d) must be multiples of 32", p->H, p->I);
    MKD_REQUIRE(tile_offsets_ok(p->T, p->H, 2LL * p->I, p->H) &&
                    tile_offsets_ok((long long)p->T * p->K, p->I, p->H, p->I),
                MKD_ERR_UNSUPPORTED,
                "moe_prefill: T=%d K=%d H=%d I=%d puts an operand past 2^31 bytes (32-bit buffer offsets)",
                p->T, p->K, p->H, p->I);
  } else {
    MKD_REQUIRE(p->T > 0 && p->T <= 128, MKD_ERR_INVALID,
                "moe_tkg: only T <= 128 tokens are supported in selective mode, got %d", p->T);
  }
  MKD_REQUIRE(p->E > 0 && p->E <= 512 && p->K >= 1 && p->K <= 8 && p->K <= p->E, MKD_ERR_INVALID,
              "moe_tkg: bad E=%d / K=%d", p->E, p->K);
  if (p->weight_format == MKD_FP8_E4M3) {
    MKD_REQUIRE(!tiled, MKD_ERR_UNSUPPORTED, "moe_prefill: bf16 expert weights only");
    MKD_REQUIRE(p->H % 32 == 0 && p->I % 32 == 0, MKD_ERR_INVALID,
                "moe_tkg: fp8 experts need H (%d) and I (%d) multiples of 32", p->H, p->I);
  } else if (p->weight_format) {
    if (int rc = check_mx_dims(2 * p->I, p->H, 2)) return rc;
    if (int rc = check_mx_dims(p->H, p->I, 1)) return rc;
  } else {
    if (int rc = check_gemm_dims(2 * p->I, p->H, 2)) return rc;
    if (int rc = check_gemm_dims(p->H, p->I, 1)) return rc;
  }
  MKD_REQUIRE(p->scaling_mode == MKD_SCALE_NONE || p->scaling_mode == MKD_SCALE_POST,
              MKD_ERR_UNSUPPORTED, "moe_tkg: only NO_SCALE and POST_SCALE affinity scaling are supported");
  MKD_REQUIRE(!(p->scaling_mode == MKD_SCALE_POST && !p->expert_affinities && !p->slot_weights),
              MKD_ERR_NULL, "moe_tkg: POST_SCALE needs expert_affinities");
  MKD_REQUIRE(p->activation >= MKD_ACT_SILU && p->activation <= MKD_ACT_GELU_TANH, MKD_ERR_UNSUPPORTED,
              "moe_tkg: unsupported activation %d", p->activation);
  MKD_REQUIRE(p->weight_format == 0 || p->weight_format == MKD_MX_E4M3 ||
                  p->weight_format == MKD_MX_E2M1 || p->weight_format == MKD_FP8_E4M3, MKD_ERR_INVALID,
              "moe_tkg: unknown weight_format %d", p->weight_format);
  if (p->weight_format) {
    MKD_REQUIRE(p->gate_up_scales && p->down_scales, MKD_ERR_NULL,
                "moe_tkg: MX / fp8 weights need their scales");
    MKD_REQUIRE(!p->round_qwen, MKD_ERR_UNSUPPORTED, "moe_tkg: round_qwen applies to bf16 weights only");
  }
  MKD_REQUIRE(workspace, MKD_ERR_NULL, "moe_tkg: null workspace");
  Carver c{static_cast<char*>(workspace), workspace_bytes};
  MoeWs w = carve_moe(c, p->T, p->H, p->E, p->I, p->K);
  MKD_REQUIRE(c.ok, MKD_ERR_WORKSPACE, "moe_tkg: workspace %zu < %zu bytes", workspace_bytes, c.used);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int TK = p->T * p->K;
  if (p->slot_weights) {
    hipLaunchKernelGGL(copy_slot_weights, dim3((TK + 255) / 256), dim3(256), 0, s, p->slot_weights, TK, w.slot_w);
  } else {
    hipLaunchKernelGGL(gather_slot_weights, dim3((TK + 255) / 256), dim3(256), 0, s,
                       p->scaling_mode == MKD_SCALE_POST ? p->expert_affinities : nullptr,
                       p->expert_index, p->T, p->E, p->K, w.slot_w);
  }
  MKD_TRY(hipGetLastError(), "slot weights");
  return moe_core(static_cast<const uint16_t*>(p->hidden), p->gate_up_packed, p->down_packed,
                  p->expert_index, w.slot_w, static_cast<const uint16_t*>(p->gate_up_bias),
                  static_cast<const uint16_t*>(p->down_bias),
                  static_cast<const uint16_t*>(p->residual), static_cast<uint16_t*>(p->output),
                  p->output_f32, p->T, p->H, p->E, p->I, p->K, p->activation, p->alpha,
                  p->gate_hi, p->gate_lo, p->up_hi, p->up_lo, p->round_qwen, w, s, true,
                  p->weight_format, p->gate_up_scales, p->down_scales, tiled);
}
}  // namespace

extern "C" {

int mkd_moe_tkg(const mkd_moe_args* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = stale_check("mkd_moe_tkg")) return rc;
  return moe_entry(p, workspace, workspace_bytes, stream, false);
}

int mkd_moe_prefill(const mkd_moe_args* p, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = stale_check("mkd_moe_prefill")) return rc;
  return moe_entry(p, workspace, workspace_bytes, stream, true);
}

int mkd_quantize_mx(const void* x, int x_dtype, int rows, int k, int ldx, int fmt, void* codes,
                    void* scales, int k_pad, void* stream) {
  if (int rc = stale_check("mkd_quantize_mx")) return rc;
  MKD_REQUIRE(x && codes && scales, MKD_ERR_NULL, "quantize_mx: null pointer");
  MKD_REQUIRE(x_dtype == MKD_DT_BF16 || x_dtype == MKD_DT_F32, MKD_ERR_INVALID, "quantize_mx: bad dtype");
  MKD_REQUIRE(fmt == MKD_MX_E4M3 || fmt == MKD_MX_E2M1, MKD_ERR_INVALID, "quantize_mx: bad format %d", fmt);
  MKD_REQUIRE(rows > 0 && k > 0 && k % 32 == 0 && k_pad >= k && k_pad % 128 == 0, MKD_ERR_INVALID,
              "quantize_mx: need rows > 0, k %% 32 == 0, k_pad >= k, k_pad %% 128 == 0 (rows=%d k=%d k_pad=%d)",
              rows, k, k_pad);
  const int vec = x_dtype == MKD_DT_F32 ? 4 : 8;   // elements per 16 bytes
  MKD_REQUIRE(ldx >= k && ldx % vec == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(codes) & 15) == 0, MKD_ERR_INVALID,
              "quantize_mx: rows must be 16-byte aligned (ldx=%d)", ldx);
  MKD_TRY(mx_quantize_launch(x, x_dtype == MKD_DT_F32, rows, k, ldx, fmt, static_cast<uint8_t*>(codes),
                             static_cast<uint8_t*>(scales), k_pad, static_cast<hipStream_t>(stream)),
          "quantize_mx launch");
  return MKD_OK;
}

size_t mkd_packed_mx_bytes(int groups, int n, int k, int fmt) {
  if (groups <= 0 || n <= 0 || k <= 0 || (fmt != MKD_MX_E4M3 && fmt != MKD_MX_E2M1)) return 0;
  return (size_t)mx_packed_code_bytes(groups, n, k, fmt);
}

size_t mkd_packed_mx_scale_bytes(int groups, int n, int k) {
  if (groups <= 0 || n <= 0 || k <= 0) return 0;
  return (size_t)mx_packed_scale_bytes(groups, n, k);
}

int mkd_pack_mx_weights(const void* codes, const void* scales, void* dst, void* dst_scales,
                        int groups, int n, int k, long long g_stride, long long row_stride,
                        long long s_g_stride, long long s_row_stride, int fmt,
                        int interleave_half, void* stream) {
  if (int rc = stale_check("mkd_pack_mx_weights")) return rc;
  MKD_REQUIRE(codes && scales && dst && dst_scales, MKD_ERR_NULL, "pack_mx_weights: null pointer");
  MKD_REQUIRE(fmt == MKD_MX_E4M3 || fmt == MKD_MX_E2M1, MKD_ERR_INVALID, "pack_mx_weights: bad format %d", fmt);
  MKD_REQUIRE(groups > 0 && n > 0 && k > 0 && k % 32 == 0, MKD_ERR_INVALID,
              "pack_mx_weights: need k %% 32 == 0 (groups=%d n=%d k=%d)", groups, n, k);
  MKD_REQUIRE(interleave_half == 0 || (interleave_half % 16 == 0 && 2 * interleave_half == n),
              MKD_ERR_INVALID, "pack_mx_weights: interleave_half %d must be n/2 and a multiple of 16",
              interleave_half);
  MKD_TRY(mx_pack_launch(static_cast<const uint8_t*>(codes), static_cast<const uint8_t*>(scales),
                         static_cast<uint8_t*>(dst), static_cast<uint8_t*>(dst_scales), groups, n, k,
                         g_stride, row_stride, s_g_stride, s_row_stride, fmt, interleave_half,
                         static_cast<hipStream_t>(stream)),
          "pack_mx_weights launch");
  return MKD_OK;
}

// ---------------------------------------------------------------------------
// attention block
// ---------------------------------------------------------------------------
struct AttnWs {
  uint16_t* hnorm;
  float* qkv;
  uint16_t *attn, *kvn, *prep;
  float *po, *pml;
  uint16_t* xq;               // statically quantised projection inputs (FP8 projections)
  int chunk, n_chunks;
};

// B: query rows (sequences x new tokens each); s_tkg new tokens per sequence
// (the attended window ends s_tkg - 1 positions past S_max at most)
static AttnWs carve_attn(Carver& c, int B, int H, int nq, int nkv, int d, int S_max, int s_tkg = 1) {
  AttnWs w;
  w.chunk = attn_chunk_for(B, nkv, S_max);
  w.n_chunks = (S_max + s_tkg + w.chunk - 1) / w.chunk;
  w.hnorm = c.take<uint16_t>((size_t)B * H);
  // the QKV projection of 17..128 tokens comes as split-K partials, and of a
  // prefill pass as the tiled GEMM's K slices where its tiles leave CUs idle
  const int qparts = std::max({1, gemm_mid_kgrid((nq + 2 * nkv) * d, H, B),
                               B >= 256 ? gemm_tile_kgrid((nq + 2 * nkv) * d, H, B) : 1,
                               (qkv_norm_supported(B, (nq + 2 * nkv) * d, H) &&
                                qkv_norm_extra_tiles((nq + 2 * nkv) * d, H, d)) ? 4 : 1});
  w.qkv = c.take<float>((size_t)qparts * B * (nq + 2 * nkv) * d);
  w.attn = c.take<uint16_t>((size_t)B * nq * d);
  w.kvn = c.take<uint16_t>((size_t)B * 2 * nkv * d);
  w.prep = c.take<uint16_t>((size_t)B * (nq + 2 * nkv) * d);
  w.po = c.take<float>((size_t)B * nq * w.n_chunks * d);
  w.pml = c.take<float>((size_t)B * nq * w.n_chunks * 2);
  w.xq = c.take<uint16_t>((size_t)B * std::max(H, nq * d));
  return w;
}

size_t mkd_attention_workspace_bytes(int B, int H, int nq, int nkv, int d, int S_max) {
  return mkd_attention_workspace_bytes_tkg(B, 1, H, nq, nkv, d, S_max);
}

size_t mkd_attention_workspace_bytes_tkg(int B, int s_tkg, int H, int nq, int nkv, int d, int S_max) {
  const int nt = s_tkg > 1 ? s_tkg : 1;
  Carver c{nullptr, 0};
  carve_attn(c, B * nt, H, nq, nkv, d, S_max, nt);
  return c.used;
}

// o_parts != null: the output projection writes fp32 split-K partials
// [kgrid][B][H_out] there (the caller's next norm folds them into the residual)
// instead of applying the bf16 / residual epilogue.
// join != null (with o_parts, one partial): attention, chunk combine and the
// output projection run as one launch where attn_join_supported allows,
// synchronised through join's flag words.
static int attention_core(const mkd_attention_args* p, AttnWs& w, const int* pos_for_rope,
                          const float* inv_freq, hipStream_t s, float* o_parts = nullptr,
                          int o_kgrid = 1, const QkvNormArgs* qn = nullptr, bool prefill = false,
                          const AttnJoinArgs* join = nullptr) {
  const int qkv_n = (p->nq + 2 * p->nkv) * p->d;
  const int NT = p->s_tkg > 1 ? p->s_tkg : 1;
  const int rows = p->B * NT;            // query tokens: NT consecutive rows per sequence
  int qkv_parts = 1, qkv_split_row = 0;
  // 1. optional RMSNorm
  const void* xin = p->X;
  if (p->rmsnorm_gamma) {
    MKD_TRY(rmsnorm_launch(p->X, 0, static_cast<const uint16_t*>(p->rmsnorm_gamma),
                           w.hnorm, nullptr, rows, p->H, p->H,
                           p->hidden_actual > 0 ? p->hidden_actual : p->H, p->rmsnorm_eps,
                           p->rmsnorm_order, s), "attn rmsnorm");
    xin = w.hnorm;
  }
  // 2. QKV projection (fp32 out); with qn, the residual update and the norm
  // are formed inside the projection kernel itself
  if (qn) {
    QkvNormArgs q = *qn;
    q.w = static_cast<const uint16_t*>(p->w_qkv_packed);
    q.N = qkv_n; q.K = p->H; q.T = rows; q.d = p->d;
    q.y = w.qkv; q.ldy = qkv_n;
    q.part_stride = (long long)rows * qkv_n;
    const int ps = prof_begin(MKD_KCLASS_QKV, s);
    MKD_TRY(qkv_norm_launch(q, s), "qkv + norm");
    prof_end(ps, s);
    if (const int xt = qkv_norm_extra_tiles(qkv_n, p->H, p->d)) {   // the last tiles as K quarters
      qkv_parts = 4;
      qkv_split_row = (qkv_n / 16 - xt) * 16;
    }
  } else if (p->quant_qkv == MKD_QUANT_STATIC) {
    // e4m3 weights, statically quantised input, per-segment dequantisation
    W8Args q;
    memset(&q, 0, sizeof(q));
    q.w = static_cast<const uint8_t*>(p->w_qkv_packed);
    q.x_bf16 = static_cast<const uint16_t*>(xin);
    q.ldx = p->H; q.T = rows; q.N = qkv_n; q.K = p->H;
    q.w_scale = p->w_scale_qkv; q.in_scale = p->in_scale_qkv;
    q.seg0 = p->nq * p->d; q.seg1 = (p->nq + p->nkv) * p->d;
    q.bias = static_cast<const uint16_t*>(p->bias_qkv);
    q.y_f32 = w.qkv; q.ldy = qkv_n;
    const int ps = prof_begin(MKD_KCLASS_QKV, s);
    MKD_TRY(gemm_w8_launch(q, w.xq, s), "qkv (fp8 static)");
    prof_end(ps, s);
  } else {
    GemmArgs g = dense_args(p->w_qkv_packed, xin, p->H, qkv_n, p->H, rows, w.qkv, qkv_n);
    g.bias = static_cast<const uint16_t*>(p->bias_qkv);
    const int ps = prof_begin(MKD_KCLASS_QKV, s);
    // the decode step at 17..128 tokens: activation slices in LDS, K-split partials
    // that the head preparation adds in order
    const int kq = o_parts ? gemm_mid_kgrid(qkv_n, p->H, rows) : 0;
    if (kq) {
      g.part_stride = (long long)rows * qkv_n;
      MKD_TRY(gemm_mid_launch(g, kq, false, s), "qkv (mid)");
      qkv_parts = kq;
    } else {
      if (rows >= 256 && gemm_tile_supported(qkv_n, p->H, EPI_SCALE_F32)) {
        const int kt = gemm_tile_kgrid(qkv_n, p->H, rows);   // a short prefill pass: K slices
        if (kt > 1) {
          g.kgrid = kt;
          g.part_stride = (long long)rows * qkv_n;
          qkv_parts = kt;
        }
      }
      if (int rc = dense_gemm(g, EPI_F32, false, s)) return rc;
    }
    prof_end(ps, s);
  }
  // 3. q/k norm + RoPE + staging
  AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.qkv = w.qkv; a.ld_qkv = qkv_n;
  a.qkv_nparts = qkv_parts; a.qkv_part_stride = (long long)rows * qkv_n;
  a.qkv_split_row = qkv_split_row;
  a.q_norm = static_cast<const uint16_t*>(p->q_norm);
  a.k_norm = static_cast<const uint16_t*>(p->k_norm);
  a.qk_eps = p->qk_eps;
  a.q_norm_post = static_cast<const uint16_t*>(p->q_norm_post);
  a.k_norm_post = static_cast<const uint16_t*>(p->k_norm_post);
  a.qk_post_eps = p->qk_post_eps;
  a.cos = p->cos; a.sin = p->sin; a.inv_freq = inv_freq; a.pos = pos_for_rope;
  a.kv_new = w.kvn;
  a.k_cache = static_cast<uint16_t*>(p->k_cache);
  a.v_cache = static_cast<uint16_t*>(p->v_cache);
  a.cache_h_stride = (long long)p->S_max * p->d;
  a.cache_b_stride = a.cache_h_stride * p->nkv;
  a.n_prior = p->n_prior;
  a.mask = p->mask; a.mask_s_ctx = p->mask_s_ctx;
  a.sink = p->sink;
  a.scale = p->softmax_scale > 0.f ? p->softmax_scale : 1.0f / sqrtf((float)p->d);
  a.round_qwen = p->round_qwen;
  a.B = rows; a.s_tkg = NT; a.nq = p->nq; a.nkv = p->nkv; a.d = p->d; a.S_max = p->S_max;
  a.chunk = w.chunk; a.n_chunks = w.n_chunks;
  a.part_o = w.po; a.part_ml = w.pml;
  // large grids prepare the q / k / v heads once per (sequence, kv head) in a
  // launch of their own; small ones inside every attention block
  a.prep = (NT > 1 || (long long)w.n_chunks * p->nkv * rows > 1024) ? w.prep : nullptr;
  a.attn_out = w.attn;
  a.update_cache = p->update_cache;
  a.write_pos = p->kv_cache_update_idx;
  a.window = p->window;
  a.block_table = p->active_blocks_table;
  a.tbl_stride = p->blocks_per_seq; a.blk_len = p->block_len; a.num_blocks = p->num_blocks;
  if (prefill) {
    // the B tokens belong to one sequence whose cache (or block-table row) the
    // caller's pointers already select
    a.cache_b_stride = 0;
    a.tbl_stride = 0;
    a.prep = w.prep;
    a.prefill = 1;
  }
  // fp8 / transposed-K caches: the option path of attn_kvfmt.hip
  a.kv_fp8 = (p->kv_format & MKD_KV_FP8) != 0;
  a.k_transposed = (p->kv_format & MKD_KV_K_TRANSPOSED) != 0;
  a.k_scale = p->k_scale;
  a.v_scale = p->v_scale;
  const bool kvfmt = a.kv_fp8 || a.k_transposed;
  if (kvfmt) a.prep = w.prep;
  const int rope_mode = p->cos ? 1 : (inv_freq ? 2 : 0);
  if (join && !kvfmt && o_parts && o_kgrid <= 1 && p->w_out_packed && attn_join_supported(a, p->H_out)) {
    AttnJoinArgs j = *join;
    j.w_out = static_cast<const uint16_t*>(p->w_out_packed);
    j.bias = static_cast<const uint16_t*>(p->bias_out);
    j.y = o_parts;
    j.N = p->H_out;
    const int ps = prof_begin(MKD_KCLASS_ATTN, s);
    MKD_TRY(attn_join_launch(a, j, rope_mode, s), j.rw ? "attention + combine + o_proj + router"
                                                        : "attention + combine + o_proj");
    prof_end(ps, s);
    return MKD_OK;
  }
  // the caller left its router to the joined launch
  MKD_REQUIRE(!(join && join->rw), MKD_ERR_UNSUPPORTED,
              "attention: the joined launch with its router stage does not fit this layer");
  if (kvfmt) {
    MKD_REQUIRE(!prefill && a.window == 0, MKD_ERR_UNSUPPORTED,
                "attention: fp8 / transposed-K caches are served by the operator path only");
    const int ps = prof_begin(MKD_KCLASS_ATTN, s);
    MKD_TRY(attn_kvfmt_launch(a, rope_mode, s), "attention (fp8 / transposed-K cache)");
    prof_end(ps, s);
    AttnArgs ac = a;
    ac.update_cache = 0;               // the new rows are stored below, in the cache's format
    MKD_TRY(attn_combine_launch(ac, s), "attention combine");
    MKD_TRY(attn_kvfmt_store_launch(a, s), "kv store (fp8 / transposed-K cache)");
  } else if (prefill && attn_prefill_ok(a)) {
    // a context-encoding pass: query tiles read each cache row once per 16 tokens
    const int ps = prof_begin(MKD_KCLASS_ATTN, s);
    MKD_TRY(attn_prefill_launch(a, rope_mode, s), "prefill attention");
    prof_end(ps, s);
  } else {
    {  // q/k norm + RoPE and split-K attention in one launch
      const int ps = prof_begin(MKD_KCLASS_ATTN, s);
      MKD_TRY(attn_decode_launch(a, rope_mode, s), "attention");
      prof_end(ps, s);
    }
    MKD_TRY(attn_combine_launch(a, s), "attention combine + kv scatter");
  }
  // 5. output projection
  if (p->w_out_packed && p->quant_out == MKD_QUANT_STATIC) {
    MKD_REQUIRE(!o_parts && !p->residual, MKD_ERR_UNSUPPORTED,
                "attention: the fp8 output projection writes bf16 rows without a residual");
    W8Args q;
    memset(&q, 0, sizeof(q));
    q.w = static_cast<const uint8_t*>(p->w_out_packed);
    q.x_bf16 = w.attn;
    q.ldx = p->nq * p->d; q.T = rows; q.N = p->H_out; q.K = p->nq * p->d;
    q.w_scale = p->w_scale_out; q.in_scale = p->in_scale_out;
    q.seg0 = q.seg1 = p->H_out;
    q.bias = static_cast<const uint16_t*>(p->bias_out);
    q.y_bf16 = static_cast<uint16_t*>(p->out); q.ldy = p->H_out;
    const int ps = prof_begin(MKD_KCLASS_OPROJ, s);
    MKD_TRY(gemm_w8_launch(q, w.xq, s), "o_proj (fp8 static)");
    prof_end(ps, s);
  } else if (p->w_out_packed) {
    GemmArgs o = dense_args(p->w_out_packed, w.attn, p->nq * p->d, p->H_out, p->nq * p->d, rows,
                            p->out, p->H_out);
    o.bias = static_cast<const uint16_t*>(p->bias_out);
    o.residual = static_cast<const uint16_t*>(p->residual);
    const int ps = prof_begin(MKD_KCLASS_OPROJ, s);
    if (o_parts) {
      o.y = o_parts;
      o.residual = nullptr;
      o.part_stride = (long long)rows * p->H_out;
      if (o_kgrid > 1 && rows <= 128) {   // 17..128 tokens: K-split partials (gemm_mid_kgrid)
        MKD_TRY(gemm_mid_launch(o, o_kgrid, false, s), "o_proj (mid)");
      } else {
        o.KW = choose_kw(p->nq * p->d, 512, (p->H_out + 15) / 16);
        o.kgrid = o_kgrid;   // prefill passes: K slices of the tiled GEMM (gemm_tile_kgrid)
        if (int rc = dense_gemm(o, EPI_F32, false, s)) return rc;
      }
    } else if (int rc = dense_gemm(o, p->residual ? EPI_RESID_BF16 : EPI_BF16, false, s)) {
      return rc;
    }
    prof_end(ps, s);
  } else {
    MKD_TRY(hipMemcpyAsync(p->out, w.attn, (size_t)rows * p->nq * p->d * 2, hipMemcpyDeviceToDevice, s),
            "attn copy");
  }
  return MKD_OK;
}

static int validate_attn(const mkd_attention_args* p) {
  MKD_REQUIRE(p, MKD_ERR_NULL, "attention: null args");
  MKD_REQUIRE(p->X && p->w_qkv_packed && p->k_cache && p->v_cache && p->n_prior && p->out,
              MKD_ERR_NULL, "attention: null pointer");
  MKD_REQUIRE(p->B > 0 && p->B <= 128, MKD_ERR_INVALID, "attention: B %d must be in [1, 128]", p->B);
  MKD_REQUIRE(p->s_tkg >= 0 && p->s_tkg <= 8, MKD_ERR_UNSUPPORTED, "attention: s_tkg %d must be in [0, 8]",
              p->s_tkg);
  if (p->s_tkg > 1) {
    MKD_REQUIRE(p->B * p->s_tkg <= 128, MKD_ERR_INVALID, "attention: B * s_tkg = %d must be <= 128",
                p->B * p->s_tkg);
    MKD_REQUIRE(p->window == 0 && !p->residual, MKD_ERR_UNSUPPORTED,
                "attention: several new tokens per sequence with a ring cache or a residual are not supported");
    MKD_REQUIRE(!p->update_cache || p->kv_cache_update_idx, MKD_ERR_NULL,
                "attention: several new tokens per sequence need kv_cache_update_idx");
    MKD_REQUIRE(!p->mask || p->mask_s_ctx >= p->s_tkg, MKD_ERR_INVALID,
                "attention: mask_s_ctx %d < s_tkg %d", p->mask_s_ctx, p->s_tkg);
  }
  MKD_REQUIRE(p->d == 64 || p->d == 128, MKD_ERR_UNSUPPORTED, "attention: d_head %d must be 64 or 128", p->d);
  MKD_REQUIRE(p->nkv > 0 && p->nq % p->nkv == 0, MKD_ERR_INVALID, "attention: q_heads %d not a multiple of kv_heads %d", p->nq, p->nkv);
  const int g = p->nq / p->nkv;
  MKD_REQUIRE(g == 1 || g == 2 || g == 4 || g == 8 || g == 16, MKD_ERR_UNSUPPORTED, "attention: GQA group %d unsupported", g);
  MKD_REQUIRE(p->S_max > 0, MKD_ERR_INVALID, "attention: S_max must be > 0");
  if (int rc = check_gemm_dims((p->nq + 2 * p->nkv) * p->d, p->H, 1)) return rc;
  if (p->w_out_packed) {
    if (int rc = check_gemm_dims(p->H_out, p->nq * p->d, 1)) return rc;
  }
  MKD_REQUIRE(!p->residual || p->w_out_packed, MKD_ERR_INVALID, "attention: residual needs W_out");
  MKD_REQUIRE(p->quant_qkv == MKD_QUANT_NONE || p->quant_qkv == MKD_QUANT_STATIC, MKD_ERR_UNSUPPORTED,
              "attention: quant_qkv %d must be NONE or STATIC", p->quant_qkv);
  MKD_REQUIRE(p->quant_out == MKD_QUANT_NONE || p->quant_out == MKD_QUANT_STATIC, MKD_ERR_UNSUPPORTED,
              "attention: quant_out %d must be NONE or STATIC", p->quant_out);
  MKD_REQUIRE(!p->quant_qkv || (p->w_scale_qkv && p->in_scale_qkv), MKD_ERR_NULL,
              "attention: the static fp8 QKV projection needs w_scale_qkv and in_scale_qkv");
  MKD_REQUIRE(!p->quant_out || (p->w_out_packed && p->w_scale_out && p->in_scale_out && !p->residual),
              MKD_ERR_INVALID,
              "attention: the static fp8 output projection needs W_out, w_scale_out, in_scale_out, no residual");
  MKD_REQUIRE((p->kv_format & ~(MKD_KV_FP8 | MKD_KV_K_TRANSPOSED)) == 0, MKD_ERR_INVALID,
              "attention: unknown kv_format bits 0x%x", p->kv_format);
  if (p->kv_format) {
    MKD_REQUIRE(p->window == 0, MKD_ERR_UNSUPPORTED, "attention: fp8 / transposed-K caches with a ring cache");
    MKD_REQUIRE(!(p->kv_format & MKD_KV_K_TRANSPOSED) || !p->active_blocks_table, MKD_ERR_INVALID,
                "attention: a transposed K cache must be flat (attention_block_tkg.py:197-202)");
    MKD_REQUIRE(!(p->kv_format & MKD_KV_FP8) || (p->k_scale && p->v_scale), MKD_ERR_NULL,
                "attention: fp8 KV needs k_scale and v_scale");
  }
  MKD_REQUIRE(!p->mask || p->mask_s_ctx >= 1, MKD_ERR_INVALID, "attention: mask_s_ctx must be >= 1");
  MKD_REQUIRE(!(p->cos && !p->sin), MKD_ERR_NULL, "attention: cos without sin");
  if (p->active_blocks_table) {
    MKD_REQUIRE(p->block_len > 0 && p->blocks_per_seq > 0 && p->num_blocks > 0, MKD_ERR_INVALID,
                "attention: block cache needs block_len, blocks_per_seq, num_blocks > 0");
    MKD_REQUIRE((long long)p->blocks_per_seq * p->block_len == p->S_max, MKD_ERR_INVALID,
                "attention: S_max %d != blocks_per_seq %d * block_len %d", p->S_max,
                p->blocks_per_seq, p->block_len);
  } else {
    MKD_REQUIRE(!p->update_cache || p->kv_cache_update_idx, MKD_ERR_NULL,
                "attention: update_cache needs kv_cache_update_idx");
  }
  return MKD_OK;
}

size_t mkd_packed_fp8_bytes(int G, int N, int K) {
  return (G > 0 && N > 0 && K > 0) ? (size_t)G * N * K : 0;
}

int mkd_pack_fp8_weights(const void* src, void* dst, int G, int N, int K, void* stream) {
  if (int rc = stale_check("mkd_pack_fp8_weights")) return rc;
  MKD_REQUIRE(src && dst, MKD_ERR_NULL, "pack_fp8_weights: null pointer");
  MKD_REQUIRE(G > 0 && N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0, MKD_ERR_INVALID,
              "pack_fp8_weights: G %d > 0, N %d a multiple of 16 and K %d of 32 required", G, N, K);
  MKD_TRY(w8_pack_launch(static_cast<const uint8_t*>(src), G, N, K, static_cast<uint8_t*>(dst),
                         static_cast<hipStream_t>(stream)), "pack fp8 weights");
  return MKD_OK;
}

int mkd_attention_block_tkg(const mkd_attention_args* p, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (int rc = stale_check("mkd_attention_block_tkg")) return rc;
  if (int rc = validate_attn(p)) return rc;
  MKD_REQUIRE(workspace, MKD_ERR_NULL, "attention: null workspace");
  Carver c{static_cast<char*>(workspace), workspace_bytes};
  const int nt = p->s_tkg > 1 ? p->s_tkg : 1;
  AttnWs w = carve_attn(c, p->B * nt, p->H, p->nq, p->nkv, p->d, p->S_max, nt);
  MKD_REQUIRE(c.ok, MKD_ERR_WORKSPACE, "attention: workspace %zu < %zu bytes", workspace_bytes, c.used);
  return attention_core(p, w, nullptr, nullptr, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------------
// multi-layer Qwen3 decode step
// ---------------------------------------------------------------------------
// Persistent layer kernel (layer_mk.hip) plan: possible for the Qwen3 flow with
// bf16 experts and up to kLkMaxB tokens when the shapes and the LDS budget
// allow (its buffers are then always part of the workspace); used when the
// decode path is set to it, otherwise every layer runs the multi-kernel sequence.
static int g_decode_path = 0;   // 0 multi-kernel layers, 1 persistent layer kernel where eligible
static int g_inlaunch_sync = 1;  // 1: stages joined into one launch (in-launch waits) where eligible
// the router stage inside the joined attention launch where that launch runs
static constexpr bool g_router_in_attention = true;

static int lk_device_cus() { return device_cus(); }

struct LkPlan {
  bool on = false;
  int NB = 0, LW = 0, nch_max = 0;
  int LBq = 0, LBo = 0, LBr = 0, LBgu = 0, LBdn = 0;
  int lds_a = 0, lds_b = 0, lds_c = 0, lds_s = 0, lds_total = 0;
};

// Units per block (LB) and per wave (LW) of a split-K stage, over every group count.
// Units per block (LB; row blocks for the down stage, rbm) and per wave (LW)
// of a split-K stage, over every group count.
static void lk_bounds(int NRB, int KB, int ngmax, int NB, int& LB, int& LW, bool rbm = false) {
  LB = LW = 0;
  for (int ng = 1; ng <= ngmax; ++ng) {
    const int F = ng * NRB * KB, span = rbm ? ng * KB : KB;
    const long long fpb = lk_fpb(F, span, NB);
    const long long fpw = (fpb + 7) / 8;
    LB = std::max(LB, (int)((fpb + span - 1) / span + 1));
    LW = std::max(LW, (int)((fpw + KB - 1) / KB + 1));
  }
}

static size_t a16(size_t n) { return (n + 15) & ~size_t(15); }

static LkPlan lk_plan(const mkd_qwen3_model* m, int B) {
  LkPlan p;
  const bool biasless = !m->b_qkv && !m->b_o && !m->sinks && !m->router_bias && !m->gate_up_bias &&
                        !m->down_bias && !m->window && !m->layer_s_max;
  if (m->variant != MKD_VARIANT_QWEN3 || m->expert_format != 0 || !biasless || !m->layer_table) return p;
  if ((long long)m->num_layers * kLkBarriers >= (1LL << 30)) return p;
  if (B < 1 || B > kLkMaxB || (m->d != 64 && m->d != 128) || m->nkv < 1 || m->nq % m->nkv != 0 ||
      m->nq / m->nkv > 16 || m->H % 32 != 0 || m->I % 32 != 0 || m->E % 16 != 0 || m->E > 512 ||
      m->K < 1 || m->K > 8 || m->K > m->E || (m->nq * m->d) % 32 != 0 || !m->q_norm || !m->k_norm ||
      B * m->H > kLkMaxRowElems)
    return p;
  const int NB = std::min(lk_device_cus(), kLkMaxNB);
  if (NB < 8) return p;
  const int ngmax = std::min(m->E, B * m->K);
  const int qkv_n = (m->nq + 2 * m->nkv) * m->d;
  {  // every stage's fragment count fits the kernel's 32-bit partition arithmetic
    const long long frags[] = {(long long)qkv_n / 16 * (m->H / 32), (long long)m->H / 16 * (m->nq * m->d / 32),
                               (long long)m->E / 16 * (m->H / 32), (long long)ngmax * (2 * m->I / 16) * (m->H / 32),
                               (long long)ngmax * (m->H / 16) * (m->I / 32)};
    for (long long f : frags)     // also bounds every divisor of the partition (< 2^20)
      if (f >= (1LL << 20)) return p;
  }
  int lw, LW = 0;
  lk_bounds(qkv_n / 16, m->H / 32, 1, NB, p.LBq, lw); LW = std::max(LW, lw);
  lk_bounds(m->H / 16, m->nq * m->d / 32, 1, NB, p.LBo, lw); LW = std::max(LW, lw);
  lk_bounds(m->E / 16, m->H / 32, 1, NB, p.LBr, lw); LW = std::max(LW, lw);
  lk_bounds(2 * m->I / 16, m->H / 32, ngmax, NB, p.LBgu, lw); LW = std::max(LW, lw);
  lk_bounds(m->H / 16, m->I / 32, ngmax, NB, p.LBdn, lw, true); LW = std::max(LW, lw);
  p.LW = LW;
  p.NB = NB;
  p.nch_max = (m->S_max + 1 + 127) / 128;
  const int gqa = m->nq / m->nkv, d = m->d;
  const size_t A = a16((size_t)2 * B * m->H);
  const size_t Bs = a16(std::max({(size_t)2 * B * std::max(m->H, m->nq * d), (size_t)6 * B * m->H,
                                  (size_t)2 * B * m->K * m->I}));
  const size_t Cs = a16(std::max((size_t)8 * LW * 1024,
                                 (size_t)16 * d * 2 + 2 * d * 2 + 2 * 8 * 16 * 4 + (size_t)8 * gqa * d * 4));
  const size_t S = kLkSelBytes;
  const size_t total = A + Bs + Cs + S;
  if (total + kLkStaticLds > 160 * 1024) return p;
  p.lds_a = 0;
  p.lds_b = (int)A;
  p.lds_c = (int)(A + Bs);
  p.lds_s = (int)(A + Bs + Cs);
  p.lds_total = (int)total;
  p.on = true;
  return p;
}

struct LkWs {
  LkPlan plan;
  float *pq = nullptr, *po = nullptr, *pr = nullptr, *pgu = nullptr, *pdn = nullptr;
  float *apo = nullptr, *aml = nullptr;
  unsigned* bar = nullptr;
};

static LkWs carve_lk(Carver& c, const mkd_qwen3_model* m, int B) {
  LkWs w;
  w.plan = lk_plan(m, B);
  if (!w.plan.on) return w;
  const LkPlan& p = w.plan;
  const size_t ent = (size_t)p.NB * kLkMaxB * 16;
  w.pq = c.take<float>(ent * p.LBq);
  w.po = c.take<float>(ent * p.LBo);
  w.pr = c.take<float>(ent * p.LBr);
  w.pgu = c.take<float>(ent * p.LBgu);
  w.pdn = c.take<float>(ent * p.LBdn);
  w.apo = c.take<float>((size_t)B * m->nq * p.nch_max * m->d);
  w.aml = c.take<float>((size_t)B * m->nq * p.nch_max * 2);
  w.bar = c.take<unsigned>(kLkBarWords);
  return w;
}

// K split of the output projection in the decode step: the LDS-staged GEMM's at
// 17..128 tokens (partials added by the post-attention norm), else none.
// K split of the output projection in the decode step: the LDS-staged GEMM's at
// 17..128 tokens (partials added by the post-attention norm), else none.
static int o_proj_kgrid(const mkd_qwen3_model* m, int B) {
  // a prefill pass (the tiled GEMM): K slices where the output tiles leave CUs idle
  if (B >= 256 && gemm_tile_supported(m->H, m->nq * m->d, EPI_SCALE_F32))
    return gemm_tile_kgrid(m->H, m->nq * m->d, B);
  return std::max(1, gemm_mid_kgrid(m->H, m->nq * m->d, B));
}

struct StepWs {
  AttnWs attn;
  uint16_t *r, *nbf;
  float *nf32, *logits, *cos, *sin, *oparts;
  MoeWs moe;
  LkWs lk;
  // in-launch synchronisation of the joined expert launch: word 0 the timeout
  // word, then per layer that launch's flags (sync_words in all, cleared once
  // per call)
  unsigned* sync;
  int sync_words, layer_words, flag_words, attn_words;
  // the joined attention launch's data-polled exchange at one token: per layer
  // the chunk partials (O, then max / sum) and the projection partials, filled
  // with kPollEmpty at the start of every decode call
  float* poll;
  long long poll_po, poll_pml, poll_y, poll_h, poll_layer;   // words per layer
  float* rss;   // the K-sliced router form's slice sums of squares (one token)
};

static StepWs carve_step(Carver& c, const mkd_qwen3_model* m, int B) {
  StepWs w;
  w.attn = carve_attn(c, B, m->H, m->nq, m->nkv, m->d, m->S_max);
  w.r = c.take<uint16_t>((size_t)B * m->H);
  w.nbf = c.take<uint16_t>((size_t)B * m->H);
  w.nf32 = c.take<float>((size_t)B * m->H);
  w.logits = c.take<float>((size_t)16 * B * m->E);  // split-K partials (<= 16)
  w.rss = c.take<float>(64);
  w.cos = c.take<float>((size_t)B * m->d);
  w.sin = c.take<float>((size_t)B * m->d);
  w.oparts = c.take<float>((size_t)std::max({2, o_proj_kgrid(m, B), B == 1 ? attn_join_y_parts(m->nq) : 1}) *
                           B * m->H);   // o_proj split-K partials
  w.moe = carve_moe(c, B, m->H, m->E, m->I, m->K);
  w.lk = carve_lk(c, m, B);
  w.flag_words = moe_fused_supported(B, m->K, m->E, m->H, m->I) ? moe_fused_flag_words(B, m->K, m->E, m->I) : 0;
  // the joined attention launch's flags (chunk and combine blocks)
  w.attn_words = B <= kJoinMaxB ? attn_join_flag_words(B, m->nq, m->nkv, w.attn.n_chunks, m->H) : 0;
  w.layer_words = w.flag_words + w.attn_words;
  w.sync_words = w.layer_words ? 64 + m->num_layers * w.layer_words : 0;
  w.sync = w.sync_words ? c.take<unsigned>(w.sync_words) : nullptr;
  w.poll = nullptr;
  w.poll_po = w.poll_pml = w.poll_y = w.poll_h = w.poll_layer = 0;
  if (B == 1 && (w.attn_words > 0 || w.flag_words > 0)) {
    if (w.attn_words > 0) {
      w.poll_po = (long long)m->nq * w.attn.n_chunks * m->d;
      w.poll_pml = (long long)m->nq * w.attn.n_chunks * 2;
      w.poll_y = (long long)attn_join_y_parts(m->nq) * m->H;
    }
    if (w.flag_words > 0) w.poll_h = ((long long)m->K * m->I + 1) / 2;   // h rows, bf16 pairs
    w.poll_layer = w.poll_po + w.poll_pml + w.poll_y + w.poll_h;
    w.poll = c.take<float>((size_t)(w.poll_layer * m->num_layers));
  }
  return w;
}

// The decode layers as ONE persistent kernel launch (all layers).
static int decode_layers_lk(const mkd_qwen3_model* m, int B, uint16_t* x, const int* position_ids,
                            const float* cos, const float* sin, StepWs& w, hipStream_t s) {
  const LkPlan& p = w.lk.plan;
  const int ha = m->H_actual > 0 ? m->H_actual : m->H;
  const int qkv_n = (m->nq + 2 * m->nkv) * m->d;
  MKD_TRY(layer_reset_launch(w.lk.bar, s), "layer kernel barrier reset");
  LayerArgs L;
  memset(&L, 0, sizeof(L));
  L.B = B; L.H = m->H; L.nq = m->nq; L.nkv = m->nkv; L.gqa = m->nq / m->nkv; L.d = m->d;
  L.E = m->E; L.K = m->K; L.I = m->I; L.S_max = m->S_max; L.NB = p.NB;
  L.num_layers = m->num_layers;
  L.layers = static_cast<const LkLayer*>(m->layer_table);
  L.eps = m->eps; L.inv_h = 1.0f / (float)ha; L.qk_eps = m->eps;
  L.scale = 1.0f / sqrtf((float)m->d);
  L.q = LkGemv{nullptr, 0, qkv_n / 16, m->H / 32, w.lk.pq, p.LBq, p.LW};
  L.o = LkGemv{nullptr, 0, m->H / 16, m->nq * m->d / 32, w.lk.po, p.LBo, p.LW};
  L.r = LkGemv{nullptr, 0, m->E / 16, m->H / 32, w.lk.pr, p.LBr, p.LW};
  L.gu = LkGemv{nullptr, (long long)2 * m->I * m->H, 2 * m->I / 16, m->H / 32, w.lk.pgu, p.LBgu, p.LW};
  L.dn = LkGemv{nullptr, padded_rows(m->H) * m->I, m->H / 16, m->I / 32, w.lk.pdn, p.LBdn, p.LW};
  L.cache_h_stride = (long long)m->S_max * m->d;
  L.cache_b_stride = L.cache_h_stride * m->nkv;
  L.block_table = m->block_table;
  L.tbl_stride = m->blocks_per_seq; L.blk_len = m->block_len; L.num_blocks = m->num_blocks;
  L.cos = cos; L.sin = sin; L.pos = position_ids;
  L.x = x;
  L.attn_po = w.lk.apo; L.attn_ml = w.lk.aml; L.nch_max = p.nch_max;
  L.attn_out = w.attn.attn;
  L.bar = w.lk.bar;
  L.router_mode = MKD_ROUTER_QWEN;
  L.lds_a = p.lds_a; L.lds_b = p.lds_b; L.lds_c = p.lds_c; L.lds_s = p.lds_s;
  L.lds_total = p.lds_total;
  if (m->route_log) {
    const RouteLogLayout lo = route_log_layout(B, m->E, m->K, m->H);
    L.route_log = static_cast<char*>(m->route_log);
    L.log_stride = lo.stride; L.log_w = lo.w; L.log_logits = lo.logits; L.log_r = lo.r;
  }
  const int ps = prof_begin(MKD_KCLASS_LAYER, s);
  MKD_TRY(layer_kernel_launch(L, s), "persistent decode kernel");
  prof_end(ps, s);
  return MKD_OK;
}

// The largest carve over every batch up to B: a workspace sized for the maximum
// batch serves every smaller batch (whose plan may use the persistent kernel).
size_t mkd_qwen3_workspace_bytes(const mkd_qwen3_model* m, int B) {
  if (!m) return 0;
  size_t most = 0;
  for (int b = 1; b <= std::max(B, 1); ++b) {
    Carver c{nullptr, 0};
    carve_step(c, m, b);
    most = std::max(most, c.used);
  }
  return most;
}

// prefill_seq >= 0: the B tokens are consecutive tokens of sequence prefill_seq
// (context encoding); < 0: one token of each of B sequences (decode).
// The router top-k formed inside the gate/up blocks (a few tokens, bf16 experts,
// the whole gate/up grid resident at once) ...
static bool defer_select_ok(const mkd_qwen3_model* m, int B) {
  const int gmax = m->E < B * m->K ? m->E : B * m->K;
  const int kw = gate_up_kw(m->H, m->I, gmax);
  return router_fused_supported(B, m->E, m->H) && !m->expert_format && kw > 0 &&
         gemm_sel_supported(B, m->K, m->E, m->H / kw) &&
         (long long)((2 * m->I + 31) / 32) * gmax <= 2LL * lk_device_cus();
}
// ... and then gate/up and down joined in one launch (mode 0).
static bool joined_experts_planned(const mkd_qwen3_model* m, int B) {
  const int gmax = m->E < B * m->K ? m->E : B * m->K;
  return g_inlaunch_sync && defer_select_ok(m, B) && moe_fused_supported(B, m->K, m->E, m->H, m->I) &&
         gate_up_kw(m->H, m->I, gmax) * 8 == m->H;
}

// ... and attention, combine and output projection in one launch (mode 0, a
// few tokens): the same test attention_core applies, on the step's shapes.
static bool joined_attention_planned(const mkd_qwen3_model* m, int B) {
  if (!g_inlaunch_sync || B > kJoinMaxB || o_proj_kgrid(m, B) > 1 || !m->w_o) return false;
  AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.B = B; a.nq = m->nq; a.nkv = m->nkv; a.d = m->d; a.S_max = m->S_max;
  a.chunk = attn_chunk_for(B, m->nkv, m->S_max);
  a.n_chunks = (m->S_max + 1 + a.chunk - 1) / a.chunk;
  if ((long long)a.n_chunks * m->nkv * B > 1024) return false;   // the large-grid prep launch
  return attn_join_supported(a, m->H);
}

// ... and with it the router stage (residual add, post-attention norm, router
// GEMM) as that launch's last blocks, where the router's shapes fit both.
static bool router_in_attention_planned(const mkd_qwen3_model* m, int B, int l) {
  if (!g_router_in_attention || !joined_attention_planned(m, B) || !router_fused_supported(B, m->E, m->H) ||
      !attn_join_router_supported(B, m->E, m->H) || m->H % 16)
    return false;
  return l < 0 || !m->layer_s_max || m->layer_s_max[l] == m->S_max;
}

static int decode_layers(const mkd_qwen3_model* m, int B, void* hidden, const int* position_ids,
                         const float* cos, const float* sin, void* workspace,
                         size_t workspace_bytes, void* stream, int prefill_seq) {
  const bool prefill = prefill_seq >= 0;
  MKD_REQUIRE(m && hidden && position_ids && workspace, MKD_ERR_NULL, "decode_layers: null pointer");
  MKD_REQUIRE(m->num_layers > 0, MKD_ERR_INVALID, "decode_layers: num_layers must be > 0");
  const int max_b = prefill ? kMaxPrefillT : 128;
  MKD_REQUIRE(B > 0 && B <= max_b, MKD_ERR_INVALID, "decode_layers: %d tokens must be in [1, %d]", B, max_b);
  MKD_REQUIRE(cos || m->inv_freq, MKD_ERR_NULL, "decode_layers: need cos/sin or inv_freq");
  MKD_REQUIRE(m->E <= 512 && m->K >= 1 && m->K <= 8, MKD_ERR_INVALID, "decode_layers: bad E/K");
  MKD_REQUIRE(m->H % 8 == 0 && m->H <= 8192, MKD_ERR_INVALID, "decode_layers: bad H");
  MKD_REQUIRE(m->expert_format == 0 || m->expert_format == MKD_MX_E4M3 ||
                  m->expert_format == MKD_MX_E2M1, MKD_ERR_INVALID,
              "decode_layers: unknown expert_format %d", m->expert_format);
  if (m->expert_format) {
    MKD_REQUIRE(m->gate_up_scales && m->down_scales, MKD_ERR_NULL, "decode_layers: MX experts need scales");
    if (int rc = check_mx_dims(2 * m->I, m->H, 2)) return rc;
    if (int rc = check_mx_dims(m->H, m->I, 1)) return rc;
  } else {
    if (int rc = check_gemm_dims(2 * m->I, m->H, 2)) return rc;
    if (int rc = check_gemm_dims(m->H, m->I, 1)) return rc;
  }
  if (int rc = check_gemm_dims(m->E, m->H, 1)) return rc;
  if (m->block_table)
    MKD_REQUIRE(m->block_len > 0 && m->num_blocks > 0 &&
                    (long long)m->blocks_per_seq * m->block_len == m->S_max,
                MKD_ERR_INVALID, "decode_layers: S_max %d != blocks_per_seq %d * block_len %d",
                m->S_max, m->blocks_per_seq, m->block_len);
  Carver c{static_cast<char*>(workspace), workspace_bytes};
  StepWs w = carve_step(c, m, B);
  MKD_REQUIRE(c.ok, MKD_ERR_WORKSPACE, "decode_layers: workspace %zu < %zu bytes", workspace_bytes, c.used);
  if (m->route_log)
    MKD_REQUIRE(m->route_log_bytes >= mkd_qwen3_route_log_bytes(m, B), MKD_ERR_WORKSPACE,
                "decode_layers: route log %zu < %zu bytes", m->route_log_bytes,
                mkd_qwen3_route_log_bytes(m, B));
  const RouteLogLayout rlo = route_log_layout(B, m->E, m->K, m->H);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // no tables given: this call forms them (in the persistent path's own launch,
  // or in the one launch that starts the multi-kernel path)
  const bool rope_here = !cos;
  if (rope_here) {
    cos = w.cos;
    sin = w.sin;
  }
  uint16_t* x = static_cast<uint16_t*>(hidden);
  for (int l = 0; l < m->num_layers; ++l)
    MKD_REQUIRE(m->w_qkv[l] && m->w_o[l] && m->router[l] && m->gate_up[l] && m->down[l] &&
                m->k_cache[l] && m->v_cache[l] && m->ln_in[l] && m->ln_post[l] &&
                (!m->expert_format || (m->gate_up_scales[l] && m->down_scales[l])),
                MKD_ERR_NULL, "decode_layers: null weight in layer %d", l);
  if (w.lk.plan.on && g_decode_path == 1 && !prefill) {
    if (rope_here)
      MKD_TRY(rope_table_launch(position_ids, m->inv_freq, B, m->d, w.cos, w.sin, s), "rope table");
    return decode_layers_lk(m, B, x, position_ids, cos, sin, w, s);
  }
  // Qwen3 flow: pre-attention norm (x*rinv)*g, Qwen rounding points, fp32 router
  // input.  GPT-OSS flow: rmsnorm_tkg's (x*g)*rinv with H_actual everywhere,
  // biases, sinks, sliding windows, bf16 router input with logit top-k.
  const bool oss = m->variant == MKD_VARIANT_GPT_OSS;
  const int ha = m->H_actual > 0 ? m->H_actual : m->H;
  const int pre_order = oss ? 0 : 1;
  auto at = [](const void* const* arr, int l) -> const void* { return arr ? arr[l] : nullptr; };
  for (int l = 0; l < m->num_layers; ++l) {
    const int wl = m->window ? m->window[l] : 0;
    const int sl = m->layer_s_max ? m->layer_s_max[l] : m->S_max;
    MKD_REQUIRE(sl > 0 && sl <= m->S_max && wl >= 0 && wl <= sl && (wl == 0 || wl >= 2) &&
                    !(wl && m->block_table),
                MKD_ERR_INVALID, "decode_layers: layer %d window %d / cache rows %d invalid", l, wl, sl);
    // a ring cache of W - 1 prior rows cannot take several tokens' rows before
    // their attention: the later tokens would overwrite rows the earlier ones read
    MKD_REQUIRE(!(prefill && wl && B > 1), MKD_ERR_UNSUPPORTED,
                "prefill_layers: layer %d has a sliding window; prefill it one token per call", l);
  }
  // Small batches (Qwen flow): the MoE finalize and each layer's pre-attention
  // norm are formed inside that layer's QKV projection kernel.  Otherwise layer
  // l's pre-attention norm is produced by the previous layer's MoE finalize (one
  // fused kernel) and layer 0 normalises the input here.
  const int qkv_n = (m->nq + 2 * m->nkv) * m->d;
  const bool fuse_qn = !oss && !m->b_qkv && qkv_norm_supported(B, qkv_n, m->H);
  if (!fuse_qn)
    MKD_TRY(rmsnorm_launch(x, 0, static_cast<const uint16_t*>(m->ln_in[0]), w.attn.hnorm, nullptr, B,
                           m->H, m->H, ha, m->eps, pre_order, s), "pre norm");
  const int o_kgrid = o_proj_kgrid(m, B);
  // the joined expert launch (router select + gate/up + down) where the select
  // is deferred into the gate/up blocks and the shapes fit it
  const bool defer_ok = defer_select_ok(m, B);
  const bool fused_moe = joined_experts_planned(m, B) && w.flag_words > 0;
  const bool join_attn = g_inlaunch_sync && !prefill && w.attn_words > 0 && o_kgrid <= 1;
  {
    // the RoPE tables, the in-launch sync words and the data-polled exchange
    // words (chunk partials only up to the position), one launch
    DecodeBeginArgs db;
    memset(&db, 0, sizeof(db));
    db.pos = position_ids; db.inv_freq = m->inv_freq; db.B = B; db.d = m->d;
    if (rope_here) { db.cos = w.cos; db.sin = w.sin; }
    if (fused_moe || join_attn) { db.sync = w.sync; db.sync_words = w.sync_words; }
    if ((join_attn || fused_moe) && w.poll) {
      db.poll = reinterpret_cast<uint32_t*>(w.poll);
      db.layer_words = w.poll_layer; db.po = w.poll_po; db.pml = w.poll_pml;
      db.layers = m->num_layers; db.nq = w.poll_po ? m->nq : 0; db.n_chunks = w.attn.n_chunks; db.D = m->d;
      db.chunk = w.attn.chunk; db.S_max = m->S_max;
    }
    MKD_TRY(decode_begin_launch(db, s), "decode begin (rope tables, sync words, exchange buffers)");
  }
  for (int l = 0; l < m->num_layers; ++l) {
    const int wl = m->window ? m->window[l] : 0;
    const bool mx_experts = m->expert_format == MKD_MX_E4M3 || m->expert_format == MKD_MX_E2M1;
    bool x_mx_ready = false;   // the post-attention norm wrote the experts' MXFP8 input
    mkd_attention_args ap;
    memset(&ap, 0, sizeof(ap));
    ap.X = w.attn.hnorm;                       // already normalised
    ap.w_qkv_packed = m->w_qkv[l];
    ap.bias_qkv = at(m->b_qkv, l);
    ap.q_norm = at(m->q_norm, l); ap.k_norm = at(m->k_norm, l); ap.qk_eps = m->eps;
    ap.cos = cos; ap.sin = sin;
    ap.k_cache = m->k_cache[l]; ap.v_cache = m->v_cache[l];
    // prefill: the caches (or block-table row) of sequence prefill_seq; a windowed
    // layer (one token per call) keeps the decode order -- its ring row still
    // holds the oldest attended position until the attention has read it
    if (prefill && !m->block_table) {
      const size_t seq_off = (size_t)prefill_seq * m->nkv *
                             (size_t)(m->layer_s_max ? m->layer_s_max[l] : m->S_max) * m->d;
      ap.k_cache = static_cast<uint16_t*>(m->k_cache[l]) + seq_off;
      ap.v_cache = static_cast<uint16_t*>(m->v_cache[l]) + seq_off;
    }
    ap.n_prior = position_ids;
    ap.sink = static_cast<const float*>(at(m->sinks, l));
    ap.window = wl;
    ap.update_cache = 1;
    ap.kv_cache_update_idx = (m->block_table || wl) ? nullptr : position_ids;
    ap.active_blocks_table = wl ? nullptr : m->block_table;
    if (prefill && ap.active_blocks_table) ap.active_blocks_table += (size_t)prefill_seq * m->blocks_per_seq;
    ap.blocks_per_seq = m->blocks_per_seq; ap.block_len = m->block_len; ap.num_blocks = m->num_blocks;
    ap.w_out_packed = m->w_o[l];
    ap.bias_out = at(m->b_o, l);
    ap.out = w.r;
    ap.B = B; ap.H = m->H; ap.H_out = m->H; ap.nq = m->nq; ap.nkv = m->nkv; ap.d = m->d;
    ap.S_max = m->layer_s_max ? m->layer_s_max[l] : m->S_max;
    ap.round_qwen = oss ? 0 : 1;
    QkvNormArgs qn = {};
    if (fuse_qn) {
      qn.r = l == 0 ? x : w.r;                 // previous layer's post-attention residual
      qn.ld_r = m->H;
      qn.dsum = l == 0 ? nullptr : w.moe.ybuf; // its expert outputs (already weighted)
      qn.dK = m->K; qn.ds_row = (long long)m->K * m->H; qn.ds_k = m->H;
      qn.gamma = static_cast<const uint16_t*>(m->ln_in[l]);
      qn.eps = m->eps; qn.inv_h = 1.0f / (float)ha;
      qn.resid_out = l == 0 ? nullptr : x;
    }
    unsigned* lsync = w.sync ? w.sync + 64 + (size_t)l * w.layer_words : nullptr;
    AttnJoinArgs ja = {};
    ja.flags = lsync ? lsync + w.flag_words : nullptr;
    ja.err = w.sync;
    // the residual add, post-attention norm and router GEMM as the joined
    // attention launch's last blocks (replacing the router launch)
    const bool router_join = join_attn && lsync && router_in_attention_planned(m, B, l);
    // one token: the router blocks each own a K slice (their partial logits lack
    // the 1 / rms factor, applied -- with the experts' input -- by the expert
    // launch), where that launch is the joined one with the split routing
    const int kslice = (router_join && fused_moe && defer_ok && !oss && !m->router_bias && w.poll && w.poll_po)
                           ? attn_join_kslice_parts(B, m->nq, m->nkv, m->d,
                                                    m->layer_s_max ? m->layer_s_max[l] : m->S_max, m->E, m->H)
                           : 0;
    if (router_join) {
      ja.rx = static_cast<const uint16_t*>(x);
      ja.rgamma = static_cast<const uint16_t*>(m->ln_post[l]);
      ja.rw = static_cast<const uint16_t*>(m->router[l]);
      ja.rparts = w.logits;
      ja.rresid = w.r; ja.rhnorm = w.nbf;
      ja.reps = m->eps; ja.rinv_h = 1.0f / (float)ha;
      ja.E = m->E; ja.rx_f32 = oss ? 0 : 1;
      ja.rss = kslice ? w.rss : nullptr;
      if (w.poll && w.poll_po) {
        float* pl = w.poll + (size_t)l * w.poll_layer;
        ja.poll_po = pl;
        ja.poll_pml = pl + w.poll_po;
        ja.poll_y = pl + w.poll_po + w.poll_pml;
      }
    }
    if (int rc = attention_core(&ap, w.attn, position_ids, nullptr, s, w.oparts, o_kgrid,
                                fuse_qn ? &qn : nullptr, prefill && !wl,
                                join_attn && lsync ? &ja : nullptr))
      return rc;
    // router (split-K GEMM) + top-k + expert groups in one select launch: Qwen
    // fp32 input and fused flow; GPT-OSS bf16 input, biased logits, top-k then
    // softmax over the top-k (router_topk.py:868-887)
    RouterArgs ra;
    memset(&ra, 0, sizeof(ra));
    ra.T = B; ra.E = m->E; ra.K = m->K; ra.mode = oss ? 0 : MKD_ROUTER_QWEN;
    ra.bias = static_cast<const uint16_t*>(at(m->router_bias, l));
    ra.idx_out = w.moe.idx; ra.slot_w = w.moe.slot_w;
    char* rec = m->route_log ? static_cast<char*>(m->route_log) + (size_t)l * rlo.stride : nullptr;
    if (rec) {   // this layer's routing record
      ra.idx_out = reinterpret_cast<int*>(rec + rlo.idx);
      ra.topk_out = reinterpret_cast<float*>(rec + rlo.w);
      ra.logits_out = reinterpret_cast<float*>(rec + rlo.logits);
    }
    ra.n_groups = w.moe.n_groups; ra.grp_expert = w.moe.grp_expert;
    ra.grp_count = w.moe.grp_count; ra.grp_offset = w.moe.grp_offset;
    ra.pair_token = w.moe.pair_token; ra.pair_slot = w.moe.pair_slot;
    RouterArgs sel;
    bool defer_sel = false;
    if (router_join) {
      // the partial logits came from the attention launch
      sel = ra;
      sel.parts = w.logits;
      sel.nparts = kslice ? kslice : attn_join_router_parts(m->H);
      sel.part_stride = (long long)B * m->E;
      if (kslice) {
        sel.ss_parts = w.rss;
        sel.nss = kslice;
        sel.ss_eps = m->eps;
        sel.ss_inv_h = 1.0f / (float)ha;
      }
      defer_sel = defer_ok;
      if (!defer_sel) MKD_TRY(router_select_launch(sel, s), "router select");
    } else if (router_fused_supported(B, m->E, m->H)) {
      // the router top-k inside the gate/up blocks: each block pays the selection
      // before its weight loads, so only when the whole grid is resident at once
      // (two blocks per CU); measured at 4 tokens (1536 blocks) the select launch
      // is cheaper than three rounds of in-block selection
      defer_sel = defer_ok;
      // a few tokens: the residual add and post norm are folded into the router
      // GEMM (each block forms the row norms itself), then the select launch
      RouterFusedArgs fa = {};
      fa.r = ra;
      fa.r.parts = w.logits;
      fa.x = x; fa.o = w.oparts;
      fa.gamma = static_cast<const uint16_t*>(m->ln_post[l]);
      fa.eps = m->eps; fa.inv_h = 1.0f / (float)ha; fa.H = m->H;
      fa.resid_out = w.r; fa.hnorm = w.nbf;
      fa.w = static_cast<const uint16_t*>(m->router[l]);
      fa.x_f32 = oss ? 0 : 1;
      const int ps = prof_begin(MKD_KCLASS_ROUTER, s);
      MKD_TRY(router_fused_launch(fa, s, defer_sel ? &sel : nullptr), "residual + post norm + router");
      prof_end(ps, s);
    } else {
      // r = bf16(x + bf16(o_proj)) from the split-K partials, then the post-attention
      // RMSNorm: bf16 copy for the experts, fp32 copy for the router
      {
        NormArgs na = {};
        na.x = x; na.ld_in = m->H;
        na.dsum = w.oparts; na.dK = o_kgrid; na.ds_row = m->H; na.ds_k = (long long)B * m->H;
        na.resid_out = w.r;
        na.gamma = static_cast<const uint16_t*>(m->ln_post[l]);
        na.out_bf16 = w.nbf; na.out_f32 = oss ? nullptr : w.nf32;
        na.rows = B; na.H = m->H; na.hidden_actual = ha; na.eps = m->eps; na.order = 0;
        if (mx_experts && m->H % 32 == 0 && g_inlaunch_sync) {   // the experts' MXFP8 input, same launch
          na.mx_codes = w.moe.xq; na.mx_scales = w.moe.xs; na.mx_kpad = mx_pad(m->H);
          x_mx_ready = true;
        }
        MKD_TRY(norm_launch(na, s), "residual + post norm");
      }
      const int ps = prof_begin(MKD_KCLASS_ROUTER, s);
      if (B <= 128) {
        if (int rc = router_stage(oss ? static_cast<const void*>(w.nbf) : w.nf32, !oss, m->H,
                                  m->router[l], w.logits, ra, s))
          return rc;
      } else {
        // a long prefill pass: one router GEMM, the top-k of 16 tokens per
        // block, and the expert groups of all tokens from the indices afterwards
        RouterArgs rs = ra;
        rs.n_groups = nullptr; rs.grp_expert = rs.grp_count = rs.grp_offset = nullptr;
        rs.pair_token = rs.pair_slot = nullptr;
        if (int rc = router_stage(oss ? static_cast<const void*>(w.nbf) : w.nf32, !oss, m->H,
                                  m->router[l], w.logits, rs, s, true))
          return rc;
      }
      prof_end(ps, s);
    }
    if (rec)   // the post-attention residual the router norm read
      MKD_TRY(hipMemcpyAsync(rec + rlo.r, w.r, (size_t)B * m->H * 2, hipMemcpyDeviceToDevice, s),
              "route log residual");
    // > 128 tokens (prefill): groups from the indices, and with bf16 experts the
    // LDS-tiled grouped GEMMs (tens of tokens per expert)
    const bool long_pass = B > 128;
    if (int rc = moe_core(w.nbf, m->gate_up[l], m->down[l], long_pass ? ra.idx_out : nullptr, w.moe.slot_w,
                          static_cast<const uint16_t*>(at(m->gate_up_bias, l)),
                          static_cast<const uint16_t*>(at(m->down_bias, l)), w.r, x, nullptr, B,
                          m->H, m->E, m->I, m->K, oss ? MKD_ACT_SWISH : MKD_ACT_SILU,
                          oss ? m->act_alpha : 1.f, oss ? m->gate_hi : INFINITY,
                          oss ? m->gate_lo : -INFINITY, oss ? m->up_hi : INFINITY,
                          oss ? m->up_lo : -INFINITY, (oss || m->expert_format) ? 0 : 1,
                          w.moe, s, false, m->expert_format,
                          m->expert_format ? m->gate_up_scales[l] : nullptr,
                          m->expert_format ? m->down_scales[l] : nullptr,
                          long_pass && !m->expert_format && gemm_tile_supported(2 * m->I, m->H, EPI_SWIGLU_BF16) &&
                              gemm_tile_supported(m->H, m->I, EPI_SCALE_F32) &&
                              tile_offsets_ok(B, m->H, 2LL * m->I, m->H) &&
                              tile_offsets_ok((long long)B * m->K, m->I, m->H, m->I),
                          defer_sel ? &sel : nullptr,
                          fused_moe ? lsync : nullptr,
                          fused_moe ? w.sync : nullptr,
                          fused_moe && w.poll_h ? reinterpret_cast<uint16_t*>(w.poll + (size_t)l * w.poll_layer + w.poll_po + w.poll_pml + w.poll_y) : nullptr,
                          kslice ? w.r : nullptr,
                          kslice ? static_cast<const uint16_t*>(m->ln_post[l]) : nullptr, x_mx_ready))
      return rc;
    // x = bf16(r + bf16(sum_k expert_k)) fused with the next layer's pre-attention
    // norm (with fuse_qn: the next QKV kernel does both; after the last layer the
    // finalize alone)
    if (!fuse_qn || l + 1 == m->num_layers) {
      NormArgs na = {};
      na.x = w.r; na.ld_in = m->H;
      na.dsum = w.moe.ybuf; na.dK = m->K; na.ds_row = (long long)m->K * m->H; na.ds_k = m->H;
      na.resid_out = x;
      na.gamma = (l + 1 < m->num_layers) ? static_cast<const uint16_t*>(m->ln_in[l + 1]) : nullptr;
      na.out_bf16 = w.attn.hnorm;
      na.rows = B; na.H = m->H; na.hidden_actual = ha; na.eps = m->eps; na.order = pre_order;
      MKD_TRY(norm_launch(na, s), "moe finalize + next norm");
    }
  }
  return MKD_OK;
}

int mkd_qwen3_decode_layers(const mkd_qwen3_model* m, int B, void* hidden,
                            const int* position_ids, const float* cos, const float* sin,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = stale_check("mkd_qwen3_decode_layers")) return rc;
  return decode_layers(m, B, hidden, position_ids, cos, sin, workspace, workspace_bytes, stream, -1);
}

int mkd_qwen3_prefill_layers(const mkd_qwen3_model* m, int seq, int T, void* hidden,
                             const int* position_ids, const float* cos, const float* sin,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = stale_check("mkd_qwen3_prefill_layers")) return rc;
  MKD_REQUIRE(seq >= 0, MKD_ERR_INVALID, "prefill_layers: sequence %d must be >= 0", seq);
  return decode_layers(m, T, hidden, position_ids, cos, sin, workspace, workspace_bytes, stream, seq);
}

int mkd_embed(const int* token_ids, const void* table, void* out, int B, int H, int V,
              void* stream) {
  if (int rc = stale_check("mkd_embed")) return rc;
  MKD_REQUIRE(token_ids && table && out, MKD_ERR_NULL, "embed: null pointer");
  MKD_REQUIRE(B > 0 && H % 8 == 0 && V > 0, MKD_ERR_INVALID, "embed: bad shape");
  MKD_TRY(embed_launch(token_ids, static_cast<const uint16_t*>(table), static_cast<uint16_t*>(out),
                       B, H, V, static_cast<hipStream_t>(stream)), "embed");
  return MKD_OK;
}

size_t mkd_lm_head_workspace_bytes(int B, int H, int V) {
  (void)V;
  Carver c{nullptr, 0};
  c.take<uint16_t>((size_t)B * H);
  c.take<float>((size_t)B * 64);
  c.take<int>((size_t)B * 64);
  return c.used;
}

int mkd_lm_head_greedy(const void* hidden, const void* ln_f, float eps, const void* lm_head_packed,
                       int B, int H, int V, int hidden_actual, int norm_order, float* logits,
                       int* next_tokens, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = stale_check("mkd_lm_head_greedy")) return rc;
  MKD_REQUIRE(hidden && ln_f && lm_head_packed && logits && next_tokens && workspace, MKD_ERR_NULL,
              "lm_head: null pointer");
  MKD_REQUIRE(B > 0 && B <= 128, MKD_ERR_INVALID, "lm_head: B %d must be in [1, 128]", B);
  if (int rc = check_gemm_dims(V, H, 1)) return rc;
  Carver c{static_cast<char*>(workspace), workspace_bytes};
  uint16_t* n = c.take<uint16_t>((size_t)B * H);
  float* sv = c.take<float>((size_t)B * 64);
  int* si = c.take<int>((size_t)B * 64);
  MKD_REQUIRE(c.ok, MKD_ERR_WORKSPACE, "lm_head: workspace %zu < %zu bytes", workspace_bytes, c.used);
  hipStream_t s = static_cast<hipStream_t>(stream);
  MKD_REQUIRE(norm_order == 1 || norm_order == 2, MKD_ERR_INVALID, "lm_head: norm_order %d", norm_order);
  MKD_REQUIRE(hidden_actual <= H, MKD_ERR_INVALID, "lm_head: hidden_actual %d > H %d", hidden_actual, H);
  MKD_TRY(rmsnorm_launch(hidden, 0, static_cast<const uint16_t*>(ln_f), n, nullptr, B, H, H,
                         hidden_actual > 0 ? hidden_actual : H, eps, norm_order, s), "final norm");
  GemmArgs a = dense_args(lm_head_packed, n, H, V, H, B, logits, V);
  {
    const int ps = prof_begin(MKD_KCLASS_LM_HEAD, s);
    if (gemm_kloop_supported(V, H, B)) {   // 17..128 tokens: activation slices in LDS
      MKD_TRY(gemm_kloop_launch(a, s), "lm_head (k-loop)");
    } else if (int rc = dense_gemm(a, EPI_F32, false, s)) {
      return rc;
    }
    prof_end(ps, s);
  }
  MKD_TRY(argmax_launch(logits, B, V, next_tokens, sv, si, s), "argmax");
  return MKD_OK;
}

__global__ void decode_advance_kernel(int* ids, int* pos, const int* nxt, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) {
    ids[b] = nxt[b];
    pos[b] += 1;
  }
}

int mkd_decode_advance(int* token_ids, int* position_ids, const int* next_tokens, int B,
                       void* stream) {
  if (int rc = stale_check("mkd_decode_advance")) return rc;
  MKD_REQUIRE(token_ids && position_ids && next_tokens, MKD_ERR_NULL, "decode_advance: null pointer");
  MKD_REQUIRE(B > 0, MKD_ERR_INVALID, "decode_advance: B must be > 0");
  hipLaunchKernelGGL(decode_advance_kernel, dim3((B + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), token_ids, position_ids, next_tokens, B);
  MKD_TRY(hipGetLastError(), "decode_advance");
  return MKD_OK;
}

int mkd_profile_events(int kernel_class, void* const* start_events, void* const* stop_events,
                       int n) {
  if (kernel_class < 0) {
    g_prof.cls = -1;
    return MKD_OK;
  }
  MKD_REQUIRE(start_events && stop_events, MKD_ERR_NULL, "profile_events: null event array");
  MKD_REQUIRE(n > 0 && n <= 512, MKD_ERR_INVALID, "profile_events: n %d must be in [1, 512]", n);
  for (int i = 0; i < n; ++i) {
    g_prof.start[i] = static_cast<hipEvent_t>(start_events[i]);
    g_prof.stop[i] = static_cast<hipEvent_t>(stop_events[i]);
  }
  g_prof.n = n;
  g_prof.next = 0;
  g_prof.cls = kernel_class;
  return MKD_OK;
}

int mkd_profile_count(void) { return g_prof.next; }

size_t mkd_qwen3_route_log_bytes(const mkd_qwen3_model* m, int B) {
  if (!m || m->num_layers <= 0 || B <= 0) return 0;
  return (size_t)route_log_layout(B, m->E, m->K, m->H).stride * (size_t)m->num_layers;
}

int mkd_qwen3_route_log_layout(const mkd_qwen3_model* m, int B, size_t* offsets) {
  MKD_REQUIRE(m && offsets, MKD_ERR_NULL, "route_log_layout: null pointer");
  MKD_REQUIRE(B > 0, MKD_ERR_INVALID, "route_log_layout: B must be > 0");
  const RouteLogLayout lo = route_log_layout(B, m->E, m->K, m->H);
  offsets[0] = (size_t)lo.idx; offsets[1] = (size_t)lo.w; offsets[2] = (size_t)lo.logits;
  offsets[3] = (size_t)lo.r; offsets[4] = (size_t)lo.stride;
  return MKD_OK;
}

size_t mkd_qwen3_layer_table_bytes(const mkd_qwen3_model* m) {
  return m && m->num_layers > 0 ? sizeof(LkLayer) * (size_t)m->num_layers : 0;
}

int mkd_qwen3_write_layer_table(const mkd_qwen3_model* m, void* table, size_t table_bytes) {
  MKD_REQUIRE(m && table, MKD_ERR_NULL, "write_layer_table: null pointer");
  MKD_REQUIRE(m->num_layers > 0, MKD_ERR_INVALID, "write_layer_table: num_layers must be > 0");
  MKD_REQUIRE(table_bytes >= mkd_qwen3_layer_table_bytes(m), MKD_ERR_WORKSPACE,
              "write_layer_table: %zu < %zu bytes", table_bytes, mkd_qwen3_layer_table_bytes(m));
  std::vector<LkLayer> t((size_t)m->num_layers);
  auto at = [](const void* const* arr, int l) { return arr ? static_cast<const uint16_t*>(arr[l]) : nullptr; };
  for (int l = 0; l < m->num_layers; ++l) {
    t[l].w_qkv = at(m->w_qkv, l); t[l].w_o = at(m->w_o, l);
    t[l].q_norm = at(m->q_norm, l); t[l].k_norm = at(m->k_norm, l);
    t[l].ln_in = at(m->ln_in, l); t[l].ln_post = at(m->ln_post, l);
    t[l].router = at(m->router, l); t[l].gate_up = at(m->gate_up, l); t[l].down = at(m->down, l);
    t[l].k_cache = m->k_cache ? static_cast<uint16_t*>(m->k_cache[l]) : nullptr;
    t[l].v_cache = m->v_cache ? static_cast<uint16_t*>(m->v_cache[l]) : nullptr;
  }
  MKD_TRY(hipMemcpy(table, t.data(), sizeof(LkLayer) * t.size(), hipMemcpyHostToDevice), "layer table");
  return MKD_OK;
}

__global__ void bf16_round_check_kernel(unsigned base_hi, unsigned long long* bad) {
  const uint32_t u = (base_hi << 28) + blockIdx.x * blockDim.x + threadIdx.x;
  const float f = __uint_as_float(u);
  const uint32_t h = f2bf(f);
  bool ok;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    ok = (h & 0x7f80u) == 0x7f80u && (h & 0x7fu) != 0u;   // a NaN stays a NaN
  } else {
    const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    ok = h == r && __float_as_uint(rbf(f)) == (r << 16) &&
         (pack2bf(f, -f) & 0xffffu) == r && (pack2bf(-f, f) >> 16) == r;
  }
  const unsigned long long m = __ballot(!ok);   // the grid covers its range exactly
  if ((threadIdx.x & 63) == 0 && m) atomicAdd(bad, (unsigned long long)__popcll(m));
}

int mkd_selfcheck_bf16_round(unsigned long long* mismatches, void* stream) {
  MKD_REQUIRE(mismatches, MKD_ERR_NULL, "selfcheck_bf16_round: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (unsigned hi = 0; hi < 16; ++hi)   // 2^28 patterns per launch
    hipLaunchKernelGGL(bf16_round_check_kernel, dim3(1u << 20), dim3(256), 0, s, hi, mismatches);
  MKD_TRY(hipGetLastError(), "selfcheck_bf16_round");
  return MKD_OK;
}

int mkd_set_decode_path(int mode) {
  MKD_REQUIRE(mode >= 0 && mode <= 2, MKD_ERR_INVALID, "set_decode_path: mode %d must be 0, 1 or 2", mode);
  g_decode_path = mode == 1 ? 1 : 0;
  g_inlaunch_sync = mode == 2 ? 0 : 1;
  return MKD_OK;
}

int mkd_qwen3_decode_plan(const mkd_qwen3_model* m, int B, int* plan) {
  MKD_REQUIRE(m && plan, MKD_ERR_NULL, "decode_plan: null pointer");
  MKD_REQUIRE(B > 0 && B <= 128, MKD_ERR_INVALID, "decode_plan: %d tokens must be in [1, 128]", B);
  int p = 0;
  if (g_decode_path == 1 && lk_plan(m, B).on) {
    p |= MKD_PLAN_PERSISTENT;
  } else {
    if (joined_experts_planned(m, B)) p |= MKD_PLAN_JOINED_EXPERTS;
    if (joined_attention_planned(m, B)) p |= MKD_PLAN_JOINED_ATTENTION;
    if (router_in_attention_planned(m, B, -1) && (!m->layer_s_max || m->num_layers < 1 ||
                                                  m->layer_s_max[0] == m->S_max))
      p |= MKD_PLAN_ROUTER_IN_ATTENTION;
  }
  *plan = p;
  return MKD_OK;
}

int mkd_qwen3_layer_kernel_status(const mkd_qwen3_model* m, int B, const void* workspace,
                                  size_t workspace_bytes, int* used, int* barrier_timeout) {
  MKD_REQUIRE(m && workspace && used && barrier_timeout, MKD_ERR_NULL, "layer_kernel_status: null pointer");
  Carver c{static_cast<char*>(const_cast<void*>(workspace)), workspace_bytes};
  StepWs w = carve_step(c, m, B);
  MKD_REQUIRE(c.ok, MKD_ERR_WORKSPACE, "layer_kernel_status: workspace %zu < %zu bytes", workspace_bytes, c.used);
  *used = (w.lk.plan.on && g_decode_path == 1) ? 1 : 0;
  *barrier_timeout = 0;
  if (w.lk.plan.on) {
    unsigned e = 0;
    MKD_TRY(hipMemcpy(&e, w.lk.bar + kLkMaxNB, sizeof(e), hipMemcpyDeviceToHost), "read error word");
    *barrier_timeout = e ? 1 : 0;
  }
  if (w.sync) {   // the fused MoE launch's in-launch waits
    unsigned e = 0;
    MKD_TRY(hipMemcpy(&e, w.sync, sizeof(e), hipMemcpyDeviceToHost), "read sync word");
    if (e) *barrier_timeout = 1;
  }
  return MKD_OK;
}

}  // extern "C"
