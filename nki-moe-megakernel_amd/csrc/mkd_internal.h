// Internal launch interfaces shared by the kernel files and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

namespace mkd {

enum Epi { EPI_F32 = 0, EPI_BF16 = 1, EPI_RESID_BF16 = 2, EPI_SWIGLU_BF16 = 3, EPI_SCALE_F32 = 4 };

// Gated expert activations (GemmArgs::act; the values of the public MKD_ACT_*)
constexpr int kActSilu = 0, kActSwish = 1, kActGelu = 2, kActGeluTanh = 3;

struct GemmArgs {
  const uint16_t* w;          // frag-packed weights (group 0)
  long long w_group_stride;   // elements between experts
  const void* x;              // activations, bf16 or fp32 rows
  int ldx;                    // row stride of x (elements)
  int N, K, KW;               // output features, contraction, k per wave
  int T;                      // dense mode: number of token rows
  // grouped (MoE) mode; all null in dense mode
  const int* grp_expert;      // expert id of group g
  const int* grp_count;       // tokens in group g
  const int* grp_offset;      // first pair of group g
  const int* n_groups;        // device scalar: number of live groups
  const int* pair_row;        // x row of pair p
  const int* pair_out_row;    // output row of pair p
  // epilogue
  void* y;                    // output rows
  int ldy;                    // row stride of y (elements)
  const uint16_t* residual;   // EPI_RESID_BF16: residual rows (row stride ldy)
  const float* pair_scale;    // EPI_SCALE_F32: scale per output row (null = 1)
  const uint16_t* bias;       // bf16 bias per logical output column (null = none)
  long long bias_group_stride;  // elements between experts' biases
  // EPI_SWIGLU_BF16 options
  int act;                    // kActSilu, kActSwish (alpha), kActGelu, kActGeluTanh
  float alpha;
  float gate_hi, gate_lo, up_hi, up_lo;
  int round_qwen;             // Qwen rounding points (else one rounding of the product)
  // split of K across blocks (EPI_F32 only): block kb writes its partial sum to
  // y + kb * part_stride; the consumer adds the kgrid partials in order.
  int kgrid;                  // 0 or 1: no split
  long long part_stride;      // elements between partial outputs
  // grouped mode: the block walks every 16 * TN-token tile of its group in
  // turn (launched with one token tile: most groups of a decode batch hold a
  // few tokens, and a grid sized for the largest possible group would be
  // mostly empty blocks)
  int t_loop;
  // MX weights (mx.hip): `w` holds element codes in MX frag order and
  // w_group_stride counts bytes; x holds MXFP8 activation codes (ldx bytes per
  // row) with E8M0 scales x_scale (ldxs bytes per row, one per 32 along K).
  const uint8_t* w_scale;     // packed weight scales (group 0)
  long long w_scale_group_stride;  // bytes between experts' scales
  const uint8_t* x_scale;
  int ldxs;
};

// MX element formats (OCP MX v1.0): codes as in the C ABI (MKD_MX_*).
enum MxFmt { MX_E4M3 = 1, MX_E2M1 = 2 };

// Kernel-dispatch timing.  When `start` is set, the next GEMM or attention
// launch records the two events as part of its own dispatch packet
// (hipExtLaunchKernel), so their elapsed time is that kernel's execution alone,
// and clears the pair.  Host-side state of the library, single-threaded use.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern LaunchTiming g_launch_timing;

// Launch `kernel` on `s`, consuming g_launch_timing when it is set.
template <typename K, typename... Args>
hipError_t timed_launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
  if (g_launch_timing.start) {
    const LaunchTiming t = g_launch_timing;
    g_launch_timing = LaunchTiming{};
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, t.start, t.stop, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
  }
  return hipGetLastError();
}

int choose_kw(int K, int max_kw = 512, long long blocks = 1LL << 40);
int choose_kw_split(int K, int kgrid);
hipError_t gemm_launch(GemmArgs a, int epi, bool xf32, int tn, int groups_max,
                       int max_tokens_per_group, hipStream_t s);
// mx.hip
hipError_t mx_quantize_launch(const void* x, bool x_f32, int rows, int K, int ldx, int fmt,
                              uint8_t* codes, uint8_t* scales, int K_pad, hipStream_t s);
long long mx_packed_code_bytes(int G, int N, int K, int fmt);
long long mx_packed_scale_bytes(int G, int N, int K);
hipError_t mx_pack_launch(const uint8_t* codes, const uint8_t* scales, uint8_t* dst,
                          uint8_t* dst_scales, int G, int N, int K, long long g_stride,
                          long long row_stride, long long s_g_stride, long long s_row_stride,
                          int fmt, int interleave_half, hipStream_t s);
hipError_t gemm_mx_launch(GemmArgs a, int fmt, int epi, int groups_max, int max_tokens_per_group,
                          hipStream_t s);
int choose_kw_mx(int K_pad);
// gemm_mid.hip: dense projection of 17..128 tokens, activation slices staged in
// LDS, fp32 split-K partials (kgrid from gemm_mid_kgrid; 0 = shape not covered)
int gemm_mid_kgrid(int N, int K, int T, int max_parts = 8);
// K split of gemm_mid_launch valid for any token count (more than 128: chunks of 128)
bool gemm_mid_chunked_ok(int K, int kgrid);
hipError_t gemm_mid_launch(GemmArgs a, int kgrid, bool xf32, hipStream_t s);
// the vocabulary projection at 17..128 tokens: whole-K blocks of 128 rows
// looping over K slices staged in LDS (fp32 rows, no partials)
bool gemm_kloop_supported(int N, int K, int T);
hipError_t gemm_kloop_launch(const GemmArgs& a, hipStream_t s);
// gemm_tile.hip: LDS-tiled grouped GEMM (many tokens per expert)
bool gemm_tile_supported(int N, int K, int epi);
// total_rows: the sum of the group sizes (grouped mode: T*K pairs), else the rows.
// Dense mode with a.kgrid > 1: fp32 partials of K slices at y + slice * part_stride.
bool gemm_tile_kgrid_ok(int K, int kgrid);
int gemm_tile_kgrid(int N, int K, int T);   // K slices that fill the CUs (1: none)
hipError_t gemm_tile_launch(const GemmArgs& a, int epi, int groups_max, long long total_rows,
                            hipStream_t s);
int mx_kpad(int K);   // contraction padding of the packed MX layout

hipError_t pack_frag_launch(const uint16_t* src, uint16_t* dst, int G, int N, int K,
                            long long g_stride, long long row_stride, long long col_stride,
                            int interleave_half, hipStream_t s);

// layer_mk.hip: persistent decoder layer (small batches, Qwen3 flow, bf16 experts)
constexpr int kMaxPrefillT = 4096;   // tokens per prefill pass (mkd_qwen3_prefill_layers)
constexpr int kLkMaxB = 4;          // tokens per launch
constexpr int kLkMaxNB = 1024;      // blocks (CUs) per launch
constexpr int kLkBarWords = kLkMaxNB + 64;   // per-block flags + error word (zeroed once per step)
struct LkGemv {                     // one split-K GEMV stage
  const uint16_t* w;                // frag-packed weights (expert 0 / dense)
  long long gstride;                // elements between experts
  int NRB, KB;                      // 16-row blocks per group, 32-wide k blocks
  float* part;                      // [#CUs][LB][kLkMaxB][16] block partials
  int LB, LW;                       // partials per block, reduction slots per wave
};
// Fragments per block of a stage of F fragments over NB blocks: at least
// ceil(KB / 3), so that a unit of KB fragments spans at most 4 blocks.
__host__ __device__ inline int lk_fpb(int F, int KB, int NB) {
  const int a = (F + NB - 1) / NB, b = (KB + 2) / 3;
  return a > b ? a : b;
}
constexpr int kLkMaxRowElems = 16384;   // B * H bound (whole rows held per block)
struct LkLayer {                    // one layer's pointers (device table)
  const uint16_t *w_qkv, *w_o, *q_norm, *k_norm, *ln_in, *ln_post, *router, *gate_up, *down;
  uint16_t *k_cache, *v_cache;
};
struct LayerArgs {
  int B, H, nq, nkv, gqa, d, E, K, I, S_max, NB;
  int num_layers;
  const LkLayer* layers;            // [num_layers] device table
  float eps, inv_h, qk_eps, scale;
  LkGemv q, o, r, gu, dn;           // stage shapes and partial buffers (w set per layer)
  long long cache_b_stride, cache_h_stride;
  const int* block_table;
  int tbl_stride, blk_len, num_blocks;
  const float *cos, *sin;           // [B, d] RoPE tables
  const int* pos;                   // [B] positions (prior length and cache row)
  uint16_t* x;                      // [B, H] residual stream, in and out
  float *attn_po, *attn_ml;         // [B, nq, nch_max, d], [B, nq, nch_max, 2]
  int nch_max;
  uint16_t* attn_out;               // [B, nq * d]
  unsigned* bar;                    // kLkBarWords barrier words
  int router_mode;                  // MKD_ROUTER_* bits
  int lds_a, lds_b, lds_c, lds_s, lds_total;   // dynamic LDS carve (bytes)
  char* route_log;                  // per-layer routing records (RouteLogLayout) or null
  long long log_stride, log_w, log_logits, log_r;
};

// One layer's routing record: idx int32 [B][K], w fp32 [B][K], logits fp32
// [B][E], r bf16 [B][H], each 256-byte aligned; `stride` bytes per layer.
struct RouteLogLayout {
  long long idx, w, logits, r, stride;
};
inline RouteLogLayout route_log_layout(int B, int E, int K, int H) {
  auto up = [](long long n) { return (n + 255) / 256 * 256; };
  RouteLogLayout o;
  o.idx = 0;
  o.w = o.idx + up(4LL * B * K);
  o.logits = o.w + up(4LL * B * K);
  o.r = o.logits + up(4LL * B * E);
  o.stride = o.r + up(2LL * B * H);
  return o;
}
constexpr int kLkBarriers = 7;      // grid barriers per layer
constexpr int kLkSelBytes = 4096;   // LDS of the selection results and small per-wave scratch
constexpr int kLkStaticLds = 1024;  // static LDS of the kernel (router select_small), bound
hipError_t layer_kernel_launch(const LayerArgs& a, hipStream_t s);
hipError_t layer_reset_launch(unsigned* bar, hipStream_t s);

// qkv_norm.hip: QKV projection with the MoE finalize and pre-attention norm folded in
constexpr int kQkvNormMaxT = 4;
struct QkvNormArgs {
  const uint16_t* w;          // packed [N, K] QKV weights
  int N, K, T;
  const uint16_t* r;          // [T, ld_r] bf16 residual before the expert sum
  int ld_r;
  const float* dsum;          // partial rows added to r (null: x = r)
  int dK;
  long long ds_row, ds_k;     // element strides of dsum (token, partial)
  const uint16_t* gamma;      // [K] pre-attention norm weight
  float eps, inv_h;
  uint16_t* resid_out;        // [T, ld_r] x, the new residual stream (or null)
  float* y;                   // [T, ldy] fp32 projections
  int ldy;
  long long part_stride;      // elements between the K-quarter partials of the extra tiles
  int d;                      // head size (the K-quarter split starts on a head boundary)
  int n_main, n_extra;        // set by qkv_norm_launch
};
bool qkv_norm_supported(int T, int N, int K);
hipError_t qkv_norm_launch(const QkvNormArgs& a, hipStream_t s);
// 16-row tiles past one per CU, written as 4 K-quarter partials (0: none); rows
// from (N / 16 - extra) * 16 on then come as 4 partials at part_stride
int qkv_norm_extra_tiles(int N, int K, int d);   // launch_rules.h qkv_extra_tiles_rule on this device

// norm.hip
struct NormArgs {
  const void* x;              // [rows, ld_in] bf16 or fp32
  int x_f32, ld_in;
  const float* dsum;          // optional fp32 partial rows added to x (see norm.hip)
  int dK;                     // number of partial rows per row
  long long ds_row, ds_k;     // element strides of dsum (row, partial)
  uint16_t* resid_out;        // bf16(x + bf16(sum)) when dsum
  const uint16_t* gamma;      // null: no normalisation outputs
  uint16_t* out_bf16;
  float* out_f32;
  int rows, H, hidden_actual;
  float eps, inv_h;
  int order;                  // 0 (x*g)*rinv, 1 (x*rinv)*g, 2 g*bf16(x*rinv)
  // optional: the bf16 output rows also as MXFP8 (the MX experts' input), codes
  // [rows][mx_kpad] and E8M0 scales [rows][mx_kpad / 32], zero past H -- what
  // mx_quantize_launch writes for out_bf16 (H % 32 == 0)
  uint8_t* mx_codes;
  uint8_t* mx_scales;
  int mx_kpad;
};
hipError_t norm_launch(NormArgs a, hipStream_t s);
hipError_t rmsnorm_launch(const void* x, int x_f32, const uint16_t* gamma, uint16_t* out_bf16,
                          float* out_f32, int rows, int H, int ld_in, int hidden_actual,
                          float eps, int order, hipStream_t s);

// attention.hip
struct AttnArgs {
  const float* qkv;           // [B, (nq + 2 nkv) * d] fp32 projections (or null)
  int qkv_nparts;             // split-K partials of qkv (0 / 1: one), summed in order
  long long qkv_part_stride;  // elements between the partials
  int qkv_split_row;          // rows of a token below this come as one partial (0: all split)
  const uint16_t* qkv_bf16;   // same, bf16 (operator path) (or null)
  int ld_qkv;
  const uint16_t* q_norm;     // [d] or null
  const uint16_t* k_norm;     // [d] or null
  float qk_eps;
  const float* cos;           // [B, d] full-width table (contiguous halves duplicated)
  const float* sin;
  const float* inv_freq;      // [d/2] when cos/sin are generated from positions
  const int* pos;             // [B] cache write position == number of prior tokens
  uint16_t* k_cache;          // [B, nkv, S_max, d]
  uint16_t* v_cache;
  long long cache_b_stride, cache_h_stride;  // elements
  const int* n_prior;         // [B] prior positions attended (default pos)
  const uint8_t* mask;        // optional [S_ctx, B, nq] (1 = attend), prior part only
  int mask_s_ctx;
  const float* sink;          // optional [nq]
  float scale;
  int round_qwen;             // 1: emulate the reference's bf16 score rounding
  int B, nq, nkv, d, S_max;
  int chunk;                  // positions per split-K block
  int n_chunks;               // grid z
  float* part_o;              // [B, nq, n_chunks, d]
  float* part_ml;             // [B, nq, n_chunks, 2]
  uint16_t* attn_out;         // [B, nq * d] bf16
  int update_cache;
  const int* write_pos;       // [B] row written (default pos); < 0 -> skip
  uint16_t* kv_new;           // [B, 2, nkv, d] staged new k / v rows
  uint16_t* prep;             // [B, nkv, gqa + 2, d] prepared q / k / v rows (large grids;
                              // null: every attention block prepares them itself)
  // block (paged) KV cache: caches are [num_blocks, blk_len, nkv, d]; position t
  // of sequence b lives in block block_table[b * tbl_stride + t / blk_len] at
  // row t % blk_len; write_pos is then a global row (block * blk_len + row), or
  // derived from pos through the table when write_pos is null.  null = flat.
  const int* block_table;
  int tbl_stride, blk_len, num_blocks;
  // sliding window W > 0 (flat cache of W rows used as a ring): the prior
  // positions attended are the min(pos, W-1) filled rows and the new row goes
  // to row pos % (W-1) -- the GPT-OSS SWA layers (gpt_oss_with_megakernel.py:
  // 669-671, transformer_gpt_oss.py:139-205).  0 = full attention.
  int window;
  // prefill of one sequence's tokens in one step (prep required): the prepared
  // k / v rows are written to the cache before the attention reads it, so each
  // token attends the rows of the earlier tokens of the same step
  int prefill;
  // prefill attention, set by its launch: the CU count when the whole grid is
  // resident at two blocks per CU (block L then shares a CU with block L + CUs),
  // else 0
  int pf_pair;
  // new tokens per sequence (0 / 1: one).  With s_tkg > 1 the B rows are
  // s_tkg consecutive tokens of each of B / s_tkg sequences: row r is token
  // r % s_tkg of sequence r / s_tkg, whose window is its n_prior cache positions
  // followed by the sequence's s_tkg new tokens (their prepared k / v rows come
  // from `prep`, which is then required); the mask is [S_ctx, B / s_tkg, nq,
  // s_tkg] with new token i at slot S_ctx - s_tkg + i, and token s is written
  // at write_pos[sequence] + s
  int s_tkg;
  // per-head RMSNorm after RoPE (x * rsqrt(mean(x^2) + qk_post_eps) * w) of
  // the query heads with q_norm_post, of the key heads with k_norm_post; null:
  // not applied
  const uint16_t* q_norm_post;
  const uint16_t* k_norm_post;
  float qk_post_eps;
  // KV cache formats of the operator's option path (attn_kvfmt.hip; flat or
  // block caches, no ring, no prefill).  kv_fp8: both caches hold float8 e4m3
  // codes (one byte per element, the element offsets above unchanged); a new
  // row is stored as e4m3(clip(x * k_scale, +-240)) (v_scale for V) and the
  // attention uses the stored values as they are.  k_transposed: the flat K
  // cache is [B, nkv, d, S_max] (element (t, i) at i * S_max + t of its head).
  int kv_fp8, k_transposed;
  const float* k_scale;       // fp32 scalars in device memory (kv_fp8)
  const float* v_scale;
};
// rope_mode: 0 none, 1 cos/sin tables, 2 from pos and inv_freq
hipError_t attn_decode_launch(const AttnArgs& a, int rope_mode, hipStream_t s);
// Prefill only: the prepared heads of every token (a.prep) and their k / v
// rows written to the cache -- the first two launches of a prefill pass.
hipError_t attn_prep_write_launch(const AttnArgs& a, int rope_mode, hipStream_t s);
// Prefill attention by query tiles (attn_prefill.hip): the prep / write
// launches, then one kernel writing a.attn_out; no split-K partials.
bool attn_prefill_ok(const AttnArgs& a);
hipError_t attn_prefill_launch(const AttnArgs& a, int rope_mode, hipStream_t s);
hipError_t attn_combine_launch(const AttnArgs& a, hipStream_t s);
int attn_chunk_for(int B, int nkv, int S_max);   // positions per attention block (64/128/256)
// q / k / v head preparation of every (row, kv head) into a.prep (required)
hipError_t attn_prep_launch(const AttnArgs& a, int rope_mode, hipStream_t s);
// Option-path attention over fp8 / transposed-K caches (attn_kvfmt.hip): the
// head preparation, then split-K chunk partials in the layout attn_combine
// merges; the new rows are stored afterwards by attn_kvfmt_store_launch, after
// the combine (kernels run in stream order, so every chunk has read the cache).
hipError_t attn_kvfmt_launch(const AttnArgs& a, int rope_mode, hipStream_t s);
hipError_t attn_kvfmt_store_launch(const AttnArgs& a, hipStream_t s);

// gemm_w8.hip: dense projection with e4m3 weights and static activation
// quantisation (the STATIC paths of qkv_tkg.py / output_projection_tkg.py)
struct W8Args {
  const uint8_t* w;           // frag-packed e4m3 [N/16][K/32][64][8] (w8_pack_launch)
  const uint16_t* x_bf16;     // activations [T, ldx] bf16
  const uint16_t* x;          // the quantised activations (set by the launch)
  int ldx, T, N, K;
  const float* w_scale;       // device: [3] Q / K / V weight scales, or [1]
  const float* in_scale;      // device: [1] input scale
  int seg0, seg1;             // columns < seg0 use w_scale[0], < seg1 [1], else [2]
  const uint16_t* bias;       // [N] bf16 or null
  float* y_f32;               // exactly one of y_f32 / y_bf16
  uint16_t* y_bf16;
  int ldy;
};
hipError_t w8_pack_launch(const uint8_t* src, int G, int N, int K, uint8_t* dst, hipStream_t s);
// quantises x into xq ([T, K] bf16 scratch), then the GEMM (T <= 128)
hipError_t gemm_w8_launch(const W8Args& a, uint16_t* xq, hipStream_t s);
// routed experts with e4m3 weights (moe_tkg FP8 ROW / STATIC): gate/up + gated
// activation -> bf16 h rows (W8_SWIGLU), down x affinity -> fp32 slot rows (W8_SCALE)
enum { W8_SWIGLU = 0, W8_SCALE = 1 };
struct W8GroupArgs {
  const uint8_t* w;           // packed e4m3 [E][N/16][K/32][64][8]
  long long w_group_stride;   // bytes per expert (N * K)
  const uint16_t* x;          // bf16 rows [.., ldx]
  int ldx, N, K;              // N: 2I (gate rows, then up rows) or H
  const int* x_row;           // x row of pair p
  const int* out_row;         // output row (slot) of pair p
  GemmArgs g;                 // routing tables: n_groups, grp_expert, grp_count, grp_offset
  GemmArgs act;               // activation fields (act, alpha, clamps; round_qwen 0)
  const float* col_scale;     // [E][N] fp32 dequantisation scale per output column
  const uint16_t* bias;       // [E][N] bf16 or null
  const float* pair_scale;    // W8_SCALE: affinity per slot (null = 1)
  uint16_t* h;                // W8_SWIGLU: [slots, ldy] bf16 (ldy = I)
  float* y;                   // W8_SCALE: [slots, ldy] fp32 (ldy = H)
  int ldy;
};
hipError_t gemm_w8_grouped_launch(const W8GroupArgs& a, int epi, int groups_max, hipStream_t s);
// Attention, chunk combine and output projection in one launch (attn_mfma.hip,
// attn_joined_kernel): the chunk blocks, then the combine blocks, then the
// projection blocks of one grid, each stage waiting on the flags of the blocks
// it reads; the projection blocks load their weight slices before they wait.
constexpr int kJoinMaxB = 4;         // tokens
struct AttnJoinArgs {
  const uint16_t* w_out;      // [N, nq * d] frag-packed
  const uint16_t* bias;       // [N] or null
  float* y;                   // [B, N] fp32 projection (bias added, no residual)
  int N;
  unsigned* flags;            // attn_join_flag_words() words, zero at launch
  unsigned* err;              // set when a wait ran out
  // Router stage (rw non-null): blocks after the projection blocks wait for
  // every projection block (whose rows are then stored device-coherent and
  // flagged), form r = bf16(x + bf16(y)), the post-attention RMSNorm of r and
  // the router logits' K-split partials -- router_norm_gemm_kernel's work
  // without its launch.
  const uint16_t* rx;         // [B, N] bf16 residual stream (the layer input)
  const uint16_t* rgamma;     // [N] post-attention norm weight
  const uint16_t* rw;         // router weights [E, N], frag-packed
  float* rparts;              // [attn_join_router_parts(N)][B][E] partial logits
  uint16_t* rresid;           // [B, N] r
  uint16_t* rhnorm;           // [B, N] bf16 normalised rows (the expert input)
  float reps, rinv_h;         // norm epsilon, 1 / hidden size it averages over
  int E;
  int rx_f32;                 // 1: router operand fp32 (bf16 hi + lo), 0: bf16
  // K-sliced router form (one token, d = 128, the merge + projection blocks;
  // attn_join_kslice_supported): rss set -> the router blocks each own a K
  // slice of N / kRouterSlices and write rparts [kRouterSlices][E] as
  // sum_k W[e,k] * (r_k * gamma_k) over their slice (no 1 / rms factor), rss
  // [kRouterSlices] the slice's sum of r^2, and their slice of rresid; rhnorm is
  // not written (the consumer forms rinv and the normalised rows itself)
  float* rss;
  // set by attn_join_launch: one token with d = 128 and the router stage merges
  // the chunk partials inside the projection blocks (no combine blocks), which
  // then write o_parts K-split partials of y ([o_parts][B][N]); else 0 and 1
  int mp, o_parts;
  // data-polled exchange (one token, merge + projection form): when poll_po is
  // set, the chunk partials go to poll_po / poll_pml and the projection's
  // partials to poll_y -- buffers of this launch alone, filled with kPollEmpty
  // beforehand -- and the consumers poll the data words themselves instead of
  // waiting for flags and then loading (one coherent round trip per stage fewer)
  float* poll_po;
  float* poll_pml;
  float* poll_y;
  int dpoll;                  // set by attn_join_launch
};
constexpr uint32_t kPollEmpty = 0xffffffffu;   // a NaN no bf16-derived fp32 math produces

// Start of a decode call, one launch (misc.hip): the RoPE tables (cos non-null),
// the in-launch sync words cleared (sync non-null), and every layer's
// data-polled exchange words set to kPollEmpty (poll non-null; one token):
// of the chunk partials [nq][n_chunks][D] (then [nq][n_chunks][2]) only the
// chunks up to the token's position -- the ones the call's attention reads --
// and the rest of each layer's layer_words in full.
struct DecodeBeginArgs {
  const int* pos;             // [B] positions
  const float* inv_freq;      // [d / 2]
  int B, d;
  float* cos;                 // [B, d] or null
  float* sin;
  unsigned* sync;
  int sync_words;
  uint32_t* poll;             // [layers][layer_words] or null
  long long layer_words, po, pml;
  int layers, nq, n_chunks, D, chunk, S_max;
};
hipError_t decode_begin_launch(const DecodeBeginArgs& d, hipStream_t s);
// size of y for attn_join_launch: K-split partials of the merge + projection form
int attn_join_y_parts(int nq);
int attn_join_flag_words(int B, int nq, int nkv, int n_chunks, int N);
bool attn_join_supported(const AttnArgs& a, int N);
int attn_join_router_parts(int N);
bool attn_join_router_supported(int B, int E, int N);
// The K-sliced router form's slices (N / 256) when it applies to one token of
// these shapes (d = 128, 128-position chunks), else 0.
int attn_join_kslice_parts(int B, int nq, int nkv, int d, int S_max, int E, int N);
hipError_t attn_join_launch(const AttnArgs& a, const AttnJoinArgs& j, int rope_mode, hipStream_t s);

// moe.hip
struct RouterArgs {
  const float* parts;         // [nparts][T][E] fp32 partial logits (summed in order)
  int nparts;
  long long part_stride;      // elements between partials
  const uint16_t* bias;       // [E] bf16 or null
  int T, E, K, mode;          // mode: MKD_ROUTER_* bits
  float* logits_out;          // [T, E] or null
  float* aff_full;            // [T, E] or null
  int* idx_out;               // [T, K] or null
  float* topk_out;            // [T, K] or null
  float* slot_w;              // [T*K] or null
  // expert grouping (all null = skip)
  int *n_groups, *grp_expert, *grp_count, *grp_offset, *pair_token, *pair_slot;
  // one token, the K-sliced router form: the partials lack the post-attention
  // norm's 1 / rms, formed here from nss slice sums of squares:
  // rinv = 1 / sqrt(sum * ss_inv_h + ss_eps), logits = rinv * sum of the partials
  const float* ss_parts;
  int nss;
  float ss_eps, ss_inv_h;
};
hipError_t router_select_launch(const RouterArgs& a, hipStream_t s);
// Any number of tokens, no expert grouping (n_groups must be null): 16 tokens
// per block.
hipError_t router_select_multi_launch(const RouterArgs& a, hipStream_t s);
// Residual add + post-attention RMSNorm folded into the split-K router GEMM, then
// the select launch, for a handful of tokens (router_fused_supported).  r.parts
// must hold 16 * T * E floats.
struct RouterFusedArgs {
  RouterArgs r;               // T, E, K, mode, bias, outputs and grouping (parts unused)
  const uint16_t* x;          // [T, H] bf16 residual stream
  const float* o;             // [T, H] fp32 attention output projection
  const uint16_t* gamma;      // [H] post-attention norm weight
  float eps, inv_h;
  int H;
  uint16_t* resid_out;        // [T, H] bf16(x + bf16(o))
  uint16_t* hnorm;            // [T, H] bf16 normalised rows (expert input)
  const uint16_t* w;          // router weights [E, H], frag-packed
  int x_f32;                  // router input: 1 fp32 normalised rows (bf16 hi + lo), 0 bf16
};
bool router_fused_supported(int T, int E, int H);
// With `deferred` set the select launch is left out and the completed
// RouterArgs (partials, count, stride) are returned there for gemm_sel_launch.
hipError_t router_fused_launch(RouterFusedArgs a, hipStream_t s, RouterArgs* deferred = nullptr);
// Grouped gate/up + SwiGLU (frag GEMM, one token tile) whose blocks form the
// router top-k and expert groups themselves from r's partial logits; r's group
// tables and slot weights are written for the down projection.
constexpr int kSelMaxPairs = 64;
// Gate/up + down in one launch (gemm.hip, moe_fused_kernel): the gate/up blocks
// publish their h columns through flags[group * n_gu + tile] (zero at launch),
// the down blocks wait on their group's flags; *err is set when a wait ran out.
int device_cus();                   // compute units of the current device (0 if unknown)
constexpr int kFusedMaxRows = 4;   // tokens of the fused expert launch (rows per group)
constexpr int kFusedHnMax = 2048;  // hidden size of the experts' input formed in LDS (K-sliced router form)
struct MoeFusedArgs {
  GemmArgs gu, dn;
  RouterArgs r;
  unsigned* flags;
  unsigned* err;
  int n_gu, ngu, ndb;   // set by moe_fused_launch
  // data-polled h (one token): when set, the gate/up blocks write h here -- a
  // buffer of this launch alone, filled with kPollEmpty beforehand -- and set no
  // flags; the down blocks poll their h row itself (one coherent round trip
  // fewer than a flag wait followed by the loads)
  uint16_t* poll_h;
  // with r.ss_parts (one token): every block forms the experts' input
  // bf16((r * gamma) * rinv) from the post-attention residual itself (into LDS,
  // the gate/up operand); the first down block also stores it to hn_out
  const uint16_t* hn_r;
  const uint16_t* hn_gamma;
  uint16_t* hn_out;
};
bool moe_fused_supported(int T, int K, int E, int H, int I);
int moe_fused_flag_words(int T, int K, int E, int I);
hipError_t moe_fused_launch(MoeFusedArgs f, int groups_max, hipStream_t s);
bool gemm_sel_supported(int T, int K, int E, int nsplit);
hipError_t gemm_sel_launch(const GemmArgs& a, const RouterArgs& r, int groups_max, hipStream_t s);
// Expert groups of T*K routed slots.  With chunk_off (kRouteChunkCounts ints of
// workspace) and more than kRouteChunk slots, the slots are placed by one block
// per chunk of slots (moe_route_scatter_kernel) instead of by the one block.
constexpr int kRouteChunk = 2048;          // slots per placing block, at least
constexpr int kRouteMaxChunks = 64;
constexpr int kRouteChunkCounts = 8192;    // per-chunk counts: chunks x E <= this
int moe_route_chunk(int TK, int E);        // slots per chunk, 0 = the one-block form
hipError_t moe_route_launch(const int* idx, int T, int K, int E, int* n_groups, int* grp_expert,
                            int* grp_count, int* grp_offset, int* pair_token, int* pair_slot,
                            hipStream_t s, int* chunk_off = nullptr);
hipError_t moe_finalize_launch(const float* ybuf, int T, int K, int H, const uint16_t* resid,
                               uint16_t* out, float* out_f32, hipStream_t s);

// misc.hip
hipError_t embed_launch(const int* ids, const uint16_t* table, uint16_t* out, int B, int H, int V,
                        hipStream_t s);
hipError_t argmax_launch(const float* logits, int B, int V, int* out, float* scratch_val,
                         int* scratch_idx, hipStream_t s);
hipError_t rope_table_launch(const int* pos, const float* inv_freq, int B, int d, float* cos,
                             float* sin, hipStream_t s);

}  // namespace mkd
