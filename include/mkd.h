/*
 * mkd.h -- C ABI of the MI355X (gfx950) MoE decode library (libmkd.so).
 *
 * The library implements the token-generation hot path of a Mixture-of-Experts
 * decoder layer:  rmsnorm_tkg -> attention_block_tkg -> router_topk -> moe_tkg,
 * and the multi-layer decode step that chains them.  Each entry point below
 * names the reference operator it replaces (paths relative to the
 * KevGomes1403/nki-moe-megakernel checkout).
 *
 * Conventions
 *  - Every pointer argument is a DEVICE pointer unless stated otherwise; the
 *    caller owns all buffers.  The library never allocates device memory: any
 *    temporary storage comes from a caller-provided workspace whose size is
 *    reported by the matching *_workspace_bytes() query.  Calls that share
 *    one workspace must not overlap in time.
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).  All
 *    calls are asynchronous and stream-ordered; none synchronise the host.
 *  - Return value: 0 on success, a negative MKD_ERR_* code otherwise; the
 *    message is available from mkd_last_error() (thread-local, host memory).
 *  - bf16 tensors are raw 16-bit bfloat16 bit patterns; fp32 are IEEE floats.
 *  - KV caches are updated IN PLACE (the reference returns them aliased).
 */
#ifndef MKD_H_
#define MKD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MKD_OK 0
#define MKD_ERR_INVALID (-1)     /* bad shape / argument value            */
#define MKD_ERR_NULL (-2)        /* required pointer is NULL               */
#define MKD_ERR_UNSUPPORTED (-3) /* valid request this build cannot do     */
#define MKD_ERR_WORKSPACE (-4)   /* workspace too small                    */
#define MKD_ERR_HIP (-5)         /* HIP runtime / launch failure           */

#define MKD_DT_BF16 0
#define MKD_DT_F32 1

/* Router modes (bit field) -- router_topk.py:519-562 pipeline flags. */
#define MKD_ROUTER_SIGMOID 1   /* act_fn: 0 softmax, 1 sigmoid                     */
#define MKD_ROUTER_PRE_NORM 2  /* router_pre_norm: activation before top-k (ACT1)  */
#define MKD_ROUTER_NORM_TOPK 4 /* norm_topk_prob: L1-renormalise the top-k          */
#define MKD_ROUTER_QWEN 8      /* Qwen fused flow (moe_fused_nki.py:159-276,404-418) */

/* Expert activation (moe_tkg activation_fn) */
#define MKD_ACT_SILU 0
#define MKD_ACT_SWISH 1 /* g * sigmoid(alpha * g), GPT-OSS alpha = 1.702 */
#define MKD_ACT_GELU 2       /* g/2 (1 + erf(g / sqrt 2))                        */
#define MKD_ACT_GELU_TANH 3  /* g/2 (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))    */

/* Affinity scaling (moe_tkg expert_affinities_scaling_mode) */
#define MKD_SCALE_NONE 0
#define MKD_SCALE_POST 1

int mkd_version(void);
const char* mkd_last_error(void);

/* ---------------------------------------------------------------------------
 * rmsnorm_tkg -- replaces nki_kernels/norm/rmsnorm_tkg.py:49 (math :318-454).
 * input [rows, hidden] (bf16 or fp32), gamma [hidden] bf16, output [rows, hidden]
 * in output_dtype.  y = (x * gamma) * rsqrt(sum(x^2) / hidden_actual + eps).
 * hidden % 8 == 0, hidden <= 8192; hidden_actual <= 0 means hidden.
 * ------------------------------------------------------------------------- */
int mkd_rmsnorm_tkg(const void* input, int input_dtype, const void* gamma, void* output,
                    int output_dtype, int rows, int hidden, int hidden_actual, float eps,
                    void* stream);

/* ---------------------------------------------------------------------------
 * Weight repacking into the library's MFMA fragment layout.  Replaces the
 * layout conversion of convert_qwen3_moe_hf_to_neuron_state_dict
 * (megakernels/qwen3_moe/qwen_with_megakernel.py:171-271), which produces the
 * NKI layouts.  Source element (g, n, k) of a logical [groups][n][k] bf16
 * matrix (output feature n, contraction index k) is read at
 *   src + g*g_stride + n*row_stride + k*col_stride      (elements).
 * interleave_half > 0 (fused gate/up) pairs row block j of rows [0, half)
 * with row block j of rows [half, 2*half).  n % 16 == 0, k % 32 == 0.
 * ------------------------------------------------------------------------- */
size_t mkd_packed_bytes(int groups, int n, int k);
int mkd_pack_weights(const void* src, void* dst, int groups, int n, int k, long long g_stride,
                     long long row_stride, long long col_stride, int interleave_half,
                     void* stream);

/* ---------------------------------------------------------------------------
 * Dense decode projection on packed weights: y[r, :] = x[r, :] @ W^T (+ bias)
 * (the matmul of qkv_tkg, nki_kernels/attention/qkv_tkg.py:71, and of
 * output_projection_tkg, nki_kernels/attention/output_projection_tkg.py:66).
 * x [rows, k] (bf16, or fp32 for the router), w packed [n, k], bias [n] bf16
 * or NULL, y [rows, n] in y_dtype.  With `residual` (bf16 [rows, n], y_dtype
 * bf16) the result is bf16(residual + bf16(x @ W^T)).  rows <= 4096 (from 256
 * rows, bf16 x and fp32 y without residual run on the LDS-tiled MFMA GEMM).
 * ------------------------------------------------------------------------- */
int mkd_linear(const void* x, int x_dtype, int ldx, int rows, const void* w_packed, int n, int k,
               const void* bias, void* y, int y_dtype, int ldy, const void* residual,
               void* stream);

/* ---------------------------------------------------------------------------
 * router_topk -- replaces nki_kernels/moe/router_topk.py:69 (x in HBM, [T, H]).
 * logits = x @ w (+ w_bias) in fp32 (w packed from the reference [H, E]
 * layout as n=E, k=H); then the pipeline selected by `mode`.
 * Outputs: router_logits [T, E] fp32, expert_index [T, k] int32,
 * expert_affinities [T, E] fp32 (scattered top-k, or full activation for the
 * (ACT1, topK) pipeline), topk_affinities [T, k] fp32 (may be NULL).
 * E <= 512, k <= 8, T <= 4096 (above 128 tokens the selection runs on 16
 * tokens per block).  Ties resolve to the lowest expert index.
 * workspace: mkd_router_workspace_bytes(T, H, E) bytes (split-K partial logits).
 * ------------------------------------------------------------------------- */
size_t mkd_router_workspace_bytes(int T, int H, int E);
int mkd_router_topk(const void* x, int x_dtype, int T, int H, const void* w_packed, int E,
                    const void* w_bias, float* router_logits, float* expert_affinities,
                    int* expert_index, float* topk_affinities, int k, int mode, void* workspace,
                    size_t workspace_bytes, void* stream);

/* router_topk with no workspace argument.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, outputs and errors as mkd_router_topk for T <= 128; the split-K
 * partial logits go to a device array inside the library (2 MiB + 256 B per
 * GPU, held until the process ends), which covers every such shape (T > 128 is
 * rejected with MKD_ERR_INVALID).  Calls that overlap in time on one GPU share
 * that array and race. */
int mkd_router_topk_static(const void* x, int x_dtype, int T, int H, const void* w_packed, int E,
                           const void* w_bias, float* router_logits, float* expert_affinities,
                           int* expert_index, float* topk_affinities, int k, int mode, void* stream);

/* ---------------------------------------------------------------------------
 * MX (OCP Microscaling v1.0) formats -- the reference's MXFP8 / MXFP4 expert
 * path (selective_expert_mx_impl.py:60-531, down_projection_mx_shard_H.py:
 * 138-211; activations quantised by nisa.quantize_mx, :143-149).
 * Blocks of 32 consecutive elements along the contraction share one E8M0
 * scale byte (2^(byte-127)); elements are E4M3 (1 byte) or E2M1 (4 bits, two
 * per byte, low nibble first).
 *
 * mkd_quantize_mx: rows of x (bf16 or fp32, row stride ldx elements, 16-byte
 * aligned rows, k % 32 == 0) -> codes [rows][k_pad] (e4m3) or [rows][k_pad/2]
 * (e2m1) and scales [rows][k_pad/32]; k_pad % 128 == 0, k_pad >= k, blocks
 * past k are zero (scale byte 0).  Scale X = 2^(floor(log2 amax) - emax),
 * element = RNE(v / X) saturated (448 / 6).
 * mkd_pack_mx_weights: row-major codes [groups][n][k] (e4m3) or
 * [groups][n][k/2] (e2m1) + scales [groups][n][k/32] (byte strides) into the
 * scaled-MFMA fragment order; interleave_half as in mkd_pack_weights.
 * ------------------------------------------------------------------------- */
#define MKD_MX_E4M3 1
#define MKD_MX_E2M1 2
#define MKD_FP8_E4M3 3   /* mkd_moe_args::weight_format: e4m3 experts, per-column scales */
int mkd_quantize_mx(const void* x, int x_dtype, int rows, int k, int ldx, int fmt, void* codes,
                    void* scales, int k_pad, void* stream);
size_t mkd_packed_mx_bytes(int groups, int n, int k, int fmt);
size_t mkd_packed_mx_scale_bytes(int groups, int n, int k);
int mkd_pack_mx_weights(const void* codes, const void* scales, void* dst, void* dst_scales,
                        int groups, int n, int k, long long g_stride, long long row_stride,
                        long long s_g_stride, long long s_row_stride, int fmt,
                        int interleave_half, void* stream);

/* ---------------------------------------------------------------------------
 * moe_tkg (selective experts) -- replaces nki_kernels/moe/moe_tkg.py:56
 * with is_all_expert=False (selective_expert_impl.py:84-519; MX weights:
 * selective_expert_mx_impl.py:60-531).
 * hidden [T, H] bf16; gate_up packed per expert from [E, H, 2, I]
 * (n = 2I interleaved, k = H); down packed per expert from [E, I, H] (n = H,
 * k = I); expert_index [T, K] int32; slot scales: expert_affinities [T, E]
 * fp32 gathered at the selected experts when scaling == MKD_SCALE_POST, else 1.
 * Optional gate_up_bias [E, 2, I] and down_bias [E, H] (bf16).  Clamps are
 * applied when finite (gate <= gate_hi, gate >= gate_lo, up in [up_lo, up_hi]).
 * round_qwen = 1 emulates the Qwen fused kernel's bf16 rounding points
 * (moe_fused_nki.py:506-527).  output [T, H] bf16; with residual (bf16 [T,H])
 * output = bf16(residual + bf16(moe)).  T <= 128.
 * weight_format MKD_MX_E4M3 / MKD_MX_E2M1: the packed weights are MX
 * (mkd_pack_mx_weights, gate/up k = H, down k = I) with their packed scales;
 * the hidden rows and the bf16 SwiGLU output are quantised to MXFP8 (E4M3)
 * before each projection (selective_expert_mx_impl.py:143-149,
 * down_projection_mx_shard_H.py:74-79); round_qwen must be 0.
 * weight_format MKD_FP8_E4M3: the FP8 ROW / STATIC experts (moe_tkg.py:119-131,
 * 296-328): gate_up / down are e4m3 codes packed by mkd_pack_fp8_weights
 * (G = E; gate/up [H, 2I] per expert with the gate columns first, down [I, H]);
 * gate_up_scales / down_scales are fp32 dequantisation scales per expert and
 * output column ([E, 2I]: ROW's [E, 2, I], or STATIC's [E, 2, 1] per half;
 * [E, H]).  The activations stay bf16 (the reference's expert kernels read
 * the input scales of STATIC mode only to select the mode,
 * mlp_tkg_gate_up_projection.py:739, mlp_tkg_down_projection.py:498-502);
 * each output is acc * scale + bias before the activation / affinity.
 * Selective mode only (mkd_moe_tkg); round_qwen must be 0.
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* hidden;          /* [T, H] bf16                    */
  const void* gate_up_packed;  /* E x packed [2I, H]             */
  const void* down_packed;     /* E x packed [H, I]              */
  const float* expert_affinities; /* [T, E] or NULL               */
  const float* slot_weights;   /* [T*K] or NULL (overrides gather) */
  const int* expert_index;     /* [T, K]                         */
  const void* gate_up_bias;    /* [E, 2, I] bf16 or NULL         */
  const void* down_bias;       /* [E, H] bf16 or NULL            */
  const void* residual;        /* [T, H] bf16 or NULL            */
  void* output;                /* [T, H] bf16                    */
  float* output_f32;           /* [T, H] fp32 or NULL            */
  int T, H, E, I, K;
  int scaling_mode;            /* MKD_SCALE_*                    */
  int activation;              /* MKD_ACT_*                      */
  float alpha;                 /* swish alpha                    */
  float gate_hi, gate_lo, up_hi, up_lo; /* +-INFINITY = no clamp */
  int round_qwen;
  int weight_format;           /* 0 bf16, MKD_MX_E4M3, MKD_MX_E2M1, MKD_FP8_E4M3 */
  const void* gate_up_scales;  /* MX: packed scales of gate_up; FP8: fp32 [E, 2 I]  */
  const void* down_scales;     /* MX: packed scales of down; FP8: fp32 [E, H]       */
} mkd_moe_args;
size_t mkd_moe_workspace_bytes(int T, int H, int E, int I, int K);
int mkd_moe_tkg(const mkd_moe_args* args, void* workspace, size_t workspace_bytes, void* stream);
/* moe_prefill: the same selective-expert computation for a prefill-shaped
 * batch (many tokens per expert), on LDS-tiled grouped MFMA GEMMs (256 x 256
 * tiles, operands copied global -> LDS in MFMA order) instead of the
 * weight-streaming decode GEMMs.  The reference's
 * selective mode stops at T <= 128 (moe_tkg.py:388-392) and has no
 * counterpart for this entry; it measures the MFMA-bound regime with the same
 * packed weights and arguments.  bf16 weights only; 1 <= T <= 65535,
 * T*K <= 2^23; H and I multiples of 32.  Workspace: mkd_moe_workspace_bytes. */
int mkd_moe_prefill(const mkd_moe_args* args, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * attention_block_tkg -- replaces nki_kernels/attention/attention_block_tkg.py:83
 * for S_tkg <= 8 new tokens per sequence (s_tkg below), generalised from one kv
 * head per call to nkv >= 1 (GQA).  Stages (attention_block_tkg.py:359-583): optional
 * RMSNorm(X) -> QKV projection (+bias) -> optional pre-RoPE per-head RMSNorm ->
 * RoPE (contiguous halves) -> decode attention over the cache window (+ the
 * active token) with optional 0/1 mask and sink -> in-place KV scatter at
 * kv_cache_update_idx -> output projection (+bias).
 * ------------------------------------------------------------------------- */
typedef struct {
  const void* X;               /* [B, H] bf16                                    */
  const void* rmsnorm_gamma;   /* [H] bf16 or NULL (no pre-attention norm)       */
  float rmsnorm_eps;
  int rmsnorm_order;           /* 0: (x*g)*rinv, 1: (x*rinv)*g                   */
  const void* w_qkv_packed;    /* packed [(nq + 2 nkv) d, H]                     */
  const void* bias_qkv;        /* [(nq + 2 nkv) d] bf16 or NULL                  */
  const void* q_norm;          /* [d] bf16 or NULL                               */
  const void* k_norm;          /* [d] bf16 or NULL                               */
  float qk_eps;
  const float* cos;            /* [B, d] fp32 (halves duplicated) or NULL        */
  const float* sin;            /* [B, d] fp32 or NULL                            */
  void* k_cache;               /* [B, nkv, S_max, d] bf16, updated in place      */
  void* v_cache;
  const int* n_prior;          /* [B] prior positions attended (t < n_prior[b])  */
  const uint8_t* mask;         /* [S_ctx, B, nq] uint8 (1 attend) or NULL        */
  int mask_s_ctx;              /* S_ctx of mask (active token = S_ctx - 1)       */
  const float* sink;           /* [nq] fp32 or NULL                              */
  float softmax_scale;         /* <= 0: 1/sqrt(d)                                */
  int update_cache;
  const int* kv_cache_update_idx; /* [B] row to write; < 0 or >= S_max skips     */
  const void* w_out_packed;    /* packed [H_out, nq d] or NULL (return attention) */
  const void* bias_out;        /* [H_out] bf16 or NULL                           */
  const void* residual;        /* [B, H_out] bf16 or NULL: out = bf16(res + o)   */
  void* out;                   /* [B, H_out] bf16, or [B, nq d] bf16 without W_out */
  int B, H, H_out, nq, nkv, d, S_max;
  int round_qwen;              /* emulate the Qwen kernel's bf16 rounding points */
  /* Block (paged) KV cache, attention_block_tkg.py:199-206, 1473-1685.  When
   * active_blocks_table ([B, blocks_per_seq] int32, device) is set, k_cache /
   * v_cache are [num_blocks, block_len, nkv, d]; position t of sequence b is
   * row t % block_len of block table[b][t / block_len] (entries outside
   * [0, num_blocks) read as zero rows); S_max must be blocks_per_seq *
   * block_len; kv_cache_update_idx holds GLOBAL rows (block * block_len + row,
   * outside [0, num_blocks * block_len) skips) or NULL to derive the row of
   * position n_prior[b] from the table. */
  const int* active_blocks_table;
  int blocks_per_seq, block_len, num_blocks;
  int hidden_actual;           /* pre-attention RMSNorm divisor (X_hidden_dim_actual);
                                  <= 0: H                                         */
  int window;                  /* > 0: the cache is a ring of `window` rows (sliding
                                  window): min(n_prior, window-1) prior rows are
                                  attended and, with kv_cache_update_idx NULL, the
                                  new row goes to n_prior % (window-1)            */
  /* New tokens per sequence, S_tkg of attention_block_tkg.py:151 (0 or 1: one).
   * With s_tkg > 1 (<= 8; B * s_tkg <= 128): X, cos, sin and out hold B * s_tkg
   * rows, row b * s_tkg + s being token s of sequence b; sequence b attends its
   * n_prior[b] cache positions and then its s_tkg new tokens; mask is
   * [S_ctx, B, nq, s_tkg] uint8 with new token i at slot S_ctx - s_tkg + i
   * (attention_tkg.py: the active keys close the window); token s is written
   * at kv_cache_update_idx[b] + s (attention_block_tkg.py:1365-1470, 1611-1685;
   * a global row for a block cache), which is then required.  No ring cache
   * (window) and no residual with s_tkg > 1. */
  int s_tkg;
  /* Post-RoPE per-head RMSNorm, rmsnorm_QK_post_rope_* of
   * attention_block_tkg.py:107-110 (applied at :906-910, :1093-1138): after
   * RoPE, each query head becomes x * rsqrt(mean(x^2) + qk_post_eps) *
   * q_norm_post, each key head the same with k_norm_post, in fp32.  [d] bf16
   * each, or NULL: that norm is not applied. */
  const void* q_norm_post;
  const void* k_norm_post;
  float qk_post_eps;
  /* KV cache format (0: bf16, K as [.., S_max, d]).  MKD_KV_FP8: both caches
   * hold float8 e4m3 codes, one byte per element (k_scale / v_scale of
   * attention_block_tkg.py:133-134, :213-218, :749-754): a new k row is stored
   * as e4m3(clip(k * k_scale, -240, 240)) with round to nearest even
   * (_quantize_to_fp8, :1694-1737), v likewise with v_scale, and the attention
   * uses the stored values as they are -- no dequantisation (attention_tkg.py:
   * 749-821); the new tokens attend their own quantised rows.
   * MKD_KV_K_TRANSPOSED: the flat K cache is [B, nkv, d, S_max]
   * (K_cache_transposed, attention_block_tkg.py:112, :197-202; not with a
   * block table).  V keeps [.., S_max, d].  Neither with a ring cache.
   * k_scale / v_scale: one fp32 value each in device memory (MKD_KV_FP8). */
  int kv_format;
  const float* k_scale;
  const float* v_scale;
  /* Static FP8 quantisation of the projections (quantization_type_qkv / _out =
   * STATIC, attention_block_tkg.py:94-97, :124-127, :179-183, :225-229; qkv_tkg.py:
   * 289-305, 849-862, 946-986; output_projection_tkg.py:185-200, 549-566).  With
   * quant_qkv = MKD_QUANT_STATIC, w_qkv_packed holds e4m3 weights packed by
   * mkd_pack_fp8_weights; the (normalised) input is quantised as
   * x_q = e4m3(clip(x * (1 / in_scale_qkv[0]), -240, 240)) and the projection is
   * (x_q @ W) * (w_scale_qkv[j] * in_scale_qkv[0]) + bias, j = 0 / 1 / 2 for the
   * Q / K / V columns.  quant_out likewise for the output projection with one
   * weight scale w_scale_out[0] (no residual).  Scales: fp32 in device memory. */
  int quant_qkv, quant_out;
  const float* w_scale_qkv;    /* [3] */
  const float* in_scale_qkv;   /* [1] */
  const float* w_scale_out;    /* [1] */
  const float* in_scale_out;   /* [1] */
} mkd_attention_args;
#define MKD_QUANT_NONE 0
#define MKD_QUANT_STATIC 1
#define MKD_KV_FP8 1
#define MKD_KV_K_TRANSPOSED 2
size_t mkd_attention_workspace_bytes(int B, int H, int nq, int nkv, int d, int S_max);
/* e4m3 weights for the static FP8 projections and the FP8 experts: src G
 * contiguous [K, N] code matrices (the reference's [in, out] layouts: W_qkv
 * [H, I], W_out [nq d, H]; experts' gate/up [E, H, 2 I] and down [E, I, H];
 * N % 16 == 0, K % 32 == 0) -> dst of mkd_packed_fp8_bytes(G, N, K) bytes. */
size_t mkd_packed_fp8_bytes(int G, int N, int K);
int mkd_pack_fp8_weights(const void* src, void* dst, int G, int N, int K, void* stream);
/* The same for s_tkg new tokens per sequence (mkd_attention_args::s_tkg). */
size_t mkd_attention_workspace_bytes_tkg(int B, int s_tkg, int H, int nq, int nkv, int d, int S_max);
int mkd_attention_block_tkg(const mkd_attention_args* args, void* workspace,
                            size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Multi-layer Qwen3-MoE decode step -- replaces the megakernel
 * transformer_qwen3_moe_tkg_multilayer (megakernels/qwen3_moe/
 * transformer_qwen.py:68-417, factory :502-505): for each layer
 *   r = x + attn(rmsnorm(x));  x = r + moe(rmsnorm(r))
 * with the residual stream in bf16 and the KV caches updated in place at
 * position_ids[b].  All weight pointers are per-layer arrays in HOST memory
 * holding device pointers to packed weights.
 * ------------------------------------------------------------------------- */
typedef struct {
  int num_layers, H, nq, nkv, d, E, K, I, S_max;
  float eps;
  const void* const* w_qkv;    /* packed [(nq + 2 nkv) d, H]             */
  const void* const* w_o;      /* packed [H, nq d]                       */
  const void* const* q_norm;   /* [d] bf16                               */
  const void* const* k_norm;   /* [d] bf16                               */
  const void* const* ln_in;    /* [H] bf16                               */
  const void* const* ln_post;  /* [H] bf16                               */
  const void* const* router;   /* packed [E, H]                          */
  const void* const* gate_up;  /* E x packed [2I, H] (interleaved)       */
  const void* const* down;     /* E x packed [H, I]                      */
  void* const* k_cache;        /* [B, nkv, S_max, d] bf16                */
  void* const* v_cache;
  const float* inv_freq;       /* [d/2] fp32 device, RoPE inverse freqs  */
  int expert_format;           /* 0 bf16 experts, MKD_MX_E4M3 / MKD_MX_E2M1: MX
                                  experts (mkd_pack_mx_weights), activations
                                  quantised to MXFP8 before each projection */
  const void* const* gate_up_scales;  /* MX: packed scales per layer     */
  const void* const* down_scales;
  /* Block (paged) KV: when block_table ([B, blocks_per_seq] int32, device,
   * shared by all layers) is set, each layer's k_cache / v_cache is
   * [num_blocks, block_len, nkv, d] and S_max = blocks_per_seq * block_len; the
   * new row of sequence b goes to the table slot of position_ids[b]. */
  const int* block_table;
  int blocks_per_seq, block_len, num_blocks;
  /* Model variant.  MKD_VARIANT_QWEN3 (0): the Qwen3 fused-kernel flow above.
   * MKD_VARIANT_GPT_OSS: the stock-kernel flow of transformer_gpt_oss.py:
   * 239-522 -- RMSNorm (x*g)*rsqrt(sum/H_actual + eps) in both places, QKV and
   * o_proj biases, no q/k norm, RoPE from the cos/sin tables, attention sinks,
   * per-layer sliding windows, router top-k on biased bf16-input logits then
   * softmax over the top-k (router_pre_norm=False), experts Swish(alpha) with
   * clamps and biases, no Qwen rounding points.  The per-layer arrays below are
   * HOST arrays of device pointers (NULL array or NULL entry = none). */
  int variant;
  int H_actual;                /* RMSNorm divisor; <= 0: H                      */
  const void* const* b_qkv;    /* [(nq + 2 nkv) d] bf16                          */
  const void* const* b_o;      /* [H] bf16                                       */
  const void* const* sinks;    /* [nq] fp32                                      */
  const void* const* router_bias;  /* [E] bf16                                   */
  const void* const* gate_up_bias; /* [E, 2, I] bf16                             */
  const void* const* down_bias;    /* [E, H] bf16                                */
  const int* window;           /* host [num_layers]: sliding window W (0 = full);
                                  a windowed layer's caches hold W rows          */
  const int* layer_s_max;      /* host [num_layers] cache rows per layer, or NULL
                                  (all S_max)                                    */
  float act_alpha;             /* Swish alpha (GPT-OSS 1.702)                    */
  float gate_hi, gate_lo, up_hi, up_lo;   /* expert clamps (+-INFINITY = none)   */
  /* Device copy of the per-layer pointers (mkd_qwen3_write_layer_table), read by
   * the persistent decode path; NULL: that path is not used.                   */
  const void* layer_table;
  /* Routing log (no counterpart in the reference, whose router outputs stay on
   * chip): when set, every decode / prefill call writes, for each layer l and
   * each of its B tokens, what that layer's router actually produced, at
   * route_log + l * stride (layout from mkd_qwen3_route_log_layout):
   *   idx    int32 [B][K]  expert indices in rank order (as used by the experts)
   *   w      fp32  [B][K]  routing weights of those slots
   *   logits fp32  [B][E]  router logits (bias included) the top-k ran on
   *   r      bf16  [B][H]  the post-attention residual the router norm read
   * route_log_bytes must be >= mkd_qwen3_route_log_bytes(m, B).  NULL: no log. */
  void* route_log;
  size_t route_log_bytes;
} mkd_qwen3_model;
#define MKD_VARIANT_QWEN3 0
#define MKD_VARIANT_GPT_OSS 1
size_t mkd_qwen3_workspace_bytes(const mkd_qwen3_model* m, int B);
/* Routing log for B tokens per call: total bytes (all layers), and the byte
 * offsets of the idx / w / logits / r arrays inside one layer's record and the
 * record stride (offsets[0..4] = idx, w, logits, r, stride). */
size_t mkd_qwen3_route_log_bytes(const mkd_qwen3_model* m, int B);
int mkd_qwen3_route_log_layout(const mkd_qwen3_model* m, int B, size_t* offsets);
/* hidden [B, H] bf16 in/out; position_ids [B] int32 (device); cos/sin [B, d]
 * fp32 or NULL (then generated from position_ids and inv_freq). */
int mkd_qwen3_decode_layers(const mkd_qwen3_model* m, int B, void* hidden,
                            const int* position_ids, const float* cos, const float* sin,
                            void* workspace, size_t workspace_bytes, void* stream);
/* Context encoding (prefill) of one sequence through all layers:
 * hidden [T, H] bf16 in/out holds T consecutive tokens of sequence `seq` at
 * position_ids [T] (int32, device; normally p0 .. p0 + T - 1), 1 <= T <= 4096
 * (above 128 tokens the experts run as LDS-tiled MFMA grouped GEMMs).
 * Every token's k / v rows are written to sequence seq's cache (flat: batch
 * index seq; paged: block_table row seq) before the attention reads it, so
 * token t attends the cache rows below its position, including those of the
 * earlier tokens of the same call.  The reference's counterpart is the CTE
 * (context-encoding) layer path, qwen_with_megakernel.py:496-526.  The caller
 * keeps seq within the caches; workspace from mkd_qwen3_workspace_bytes(m, T).
 * Models with sliding-window layers take T = 1 (MKD_ERR_UNSUPPORTED otherwise).
 * Always the multi-kernel layers (the decode-path setting is ignored). */
int mkd_qwen3_prefill_layers(const mkd_qwen3_model* m, int seq, int T, void* hidden,
                             const int* position_ids, const float* cos, const float* sin,
                             void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Decode-step epilogue (the NxDI side of the reference step:
 * qwen_with_megakernel.py:533-594, main.py:390-398): embedding gather, final
 * RMSNorm (HF order), lm_head on packed [V, H], greedy arg-max.
 * ------------------------------------------------------------------------- */
/* token_ids [B] int32 (ids outside [0, V) give zero rows), table [V, H] bf16, out [B, H]. */
int mkd_embed(const int* token_ids, const void* table, void* out, int B, int H, int V,
              void* stream);
/* hidden_actual: RMSNorm divisor (<= 0: H, for a zero-padded H); norm_order: 2 =
 * weight * bf16(x * rinv) (HF Qwen3 RMSNorm), 1 = bf16((x * rinv) * weight)
 * (HF GPT-OSS RMSNorm). */
size_t mkd_lm_head_workspace_bytes(int B, int H, int V);
int mkd_lm_head_greedy(const void* hidden, const void* ln_f, float eps, const void* lm_head_packed,
                       int B, int H, int V, int hidden_actual, int norm_order, float* logits,
                       int* next_tokens, void* workspace, size_t workspace_bytes, void* stream);

/* Greedy-loop glue for a graph-captured decode step: token_ids[b] = next_tokens[b],
 * position_ids[b] += 1.  (The reference's host loop does this in NxDI.) */
int mkd_decode_advance(int* token_ids, int* position_ids, const int* next_tokens, int B,
                       void* stream);

/* ---------------------------------------------------------------------------
 * Measurement hook (no counterpart in the reference; used by bench.py).
 * After this call the i-th subsequent launch (i < n) of the kernel class below
 * records start_events[i] / stop_events[i] (hipEvent_t handles, host array) as
 * part of the GEMM / attention kernel's own dispatch (hipExtLaunchKernel), so
 * each pair times that kernel's execution alone.  Eager launches only: on a
 * capturing stream nothing is recorded.  A class whose launch has no timed
 * kernel turns the hook off.  kernel_class < 0 turns the hook off.
 * Process-global, not thread-safe.
 * ------------------------------------------------------------------------- */
#define MKD_KCLASS_MOE_GATE_UP 1
#define MKD_KCLASS_MOE_DOWN 2
#define MKD_KCLASS_QKV 3
#define MKD_KCLASS_OPROJ 4
#define MKD_KCLASS_ATTN 5
#define MKD_KCLASS_LM_HEAD 6
#define MKD_KCLASS_ROUTER 7 /* router GEMM + select (two launches, one bracket) */
#define MKD_KCLASS_LAYER 8  /* persistent decoder-layer kernel (one launch per layer) */
int mkd_profile_events(int kernel_class, void* const* start_events, void* const* stop_events,
                       int n);
int mkd_profile_count(void); /* launches recorded since the last mkd_profile_events */

/* ---------------------------------------------------------------------------
 * Decode-layer execution path (no counterpart in the reference, whose step is
 * one compiled NEFF).  mode 0 (default): each layer of
 * mkd_qwen3_decode_layers is the multi-kernel sequence.  mode 1: each layer is
 * ONE persistent kernel launch for all layers (all stages on one block per CU,
 * separated by grid barriers) when m->layer_table is set and the model is the
 * Qwen3 flow with bf16 experts, B <= 4,
 * d in {64, 128}, gqa <= 16, no biases / sinks / windows, and the stage
 * buffers fit the LDS budget; other configurations keep the multi-kernel
 * sequence.  In mode 0, where the router top-k runs inside the expert launch
 * (a single token with bf16 experts), the gate/up and down projections share
 * that launch, the down blocks waiting inside it for their expert's gate/up
 * blocks; and at up to 4 tokens the attention, its chunk combine and the
 * output projection run as one launch (the projection blocks load their
 * weights while the attention runs, then wait for the combine blocks).
 * Mode 2 is mode 0 with every stage a launch of its own.  The
 * workspace size does not depend on the mode.  Process-global.
 * mkd_qwen3_layer_kernel_status reports (after a stream sync) whether the
 * workspace's plan uses the persistent kernel and whether any of its grid
 * barriers, or any in-launch wait of the joined expert launch, timed out
 * (results of such a step are invalid; the spins are bounded so every kernel
 * completes).
 * ------------------------------------------------------------------------- */
int mkd_set_decode_path(int mode);
/* The per-layer weight and cache pointers of m as a device table (written once,
 * synchronously, to `table`, a device buffer of mkd_qwen3_layer_table_bytes(m)
 * bytes); set m->layer_table to it to enable the persistent decode path. */
size_t mkd_qwen3_layer_table_bytes(const mkd_qwen3_model* m);
int mkd_qwen3_write_layer_table(const mkd_qwen3_model* m, void* table, size_t table_bytes);
/* Which decode path mkd_qwen3_decode_layers takes for m and B tokens under the
 * current mode (no counterpart in the reference): *plan = MKD_PLAN_PERSISTENT
 * (one persistent launch for all layers) or MKD_PLAN_JOINED_EXPERTS (the
 * multi-kernel layers with gate/up and down in one launch), else 0; plus
 * MKD_PLAN_JOINED_ATTENTION when the multi-kernel layers run attention,
 * combine and output projection as one launch, and MKD_PLAN_ROUTER_IN_ATTENTION
 * when (all layers of m having one cache length) the router stage joins it. */
#define MKD_PLAN_PERSISTENT 1
#define MKD_PLAN_JOINED_EXPERTS 2
#define MKD_PLAN_JOINED_ATTENTION 4
/* ... and the residual add, post-attention norm and router GEMM run as that
 * launch's last blocks (no router launch of their own). */
#define MKD_PLAN_ROUTER_IN_ATTENTION 8
int mkd_qwen3_decode_plan(const mkd_qwen3_model* m, int B, int* plan);
/* Self-check of the device's fp32 -> bf16 rounding, which every bf16 result of
 * the library goes through (no counterpart in the reference): converts all
 * 2^32 fp32 bit patterns with the library's conversion and with the integer
 * round-to-nearest-even form, and adds the number of non-NaN patterns that
 * differ (and of NaNs that do not stay NaN) to the device word *mismatches
 * (8 bytes, zeroed by the caller).  Asynchronous on `stream`. */
int mkd_selfcheck_bf16_round(unsigned long long* mismatches, void* stream);
int mkd_qwen3_layer_kernel_status(const mkd_qwen3_model* m, int B, const void* workspace,
                                  size_t workspace_bytes, int* used, int* barrier_timeout);

#ifdef __cplusplus
}
#endif
#endif /* MKD_H_ */
