/* C ABI of the MI355X (gfx950) decode kernels for the Qwen3.5-4B int4 path.
 *
 * Plain pointers, sizes and a hipStream_t; no torch types. Every entry point is
 * asynchronous on `stream`, allocates nothing, and returns a DfStatus (0 = OK).
 * bf16 tensors are passed as uint16_t bit patterns. Scratch ("workspace") is
 * always caller-owned.
 *
 * Each declaration names the reference interface it replaces
 * (LoveManna/deltaforge, src/deltaforge/...).
 */
#ifndef DELTAFORGE_HIP_H
#define DELTAFORGE_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- int4 dequantise-GEMV family ------------------------------------------------ */

enum DfPrologue {
  DF_PRO_NONE = 0,           /* x as given                                             */
  DF_PRO_RMSNORM = 1,        /* RMSNorm(1+w) of x over K (reference.py:92-96)          */
  DF_PRO_ADD_RMSNORM = 2,    /* RMSNorm(1+w) of bf16(x + x2) (reference.py:730-735)   */
  DF_PRO_GATED_RMSNORM = 3   /* per-128 GatedRMSNorm(x, gate=x2) (reference.py:115-121) */
};

enum DfEpilogue {
  DF_EPI_STORE = 0,          /* out = bf16(y)                                          */
  DF_EPI_RESIDUAL = 1,       /* out = bf16(res + bf16(y)) (reference.py:730, 735)      */
  DF_EPI_SWIGLU = 2,         /* out = bf16(bf16(silu(gate)) * up) over alternating
                                16-column gate / up tiles (reference.py:692-693)      */
  DF_EPI_LOGITS = 3          /* as STORE; the tied LM head's own kernel instance       */
};

typedef struct DfInt4GemvArgs {
  const uint8_t* w;          /* tiled nibbles from df_int4_repack                     */
  const uint16_t* s;         /* tiled bf16 scales from df_int4_repack                 */
  const uint16_t* x;         /* [rows][ldx] bf16 activations                          */
  const uint16_t* x2;        /* ADD: residual [rows][ldx2]; GATED: gate z [rows][ldx2] */
  const uint16_t* norm_w;    /* RMSNORM/ADD: [K]; GATED: [128]                        */
  const uint16_t* res;       /* RESIDUAL: [rows][ldo] (may alias out)                 */
  uint16_t* out;             /* [rows][ldo]                                           */
  uint16_t* h_out;           /* ADD: optional [rows][K] copy of bf16(x + x2)          */
  float* part;               /* set by the library from the workspace                 */
  int rows, K, N;            /* rows <= 16; K % 256 == 0; N % 64 == 0                 */
  int ldx, ldx2, ldo;        /* row strides (elements) of x, x2 and out/res           */
  int tiles_per_workgroup;   /* 1, 2, 4 or 8 sixteen-column tiles per workgroup       */
  int ksplit, groups_per_split;  /* K split across workgroups (1 = none)              */
  int prologue, epilogue;
  float eps;
} DfInt4GemvArgs;

/* Choose the launch shape for a GEMV and report the workspace it needs (0 when the
 * K range is not split across workgroups). Replaces the launch heuristic of
 * kernels/tiled_gemv.py:291-311. */
int df_int4_gemv_plan(int rows, int K, int N, int epilogue, int target_waves,
                      int* tiles_per_workgroup, int* ksplit, int* groups_per_split,
                      size_t* workspace_bytes);
size_t df_int4_gemv_workspace_bytes(int rows, int N, int ksplit);

/* y = x @ dequant(W) with an optional fused prologue/epilogue. Every weight is
 * bf16((nibble - 8) * scale), accumulated in fp32.
 * Replaces torch_dequant_gemv_int4 (kernels/visible_int4_head.py:187-199) and
 * tiled_gemv_int4 (kernels/tiled_gemv.py:915-953); with DF_PRO_ADD_RMSNORM it is the
 * tied head with its final residual + RMSNorm (reference.py:735, 810, 764-777).
 * With ksplit > 1 a second kernel sums the fp32 partials held in the workspace;
 * calls sharing a workspace must not overlap. No atomics: results are deterministic. */
int df_int4_gemv(const DfInt4GemvArgs* args, void* workspace, size_t workspace_bytes,
                 hipStream_t stream);

/* Canonical K-major int4 (packed [K/2][N] uint8, scale [K/128][N] bf16) -> device tiling.
 * Replaces the install-time quantise/repack of kernels/tiled_gemv.py:242-278. */
int df_int4_repack(const uint8_t* packed, const uint16_t* scale, int K, int N,
                   uint8_t* w_tiled, uint16_t* s_tiled, hipStream_t stream);

/* W[k][n] = bf16((nibble - 8) * scale) from the tiled layout, [K][N] bf16.
 * Replaces dequantise_int4_k_major(...).to(bf16) (kernels/tiled_gemv.py:281-288). */
int df_int4_dequant(const uint8_t* w_tiled, const uint16_t* s_tiled, int K, int N,
                    uint16_t* out, hipStream_t stream);

/* ---- Gated DeltaNet decode step ------------------------------------------------- */

typedef struct DfGatedDeltaArgs {
  const uint16_t* qkv;       /* [B][ld_qkv] in_proj_qkv output (pre-conv)              */
  const uint16_t* a;         /* [B][ld_ab] in_proj_a output                            */
  const uint16_t* b;         /* [B][ld_ab] in_proj_b output                            */
  const uint16_t* A_log;     /* [Hv]                                                   */
  const uint16_t* dt_bias;   /* [Hv]                                                   */
  const uint16_t* conv_w;    /* [C][4]                                                 */
  const uint16_t* conv_in;   /* mode 0: [B][C][3] history (oldest first)               */
  uint16_t* conv_out;        /* mode 0: [B][C][3] new history (must not alias conv_in) */
  uint16_t* conv_ring;       /* mode 1: [B][C][4] ring, slot = position % 4            */
  const int* position;       /* mode 1: device scalar, the token's position            */
  float* state;              /* [B][Hv][Dk][Dv] fp32, updated in place                 */
  uint16_t* out;             /* [B][Hv][Dv] bf16                                       */
  int batch, ld_qkv, ld_ab;
  int num_k_heads, num_v_heads, head_k_dim, head_v_dim;
  int conv_mode;
} DfGatedDeltaArgs;

/* One token of GatedDeltaNet's middle: 4-tap causal conv + SiLU, q/k L2-norm, q scale,
 * beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias), then the gated delta rule.
 * Replaces GatedDeltaNet._causal_conv + recurrent_gated_delta_rule at seq_len 1
 * (reference.py:496-545; kernels/inline_causal_conv.py:98-129;
 * kernels/gated_delta_step.py:109-186). Requires Dk == Dv == 128, 4 taps. */
int df_gated_delta_step(const DfGatedDeltaArgs* args, hipStream_t stream);

typedef struct DfDeltaRuleArgs {
  const float* state_in;     /* [B][H][Dk][Dv] fp32                                    */
  float* state_out;          /* [B][H][Dk][Dv] fp32; may alias state_in                */
  const float* query;        /* [B][H][Dk] fp32, already L2-normed and scaled by Dk^-1/2 */
  const float* key;          /* [B][H][Dk] fp32, already L2-normed                     */
  const float* value;        /* [B][H][Dv] fp32                                        */
  const float* g;            /* [B][H] fp32 log-space decay (<= 0)                     */
  const float* beta;         /* [B][H] fp32                                            */
  float* out;                /* [B][H][Dv] fp32                                        */
  int batch, heads, key_dim, value_dim;  /* Dk == 128, Dv % 32 == 0                    */
} DfDeltaRuleArgs;

/* One gated delta-rule step on normalised inputs, all contiguous:
 * S *= exp(g); r = k^T S; delta = (v - r) beta; S += k delta^T; out = q^T S.
 * Replaces deltaforge::delta_rule_step (kernels/gated_delta_step.py:109-186). */
int df_delta_rule_step(const DfDeltaRuleArgs* args, hipStream_t stream);

typedef struct DfDeltaInputsArgs {
  const uint16_t* mixed;     /* [B][ld_mixed] bf16 conv + SiLU output (q | k | v)       */
  const uint16_t* a;         /* [B][ld_ab] bf16 in_proj_a output                        */
  const uint16_t* b;         /* [B][ld_ab] bf16 in_proj_b output                        */
  const uint16_t* A_log;     /* [Hv] bf16                                               */
  const uint16_t* dt_bias;   /* [Hv] bf16                                               */
  float* query;              /* [B][Hv][Dk] fp32 out: L2-normed, scaled by Dk^-1/2      */
  float* key;                /* [B][Hv][Dk] fp32 out: L2-normed                         */
  float* value;              /* [B][Hv][Dv] fp32 out                                    */
  float* g;                  /* [B][Hv] fp32 out: -exp(A_log) softplus(a + dt_bias)     */
  float* beta;               /* [B][Hv] fp32 out: bf16(sigmoid(b)) widened              */
  int ld_mixed, ld_ab;
  int batch, num_k_heads, num_v_heads, head_k_dim, head_v_dim;  /* Dk == 128          */
  float eps;                 /* L2-norm epsilon (1e-6 in the reference)                 */
} DfDeltaInputsArgs;

/* df_delta_rule_step's inputs from one token of Gated DeltaNet: the q/k L2 norms (key heads
 * repeated over their value heads), the q scale, v in fp32 and the two gates. Replaces the
 * torch prologue the reference runs around deltaforge::delta_rule_step when that op is
 * installed (kernels/gated_delta_step.py:189-213, 245-256). */
int df_delta_step_inputs(const DfDeltaInputsArgs* args, hipStream_t stream);

/* ---- GQA attention decode (split-KV) -------------------------------------------- */

typedef struct DfAttnDecodeArgs {
  const uint16_t* q;         /* [B][ld_q] q_proj output: per head [query D | gate D]   */
  const uint16_t* k;         /* [B][ld_kv] new key   (Hkv x D) before k_norm/RoPE      */
  const uint16_t* v;         /* [B][ld_kv] new value (Hkv x D)                         */
  const uint16_t* q_norm_w;  /* [D] (1+w)                                              */
  const uint16_t* k_norm_w;  /* [D] (1+w)                                              */
  const float* inv_freq;     /* [rotary/2] fp32 (as the model stores it)               */
  uint16_t* k_cache;         /* [B][Hkv][max_len][D]                                   */
  uint16_t* v_cache;         /* [B][Hkv][max_len][D]                                   */
  const int* position;       /* device scalar: keys already cached (= new position)    */
  uint16_t* out;             /* [B][Hq*D] gated attention output                       */
  int batch, ld_q, ld_kv, num_q_heads, num_kv_heads, head_dim, rotary_dim, max_len;
  int splits;                /* fixed grid; empty splits are allowed                   */
  int gate;                  /* 0 sigmoid, 1 swish (reference.py:558-568)              */
  float eps;
} DfAttnDecodeArgs;

/* Workspace of df_attention_decode / df_split_kv_decode_attention: the per-split partials
 * (a merge kernel combines them after the split kernel). It needs no clearing, and one
 * workspace serves calls of any shape on one stream (calls that overlap must not share it). */
size_t df_attention_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads,
                                           int head_dim, int splits);
int df_attention_decode_splits(int batch, int num_kv_heads, int max_keys);

/* q/k RMSNorm + partial RoPE, KV-cache write at `position`, split-KV online-softmax
 * decode over position+1 keys, deterministic log-sum-exp merge, and the output gate.
 * Replaces GatedAttention.forward's seq_len==1 path between the projections
 * (reference.py:621-676; kernels/flash_decode_splitkv.py:177-331;
 * kernels/gqa_decode.py:322-335). head_dim 256, 4 q heads per KV head. */
int df_attention_decode(const DfAttnDecodeArgs* args, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* Single-token GQA attention over a whole cache, without prologue or gate: query
 * [B][Hq][D] bf16 (already normed and rotated), key/value [B][Hkv][L][D] bf16 contiguous,
 * out[b][h] = sum_j softmax_j(scale q.k_j) v_j as bf16, split over `splits` (1..256) KV
 * ranges merged by the log-sum-exp identity. D == 256 and Hq == 4 Hkv. The workspace is
 * df_attention_decode_workspace_bytes(B, Hq, Hkv, D, splits). Replaces
 * deltaforge::split_kv_decode_attention
 * (kernels/flash_decode_splitkv.py:177-261). */
int df_split_kv_decode_attention(const uint16_t* query, const uint16_t* key, const uint16_t* value, int batch,
                                 int num_q_heads, int num_kv_heads, int key_len, int head_dim, float scale,
                                 int splits, uint16_t* out, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/* df_attention_decode without a workspace argument, for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc). It has no
 * counterpart in the reference. Its scratch (the split partials) is a file-scope device
 * array of df_attention_decode_static_capacity() bytes (about 8.5 MB), one per GPU, held
 * until the process ends; calls with batch * num_q_heads * splits > 8192 return
 * DF_WORKSPACE_TOO_SMALL. No call allocates. Every
 * call on a GPU shares that GPU's array, so calls that overlap on one GPU (two streams, or
 * two threads) race: serialise them. */
size_t df_attention_decode_static_capacity(void);
int df_attention_decode_static(const DfAttnDecodeArgs* args, hipStream_t stream);

/* ---- elementwise ops of the slot surface ---------------------------------------- */

/* rms_norm (kernels/fused_rmsnorm_residual.py:201-226; reference.py:92-96). */
int df_rms_norm(const uint16_t* x, const uint16_t* w, float eps, int rows, int n,
                uint16_t* out, hipStream_t stream);
/* add_rms_norm -> (residual + x, rms_norm(residual + x))
 * (kernels/fused_rmsnorm_residual.py:164-198). */
int df_add_rms_norm(const uint16_t* x, const uint16_t* residual, const uint16_t* w, float eps,
                    int rows, int n, uint16_t* resid_out, uint16_t* out, hipStream_t stream);
/* silu_mul: bf16(bf16(silu(gate)) * up) (kernels/fused_swiglu.py:51-80). */
int df_silu_mul(const uint16_t* gate, const uint16_t* up, size_t n, uint16_t* out,
                hipStream_t stream);
/* partial_rope over (rows = B*H*S) rows of head_dim; cos/sin [B*S][rotary] bf16,
 * row r uses cos row (r / (H*S)) * S + r % S (kernels/fused_rope.py:97-158). */
int df_partial_rope(const uint16_t* x, const uint16_t* cos, const uint16_t* sin, int batch,
                    int heads, int seq, int head_dim, int rotary_dim, uint16_t* out,
                    hipStream_t stream);
/* causal_conv step at seq_len 1, history [B][C][3] updated in place
 * (kernels/inline_causal_conv.py:98-129; kernels/fused_causal_conv.py:136-181). */
int df_causal_conv_step(const uint16_t* x, uint16_t* conv_cache, const uint16_t* weight,
                        int batch, int channels, uint16_t* out, hipStream_t stream);

/* ---- decode-loop glue ----------------------------------------------------------- */

/* Tied embedding row from the int4 head: out[b][k] = bf16((nibble - 8) * scale) of
 * vocab column t (reference.py:804 with the tied, int4-quantised table), where
 * t = tokens[b], or, when prompt != NULL, t = prompt[b * prompt_len + *position]
 * (teacher-forced prefill; positions outside the prompt write nothing). */
int df_embed_int4(const int64_t* tokens, const int64_t* prompt, int prompt_len,
                  const int* position, int batch, const uint8_t* w_tiled,
                  const uint16_t* s_tiled, int hidden, int vocab, uint16_t* out,
                  hipStream_t stream);

/* Embedding rows from a bf16 table (reference.py:804, `F.embedding`): out[b] =
 * table[t], t chosen as in df_embed_int4. For checkpoints whose embedding table is not the
 * dequantised int4 head. */
int df_embed_bf16(const int64_t* tokens, const int64_t* prompt, int prompt_len,
                  const int* position, int batch, const uint16_t* table, int hidden,
                  int vocab, uint16_t* out, hipStream_t stream);

size_t df_argmax_workspace_bytes(int rows, int n);
/* Greedy next token: first index of the max of each bf16 logits row (torch's tie rule;
 * model.py:145-147 `logits[:, -1].argmax`). After all rows are reduced, the last
 * workgroup writes tokens[row] (int64); if token_log != NULL (needs step) it also writes
 * token_log[row * log_stride + *step]; then, once, *position += advance (if position)
 * and *step += 1 (if step). The workspace must be zero-filled once before first use;
 * the kernel leaves it ready for the next call. rows <= 256. */
int df_argmax(const uint16_t* logits, int rows, int n, int64_t* tokens, int64_t* token_log,
              int log_stride, int* position, int advance, int* step, void* workspace,
              size_t workspace_bytes, hipStream_t stream);

/* ---- prompt prefill (every token of the prompt per launch) ----------------------
 * The reference runs a prompt through ReferenceModel.forward with seq_len = P
 * (reference.py:779-817): the projections as [P, K] x [K, N] products, the conv over the
 * sequence, the sequential delta-rule scan (reference.py:450-458) and causal attention. These
 * entry points are that forward's pieces. Rounding points are the reference's; only fp32
 * summation order differs. */

/* out = bf16(x @ bf16(dequant(W))), fp32 sums, W in the device tiling of df_int4_repack
 * (reference kernels/quantised_linear.py GEMV_MAX_ROWS dense fallback, which dequantises and
 * calls F.linear for more than 64 rows). epilogue DF_EPI_STORE: out [M][N]. DF_EPI_SWIGLU:
 * W's 16-column tiles alternate gate, up; out [M][N/2] = bf16(bf16(silu(gate)) * up).
 * K % 256 == 0, N % 16 == 0 (32 for SwiGLU), ldx % 8 == 0, x and w 16-byte aligned. */
typedef struct DfInt4GemmArgs {
  const uint16_t* x;
  const uint8_t* w;
  const uint16_t* s;
  uint16_t* out;
  int M, K, N, ldx, ldo, epilogue;
} DfInt4GemmArgs;
int df_int4_gemm(const DfInt4GemmArgs* args, hipStream_t stream);

/* Causal 4-tap conv + SiLU over `tokens` rows at positions pos0 .. pos0 + tokens - 1
 * (reference.py:496-510 with the decode step's fp32 tap order): x [tokens][ldx] (channels
 * 0 .. channels-1), weight [channels][4]; history from ring [channels][4] (slot = position
 * mod 4, as the decode step keeps it); afterwards the ring holds the last three inputs. */
int df_causal_conv_prefill(const uint16_t* x, int ldx, int tokens, int channels, const uint16_t* weight,
                           uint16_t* ring, int pos0, uint16_t* out, int ldo, hipStream_t stream);

/* Gated delta rule over a sequence, chunked (64 tokens) and exact in real arithmetic to the
 * token-by-token scan (reference.py:403-461): q, k L2-normalised (q / sqrt(128)), GQA value
 * head h on key head h / (Hv / Hk), beta = bf16(sigmoid(b)), g = -exp(A_log) softplus(a +
 * dt_bias). mixed: the conv output [tokens][ld_mixed] = q | k | v channels; a, b: the raw
 * bf16 gate projections [tokens][ld_ab]; state [Hv][128][128] fp32 read and updated;
 * out [tokens][ld_out] bf16 (head h at column 128 h). */
typedef struct DfDeltaPrefillArgs {
  const uint16_t* mixed;
  const uint16_t* a;
  const uint16_t* b;
  const uint16_t* A_log;
  const uint16_t* dt_bias;
  float* state;
  uint16_t* out;
  int ld_mixed, ld_ab, ld_out;
  int tokens, num_k_heads, num_v_heads;
} DfDeltaPrefillArgs;
/* Workspace (bytes) for `tokens` tokens and Hv value heads: per (64-token chunk, head), the
 * five 64 x 128 fp32 state-independent products of the chunk and its total decay. */
size_t df_delta_rule_prefill_workspace_bytes(int tokens, int num_v_heads);
int df_delta_rule_prefill(const DfDeltaPrefillArgs* args, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* GatedRMSNorm over rows (reference.py:115-121): per 128-wide head of x,
 * out = bf16(bf16(w * bf16(x rsqrt(mean x^2 + eps))) * silu(z)). */
int df_gated_rms_norm_rows(const uint16_t* x, int ldx, const uint16_t* z, int ldz, const uint16_t* weight, float eps,
                           int tokens, int heads, uint16_t* out, int ldo, hipStream_t stream);

/* The attention projection's rows (reference.py:617-639): proj [tokens][ld_proj] holds per
 * query head [query 256 | gate 256], then keys at k_col, values at v_col (head_dim 256).
 * Queries and keys get RMSNorm (1 + w) and partial RoPE at position pos0 + t; queries go to
 * q_out [tokens][Hq][256], keys and values into the caches [Hkv][max_len][256] at row pos0 + t. */
typedef struct DfQkPrefillArgs {
  const uint16_t* proj;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const float* inv_freq;
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int ld_proj, k_col, v_col;
  int tokens, pos0, max_len, num_q_heads, num_kv_heads, rotary_dim;
  float eps;
} DfQkPrefillArgs;
int df_qk_norm_rope_prefill(const DfQkPrefillArgs* args, hipStream_t stream);

/* Causal GQA attention of `tokens` queries at positions pos0 .. over cache rows 0 .. pos
 * (reference.py:645-677): scores = bf16(bf16(q.k) * scale), p = bf16(softmax_fp32),
 * o = bf16(p V), out = bf16(o * bf16(gate_fn(gate))) with gate_fn sigmoid (gate_kind 0) or
 * silu (1). Hq = 4 Hkv, head_dim 256. gate of head h, token t: gate[t * ld_gate + h *
 * gate_head_stride + d]. */
typedef struct DfAttnPrefillArgs {
  const uint16_t* q;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  const uint16_t* gate;
  uint16_t* out;
  int ld_gate, gate_head_stride, ld_out;
  int tokens, pos0, max_len, num_q_heads, num_kv_heads, gate_kind;
  float scale;
} DfAttnPrefillArgs;
int df_attention_prefill(const DfAttnPrefillArgs* args, hipStream_t stream);

/* ---- persistent decode: many bs=1 tokens in one cooperative launch ------------------
 *
 * The whole decode step of greedy_decode (model.py:108-148 driving ReferenceModel.forward,
 * reference.py:779-817) for one sequence, run as 8-way tensor parallelism over the 8 XCDs
 * of one MI355X: 256 workgroups, 32 per XCD. Per layer, XCD x owns value heads 4x..4x+3
 * (key heads 2x, 2x+1) of Gated DeltaNet, query heads 2x, 2x+1 (KV head x/2) of gated
 * attention, 1/8 of the gate/up columns and the matching K slices of out_proj / o_proj /
 * down; only those row-parallel outputs and the argmax cross XCDs. Head geometry is
 * Qwen3.5-4B's (16/32 heads of 128 for DeltaNet, 16/4 heads of 256 for attention,
 * rotary 64, 4-tap conv); hidden % 512 == 0, inter % 1024 == 0, vocab % 128 == 0,
 * hidden <= 4096.
 *
 * Weights are the tiled layout of df_int4_repack. The input projections' columns are in
 * XCD-major order:
 *   DeltaNet in_proj, 1552 columns per XCD x: q[2x], q[2x+1], k[2x], k[2x+1] (128 each),
 *     v[4x..4x+3], z[4x..4x+3] (128 each), a[4x..4x+3], b[4x..4x+3], 8 zero columns.
 *   attention q|k|v proj, 1536 columns per XCD x: for h in 2x, 2x+1 the 512 q_proj
 *     columns of head h (query 256 | gate 256), then k_proj and v_proj of KV head x/2.
 * gate/up is interleaved by 16-column tile (gate, up, gate, up ...); the others are in
 * natural order. */
typedef struct DfPersistLayer {
  int kind;                        /* 0 = Gated DeltaNet, 1 = gated attention             */
  const uint16_t* in_norm;         /* [hidden] input_layernorm (1 + w)                   */
  const uint16_t* post_norm;       /* [hidden] post_attention_layernorm (1 + w)          */
  const uint8_t* proj_w;           /* input projection, XCD-major columns (see above)    */
  const uint16_t* proj_s;
  const uint8_t* out_w;            /* out_proj / o_proj: K = 4096, N = hidden            */
  const uint16_t* out_s;
  const uint8_t* gu_w;             /* gate|up interleaved: K = hidden, N = 2 * inter     */
  const uint16_t* gu_s;
  const uint8_t* down_w;           /* K = inter, N = hidden                              */
  const uint16_t* down_s;
  const uint16_t* conv_w;          /* DeltaNet: [8192][4] conv taps                      */
  const uint16_t* A_log;           /* [32]                                               */
  const uint16_t* dt_bias;         /* [32]                                               */
  const uint16_t* gnorm_w;         /* [128] GatedRMSNorm weight                          */
  uint16_t* conv_ring;             /* [8192][4] history ring, slot position % 4          */
  float* state;                    /* [32][128][128] fp32 recurrent state                */
  const uint16_t* q_norm;          /* attention: [256] (1 + w)                           */
  const uint16_t* k_norm;          /* [256]                                              */
  uint16_t* k_cache;               /* [4][max_len][256]                                  */
  uint16_t* v_cache;
} DfPersistLayer;

typedef struct DfPersistModel {
  int hidden, inter, vocab, num_layers, max_len;
  int gate_kind;                   /* output gate: 0 sigmoid, 1 silu                     */
  float eps;
  const DfPersistLayer* layers;    /* DEVICE array [num_layers]                          */
  const uint8_t* head_w;           /* tied head, natural columns: K = hidden, N = vocab  */
  const uint16_t* head_s;
  const uint16_t* final_norm;      /* [hidden]                                           */
  const uint32_t* rope;            /* [max_len][32] RoPE table: rotary pair j of position */
                                   /* p as bf16(cos(p * f_j)) | bf16(sin(p * f_j)) << 16, */
                                   /* f_j the bf16-rounded inverse frequency (fp32 angle) */
  int* position;                   /* tokens already cached (read at launch, advanced)   */
  int64_t* tokens;                 /* [1] token the next step embeds (argmax written back) */
  const int64_t* prompt;           /* [prompt_len], teacher-forced steps read prompt[pos] */
  int prompt_len;
  int64_t* token_log;              /* generated tokens, token_log[*step] per greedy step */
  int log_capacity;
  int* step;                       /* next token_log index                               */
  uint16_t* logits;                /* [vocab] bf16 logits of the last step (or NULL)     */
  uint64_t* trace;                 /* optional: s_memrealtime (100 MHz) stamps of one    */
  int trace_step;                  /* step's phases (start, staged, end), as seen by     */
  int trace_capacity;              /* workgroup (XCD 0, rank 0); NULL disables. Honoured */
                                   /* only by a build with DF_TRACE defined              */
  const uint16_t* embed_table;     /* [vocab][hidden] bf16 embedding rows, or NULL to    */
                                   /* embed from the int4 head (the tied table)          */
} DfPersistModel;

/* Workspace for df_decode_persistent, zero-filled once before first use and kept (it
 * carries the launch-to-launch epoch). Its first four int32 are {epoch, abort, error,
 * reserved}: after a launch, a nonzero `abort` means a wait timed out (`error` says
 * which) and the outputs are invalid. */
size_t df_decode_persistent_workspace_bytes(int hidden);

/* Run `steps` decode steps from *position. teacher_forced: the token of each step is
 * prompt[position] (prefill; token_log untouched); else the previous step's argmax
 * (greedy; appended to token_log). Either way the last argmax is left in tokens[0] and
 * position advances by `steps`. Needs all 256 workgroups co-resident (cooperative
 * launch); returns DF_LAUNCH_FAILED if the device cannot host them. With the environment
 * variable DF_PERSISTENT_PLAIN_LAUNCH=1 the same grid goes out as an ordinary dispatch
 * (for profilers that cannot follow cooperative launches), after the same capacity check. */
int df_decode_persistent(const DfPersistModel* model, int steps, int teacher_forced, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DELTAFORGE_HIP_H */
