/*
 * kmoe.h — C ABI of the MI355X-native MoE feed-forward hot path.
 *
 * One MoE layer forward = router -> dispatch -> grouped SwiGLU GEMMs -> combine
 * (+ aux-loss finalisation).  Every entry point:
 *   - takes raw device pointers, sizes, dtype enums and a hipStream_t passed as
 *     `void* stream` (NULL = the null stream); all work is stream-ordered;
 *   - never allocates, never synchronises the host, never throws;
 *   - returns 0 (KMOE_OK) or a negative KMOE_ERR_* code, with a message in
 *     kmoe_last_error() (thread-local);
 *   - borrows every buffer: outputs and workspaces are caller-owned.
 *
 * Reference interfaces replaced (file:line into JBedichek/Kolmogorov-MoE-Architecture):
 *   Router.forward                   moe_arch/model/moe.py:423-462
 *   GroupedExperts.forward           moe_arch/model/moe.py:213-294
 *   MoELayer._compute_*_loss         moe_arch/model/moe.py:840-939
 *   ExpertChoiceRouter.forward       moe_arch/model/moe.py:494-530
 *   GroupedExpertsExpertChoice       moe_arch/model/moe.py:626-673, 132-158
 *   MoDRouter.forward                moe_arch/model/mod.py:67-122 (+ layers.py:148-185)
 *   moe_kernels.grouped_swiglu_forward
 *                                    moe_arch/kernels/grouped_gemm.cu:186-257
 *                                    (Python binding moe_arch/kernels/__init__.py:29-56)
 */
#ifndef KMOE_H
#define KMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KMOE_ABI_VERSION 2

/* status codes */
#define KMOE_OK 0
#define KMOE_ERR_NULL (-1)        /* a required pointer is NULL */
#define KMOE_ERR_SHAPE (-2)       /* a size is out of the supported range */
#define KMOE_ERR_DTYPE (-3)       /* unsupported dtype enum */
#define KMOE_ERR_WORKSPACE (-4)   /* workspace too small */
#define KMOE_ERR_LAUNCH (-5)      /* HIP reported an error at launch */
#define KMOE_ERR_UNSUPPORTED (-6) /* valid request this build does not implement */

/* dtype enums */
#define KMOE_DTYPE_BF16 0
#define KMOE_DTYPE_F32 1
#define KMOE_DTYPE_FP8_E4M3 2 /* OCP e4m3fn, saturating at +-448 */

/* limits */
#define KMOE_MAX_EXPERTS 64
#define KMOE_ROUTER_HIDDEN 128 /* the reference router MLP width, moe.py:346 */

const char* kmoe_last_error(void);
int kmoe_abi_version(void);
/* Version of the packed weight layouts written by kmoe_pack_weights /
 * kmoe_pack_weights_bwd (row order, padding, scale placement).  It changes whenever
 * those layouts change, so a packed cache saved by another build can be refused.
 * No counterpart in the reference (its experts have no derived weight layout).  */
#define KMOE_PACK_LAYOUT 2
int kmoe_pack_layout_version(void);

/* ------------------------------------------------------------------------ */
/* (a) Router — replaces Router.forward (moe.py:423-462) and the logits half of
 * ExpertChoiceRouter.forward (moe.py:513-514).
 *   logits[t,:] = SiLU(x[row(t)] . w_in^T) . w_out^T  (+ logit_bias), fp32 accumulate
 *   row(t) = row_index ? row_index[t] : t
 * When k > 0 (k <= min(8, E)) it also selects the top-k experts of each token, ranked by fp32
 * logit (descending; equal logits -> lowest expert index first), and writes the
 * renormalised softmax weights  w_j = p_j / sum_sel p  (moe.py:441,455-460).
 * `partials` (nullable) receives per-block sums for the aux losses; its length in
 * floats is kmoe_router_partials_len(T, E).  A block is kmoe_router_block_tokens(T)
 * tokens: one workgroup of the kernel (32 when ceil(T/32) workgroups fit the device's
 * compute units at once, else 64; a function of T and the current device only).
 *   x: (rows, d) bf16;  w_in: (128, d) bf16;  w_out: (E, 128) bf16
 *   logits: (T, E) f32; topk_idx: (T, k) int64; topk_w: (T, k) f32          */
int64_t kmoe_router_partials_len(int64_t T, int E);
int kmoe_router_block_tokens(int64_t T);
int kmoe_router(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                const void* w_out, int E, const float* logit_bias, int k, float* logits,
                int64_t* topk_idx, float* topk_w, float* partials, void* stream);

/* Aux losses — replaces MoELayer._compute_auxiliary_losses (moe.py:840-939).
 *   LB = E * sum_e (counts[e] / (T*k)) * mean_t softmax(logits)[t,e]
 *   z  = mean_t logsumexp(logits[t,:])^2
 *   out[0] = w_lb*LB + w_z*z, out[1] = LB, out[2] = z
 * counts may be NULL (then LB = 0; expert-choice uses w_z*z only, moe.py:833-836).
 * Reduces the router partials in a fixed order (deterministic).            */
int kmoe_aux_loss(const float* partials, int64_t T, int E, const int32_t* counts, int k, float w_lb,
                  float w_z, float* out, void* stream);

/* MoD router auxiliary loss — replaces MoDRouter._compute_auxiliary_loss's
 * binary_cross_entropy_with_logits (moe_arch/model/mod.py:141-171) over the auxiliary
 * router's logits (T) f32 (kmoe_router_train with E = 1, k = 0 on the aux_router MLP):
 * out[0] = weight / T * (sum_t softplus(logits[t]) - sum_j logits[rows[j]]), the kept
 * rows rows[0, n_keep) (distinct, each in [0, T)) being the targets equal to 1.
 * T > 0, 0 <= n_keep <= T. */
int kmoe_mod_aux_bce(const float* logits, int64_t T, const int32_t* rows, int64_t n_keep, float weight, float* out,
                     void* stream);

/* ------------------------------------------------------------------------ */
/* (b) Dispatch — replaces the sort/bincount/gather half of GroupedExperts.forward
 * (moe.py:238-272).  Stable counting sort of the T*k assignments a = t*k + j by
 * expert (ties in assignment order, = torch.argsort(stable=True)), optional
 * capacity drop (keep the first `capacity` assignments of each expert in that
 * order; capacity <= 0 keeps all), and the row gather
 *   xperm[offsets[e] + r] = x[row(t)]  for the r-th kept assignment of expert e.
 * Outputs: counts (E) routed counts before the drop; offsets (E+1) kept-row
 * offsets; row_token (T*k) token of each permuted row; slot_row (T*k) permuted
 * row of assignment a or -1 if dropped; slot_w (T*k) f32 routing weight.
 * xperm_dtype BF16 copies rows; FP8_E4M3 quantises each row with the per-token
 * scale amax(|x[row]|)/448 written to xperm_scale (one per permuted row).
 * xperm may be NULL with BF16: only the tables are written (for
 * kmoe_gemm_gate_up_rows, which gathers the rows itself).  FP8_E4M3 rows need
 * d <= 8192 (a row is quantised from registers; KMOE_ERR_UNSUPPORTED beyond).
 *   topk_w dtype: w_dtype (BF16 or F32).  workspace: kmoe_dispatch_workspace_bytes. */
size_t kmoe_dispatch_workspace_bytes(int64_t T, int k, int E);
int kmoe_dispatch(const void* x, const int32_t* row_index, int64_t T, int d, const int64_t* topk_idx,
                  const void* topk_w, int w_dtype, int k, int E, int64_t capacity, int32_t* counts,
                  int32_t* offsets, int32_t* row_token, int32_t* slot_row, float* slot_w, void* xperm,
                  int xperm_dtype, float* xperm_scale, void* workspace, size_t workspace_bytes,
                  void* stream);

/* kmoe_dispatch with the per-block expert histograms given instead of counted from
 * topk_idx: block_counts[b*E + e] = number of assignments (t, j) with t in
 * [Bb, Bb + B) and topk_idx[t*k + j] == e, B = kmoe_router_block_tokens(T), as
 * kmoe_router_hist writes them.  Same results as kmoe_dispatch, one launch fewer.
 * Workspace as kmoe_dispatch.                                                     */
int kmoe_dispatch_counted(const void* x, const int32_t* row_index, int64_t T, int d, const int64_t* topk_idx,
                          const void* topk_w, int w_dtype, int k, int E, int64_t capacity,
                          const int32_t* block_counts, int32_t* counts, int32_t* offsets, int32_t* row_token,
                          int32_t* slot_row, float* slot_w, void* xperm, int xperm_dtype, float* xperm_scale,
                          void* workspace, size_t workspace_bytes, void* stream);

/* kmoe_dispatch_counted that also writes the aux losses of kmoe_aux_loss (the
 * dispatch's load-balancing inputs of MoELayer._compute_auxiliary_losses,
 * moe.py:840-939, with counts = this dispatch's routed counts): aux_out[0..2] as
 * kmoe_aux_loss's out, bit for bit.  Up to 65536 tokens one more workgroup of the
 * table launch reduces the router's partials, so a training forward needs no launch
 * for the losses; beyond, kmoe_aux_loss runs after the dispatch.  T must be > 0. */
int kmoe_dispatch_counted_aux(const void* x, const int32_t* row_index, int64_t T, int d, const int64_t* topk_idx,
                              const void* topk_w, int w_dtype, int k, int E, int64_t capacity,
                              const int32_t* block_counts, int32_t* counts, int32_t* offsets, int32_t* row_token,
                              int32_t* slot_row, float* slot_w, void* xperm, int xperm_dtype, float* xperm_scale,
                              void* workspace, size_t workspace_bytes, const float* partials, float w_lb,
                              float w_z, float* aux_out, void* stream);

/* Allocation-free dispatch.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, semantics and results as
 * kmoe_dispatch (bit for bit), without the workspace: the per-block histograms and
 * bases live in a file-scope device array of KMOE_DISPATCH_SCRATCH_BYTES on each GPU
 * (allocated with the library's code object and held until the process ends; looked
 * up once per device, on the first call with that device current).  Sizes whose
 * kmoe_dispatch_workspace_bytes(T, k, E) exceeds it are rejected with
 * KMOE_ERR_WORKSPACE (4 MiB: T*E up to 2^25 - 8192, e.g. T = 2M tokens at E = 16).
 * It calls no allocator.  Every call on a GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race: serialise them.  Nothing in
 * the array has to start at zero (a call writes every entry it reads).              */
#define KMOE_DISPATCH_SCRATCH_BYTES (4u << 20)
int kmoe_dispatch_noalloc(const void* x, const int32_t* row_index, int64_t T, int d, const int64_t* topk_idx,
                          const void* topk_w, int w_dtype, int k, int E, int64_t capacity, int32_t* counts,
                          int32_t* offsets, int32_t* row_token, int32_t* slot_row, float* slot_w, void* xperm,
                          int xperm_dtype, float* xperm_scale, void* stream);

/* Row gather: out[r] = x[row_token[r]] for r < n_rows (rows with row_token < 0 are
 * zero-filled).  out_dtype BF16 (copy) or FP8_E4M3 (per-row scale to out_scale;
 * d <= 8192).
 * n_rows_dev (nullable): device int32 holding the number of valid rows.      */
int kmoe_gather_rows(const void* x, const int32_t* row_token, int64_t n_rows, const int32_t* n_rows_dev,
                     int d, void* out, int out_dtype, float* out_scale, void* stream);

/* ------------------------------------------------------------------------ */
/* (c) Grouped SwiGLU expert GEMMs — replaces moe_kernels.grouped_swiglu_forward
 * (grouped_gemm.cu:186-257) and the bmm block of GroupedExperts.forward
 * (moe.py:275-279).  Rows of expert e are [offsets[e], offsets[e+1]) of xperm;
 * offsets live on the device (no host sync).  max_rows >= offsets[E] bounds the
 * launch.  Weights are used in a packed, derived layout produced by
 * kmoe_pack_weights from the reference parameters w1,w2: (E,d,F), w3: (E,F,d).
 *   F_pad = round_up(F, 128); d % 64 == 0.
 *   h:   (max_rows, F_pad) bf16   h = silu(x.w1[e]) * (x.w2[e])   (ffn.py:17-64)
 *   y:   (max_rows, d)     bf16   y = h.w3[e]
 * FP8_E4M3 inputs carry per-row scales (xperm_scale / h_scale) and per-expert
 * per-output-row weight scales; accumulation is fp32, outputs bf16.          */
int kmoe_padded_ff(int F);
size_t kmoe_packed_w13_bytes(int E, int d, int F, int dtype);
size_t kmoe_packed_w3_bytes(int E, int d, int F, int dtype);
int kmoe_pack_weights(const void* w1, const void* w2, const void* w3, int w_dtype, int E, int d, int F,
                      int packed_dtype, void* w13_packed, float* w13_scale, void* w3_packed,
                      float* w3_scale, void* stream);
int kmoe_gemm_gate_up(const void* xperm, const float* xperm_scale, int in_dtype, const int32_t* offsets,
                      int E, int d, int F, int64_t max_rows, const void* w13_packed,
                      const float* w13_scale, void* h, void* stream);
/* gate_up with the dispatch gather fused into its A loads: replaces the gather
 * all_inputs = x[sorted_token_idx] + the first two bmm of GroupedExperts.forward
 * (moe.py:255-277).  Permuted row r is x[row_index ? row_index[row_token[r]] :
 * row_token[r]] (x: n_x_rows x d bf16; row_token from kmoe_dispatch, which then
 * need not write xperm).  bf16 only; same result as kmoe_gemm_gate_up on the
 * gathered rows, bit for bit.                                                 */
int kmoe_gemm_gate_up_rows(const void* x, const int32_t* row_index, int64_t n_x_rows, const int32_t* row_token,
                           const int32_t* offsets, int E, int d, int F, int64_t max_rows, const void* w13_packed,
                           void* h, void* stream);
int kmoe_gemm_down(const void* h, const float* h_scale, int in_dtype, const int32_t* offsets, int E,
                   int d, int F, int64_t max_rows, const void* w3_packed, const float* w3_scale,
                   void* y, void* stream);
/* Per-row fp8 quantisation of a bf16 matrix (used between the fp8 GEMMs):
 * scale[r] = amax(|in[r,:]|)/448, out = e4m3(sat(in/scale)), RNE; cols <= 8192. */
int kmoe_quant_rows_fp8(const void* in, int64_t rows, const int32_t* n_rows_dev, int cols, uint8_t* out,
                        float* scale, void* stream);
/* Convenience: gate_up + down on bf16 (the reference's native entry point). */
int kmoe_grouped_swiglu(const void* xperm, const int32_t* offsets, int E, int d, int F, int64_t max_rows,
                        const void* w13_packed, const void* w3_packed, void* h, void* y, void* stream);

/* ------------------------------------------------------------------------ */
/* (d) Combine — replaces the gather/scale/index_add_ tail of GroupedExperts.forward
 * (moe.py:285-292) and _pytorch_scatter_add_experts (moe.py:132-158).
 *   y[o,:] = scale[s] * sum_{j<fan, src[s,j]>=0} w[s,j] * yperm[src[s,j],:],  s = out_map ? out_map[o] : o
 * rows with s < 0 are written as zeros.  fp32 accumulate in fixed j order (no
 * atomics: bit-reproducible), y in y_dtype (BF16 or F32).                    */
int kmoe_combine(const void* yperm, int d, const int32_t* src_row, const float* src_w, int fan,
                 const int32_t* out_map, const float* scale, int64_t T_out, void* y, int y_dtype,
                 void* stream);

/* ------------------------------------------------------------------------ */
/* Capacity-balanced top-k — replaces Router._balanced_topk_assignment
 * (moe.py:353-421), taken by Router.forward when moe_balanced_routing is set
 * (moe.py:443-451).  From fp32 logits (T,E) (kmoe_router with k = 0):
 * k rounds, cap = max(T*k/E, 1); in round r an expert is full when the picks of
 * rounds < r reached cap, and each token takes its best expert (logit descending,
 * equal logits -> lowest index) that it has not picked and is not full, else its
 * best expert not picked yet.  idx (T,k) int64 in pick order; w (T,k) f32 = the
 * picks' softmax probabilities / (their sum + 1e-9).
 * workspace: kmoe_balanced_workspace_bytes (per-round counts; no zeroing needed). */
size_t kmoe_balanced_workspace_bytes(int E, int k);
int kmoe_balanced_topk(const float* logits, int64_t T, int E, int k, int64_t* idx, float* w, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Expert-choice selection — replaces ExpertChoiceRouter.forward (moe.py:494-530).
 * For each sequence b and expert e, select the C tokens of sequence b with the
 * largest fp32 logit (= largest softmax-over-tokens probability; equal logits ->
 * lowest token index first) and write
 *   idx (B,E,C) int64, w (B,E,C) f32 = p / (sum_c p + 1e-9), p = softmax over S.
 * order 1: the C slots in descending order (the reference's topk order, equal
 * logits lowest index first); order 0: in ascending token order (the same tokens
 * and weights; what a layer forward needs, without the sort).
 * Also writes the dispatch/combine tables: row_token (E*B*C, expert-major rows
 * e*B*C + b*C + c -> token b*S + idx), offsets (E+1) and the per-token combine
 * table src_row/src_w (B*S, E): permuted row of (token, expert) or -1.
 * Requires C <= S.  workspace: kmoe_ec_workspace_bytes (B*S*E floats: the logits
 * transposed to (B, E, S), so each (sequence, expert) column is read contiguously). */
size_t kmoe_ec_workspace_bytes(int B, int64_t S, int E);
int kmoe_ec_select(const float* logits, int B, int64_t S, int E, int64_t C, int order, int64_t* idx, float* w,
                   int32_t* row_token, int32_t* offsets, int32_t* src_row, float* src_w, void* workspace,
                   size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Mixture-of-Depths selection — replaces MoDRouter.forward (mod.py:67-122) and
 * the gather/scatter bookkeeping of TransformerBlock.forward (layers.py:148-185).
 *   r[b,s] = x[b,s,:] . w_mod  (fp32 accumulate)
 *   keep the `keep` largest r of each sequence (equal r -> lowest index first),
 *   sel_idx (B,keep) int64 ascending, sel_w (B,keep) f32 = softmax over the kept r
 *   in ascending-index order; token_rows (B*keep) = b*S + sel_idx; out_map (B*S)
 *   = compact index b*keep + i of a kept token, -1 otherwise.
 * x = NULL: `logits` already holds r (e.g. from kmoe_rmsnorm's mod_logits) and
 * only the selection runs (w_mod and d unused).
 * Requires 1 <= keep <= S.  workspace: kmoe_mod_workspace_bytes.            */
size_t kmoe_mod_workspace_bytes(int B, int64_t S);
int kmoe_mod_select(const void* x, int B, int64_t S, int d, const void* w_mod, int64_t keep, float* logits,
                    int64_t* sel_idx, float* sel_w, int32_t* token_rows, int32_t* out_map, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ======================================================================== */
/* Backward pass of the token-choice MoE layer (bf16).  Replaces the autograd
 * backward of Router.forward, GroupedExperts.forward and the aux losses
 * (moe.py:423-462, 213-294, 840-939; SwiGLU ffn.py:17-64) and the gradient the
 * reference's native path never produced (grouped_swiglu_with_grad,
 * moe_arch/kernels/__init__.py:167-244).  The forward saves what these need:
 * kmoe_router_train (pre-activation of the router's hidden layer) and
 * kmoe_gemm_gate_up_rows_gu (pre-activation gate and up values).            */

/* kmoe_router with the pre-activation hidden layer a = x[row(t)] . w_in^T saved
 * to hidden_pre (T, 128) f32 (nullable: then identical to kmoe_router).     */
int kmoe_router_train(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                      const void* w_out, int E, const float* logit_bias, int k, float* logits,
                      int64_t* topk_idx, float* topk_w, float* partials, float* hidden_pre, void* stream);

/* kmoe_gemm_gate_up_rows that also writes g and u (bf16) to gu (max_rows,
 * 2*F_pad) in the packed column order: per 128-column block of f, the 128 gate
 * values then the 128 up values.                                            */
int kmoe_gemm_gate_up_rows_gu(const void* x, const int32_t* row_index, int64_t n_x_rows,
                              const int32_t* row_token, const int32_t* offsets, int E, int d, int F,
                              int64_t max_rows, const void* w13_packed, void* h, void* gu, void* stream);

/* kmoe_gemm_gate_up on fp8 e4m3 rows (xperm codes with per-row scales, w13 packed
 * fp8 with per-column scales) that also writes g and u to gu (max_rows, 2*F_pad)
 * bf16 in the same packed column order, descaled (the values h's SwiGLU took): the
 * straight-through backward of the fp8 experts, whose gradients flow through the
 * dequantised operands as autograd of the fake-quantised forward gives them
 * (fp8_moe.py:179-279 computes its experts in the scaled domain and is
 * differentiated by autograd).  d % 128 == 0.                                  */
int kmoe_gemm_gate_up_fp8_gu(const void* xperm, const float* xperm_scale, const int32_t* offsets, int E, int d,
                             int F, int64_t max_rows, const void* w13_packed, const float* w13_scale, void* h,
                             void* gu, void* stream);

/* Dequantised fp8 rows for the straight-through backward's weight gradients:
 * out[r, :] = bf16(e4m3(q[r, :]) * scale[r]) (out (rows, cols) bf16) for rows r <
 * min(rows, *n_rows_dev) (n_rows_dev nullable).  cols % 8 == 0.  The fake-quantised
 * x and h of the reference's fp8 experts (fp8_moe.py:225-271) as this build's fp8
 * GEMMs take them.                                                            */
int kmoe_dequant_rows_fp8(const uint8_t* q, const float* scale, int64_t rows, const int32_t* n_rows_dev, int cols,
                          void* out, void* stream);

/* w (E, K, N) (bf16 or f32) fake-quantised per output column of each expert as
 * kmoe_pack_weights(fp8) quantises it (scale = column amax / 448, e4m3 codes,
 * saturating, nearest even), dequantised to out (E, K, N) bf16: the weights the
 * fp8 GEMMs multiplied (fp8_moe.py:171-177, 236-268 scale the whole matrix; this
 * build scales each column).                                                  */
int kmoe_fake_quant_e4m3_cols(const void* w, int w_dtype, int E, int K, int N, void* out, void* stream);

/* Combine backward (moe.py:285-292 reversed): for every kept slot r = slot_row[t,j]
 *   dyperm[r] = slot_w[t,j] * dy[t]            (bf16)
 *   dw[t,j]   = dy[t] . yperm[r]               (f32, fixed order; 0 if dropped)
 * yperm: the forward's expert output rows (max_rows, d) bf16.              */
int kmoe_combine_bwd(const void* dy, const void* yperm, const int32_t* slot_row, const float* slot_w, int k,
                     int d, int64_t T, void* dyperm, float* dw, void* stream);

/* kmoe_combine_bwd for a combine that wrote token t's output to row row_index[t] of
 * y, scaled by scale[t] (the MoD composition: the gather of layers.py:160-165, the
 * weighting by the MoD router weights and the scatter_add_ of layers.py:170-184):
 *   dyperm[r] = scale[t] w[t,j] dy[row_index[t]],  dw[t,j] = scale[t] (dy[row_index[t]] . yperm[r]),
 *   dscale[t] = sum_j w[t,j] (dy[row_index[t]] . yperm[r])   (the MoD weight's gradient)
 * row_index NULL = t, scale NULL = 1, dscale nullable.                         */
int kmoe_combine_bwd_rows(const void* dy, const void* yperm, const int32_t* slot_row, const float* slot_w, int k,
                          int d, int64_t T, const int32_t* row_index, const float* scale, void* dyperm, float* dw,
                          float* dscale, void* stream);

/* Backward packed weight layouts (derived caches, like kmoe_pack_weights):
 *   w3n : (E, round_up(F,256), d)       rows of w3 (E,F,d), K = d contiguous
 *   w13t: (E, round_up(d,256), 2*F_pad) rows i of w1/w2 (E,d,F), gate and up
 *         columns interleaved per 128 like the gu order.  WPAD bytes after rows. */
size_t kmoe_packed_w3n_bytes(int E, int d, int F);
size_t kmoe_packed_w13t_bytes(int E, int d, int F);
int kmoe_pack_weights_bwd(const void* w1, const void* w2, const void* w3, int w_dtype, int E, int d, int F,
                          void* w3n_packed, void* w13t_packed, void* stream);

/* Grouped GEMM over the routed rows: c[r, n] = a[r, :] . b_e[n, :] for the rows r of
 * expert e ([offsets[e], offsets[e+1])), K-contiguous a (rows, K) bf16 and packed
 * b (E, b_expert_rows, K + 64) bf16; columns n < n_valid stored, row stride ldc.
 * dh = dyperm . w3^T: b = w3n, K = d, N = F;  dx = dgu . w13t^T: b = w13t,
 * K = 2*F_pad, N = d.                                                        */
int kmoe_gemm_grouped(const void* a, const int32_t* offsets, int E, int K, int64_t max_rows, const void* b_packed,
                      int64_t b_expert_rows, int N, void* c, int64_t ldc, int n_valid, void* stream);

/* SwiGLU backward on the packed order: s = sigmoid(g),
 *   dg = dh * u * s * (1 + g (1 - s)),  du = dh * g * s
 * dh (rows, F_pad), gu / dgu (rows, 2*F_pad) bf16; rows < *n_rows_dev if given. */
int kmoe_swiglu_bwd(const void* dh, const void* gu, int64_t rows, const int32_t* n_rows_dev, int F, void* dgu,
                    void* stream);

/* ------------------------------------------------------------------------ */
/* Non-gated experts — GroupedExperts with an activation other than swiglu
 * (moe.py:187-191,281-283): w1 (E, d, F), w2 (E, F, d), y = silu(x . w1) . w2.
 * Forward: p = kmoe_gemm_grouped(xperm, w1t, K = d, N = F_pad), h = kmoe_silu_rows(p),
 * yperm = kmoe_gemm_grouped(h, w2t, K = F_pad, N = d).  Backward: dh = dyperm . w2^T
 * (w2n, K = d), dp = kmoe_silu_bwd(dh, p), dx = dp . w1^T (w1n, K = F_pad), and the
 * weight gradients with kmoe_gemm_wgrad_rows (dW1 = xperm^T dp, dW2 = h^T dyperm).
 * Packed layouts (bf16, K-contiguous rows, WPAD bytes after every row, zero padded):
 *   w1t (E, round_up(F,256), d):      row f = w1[e][:, f]
 *   w2t (E, round_up(d,256), F_pad):  row n = w2[e][:, n]   (kmoe_packed_w3_bytes, bf16)
 *   w2n (E, round_up(F,256), d):      row f = w2[e][f][:]   (kmoe_packed_w3n_bytes)
 *   w1n (E, round_up(d,256), F_pad):  row i = w1[e][i][:]                           */
size_t kmoe_packed_w1t_bytes(int E, int d, int F);
size_t kmoe_packed_w1n_bytes(int E, int d, int F);
int kmoe_pack_weights_plain(const void* w1, const void* w2, int w_dtype, int E, int d, int F, void* w1t_packed,
                            void* w2t_packed, void* stream);
int kmoe_pack_weights_plain_bwd(const void* w1, const void* w2, int w_dtype, int E, int d, int F, void* w2n_packed,
                                void* w1n_packed, void* stream);
/* h = silu(p) and dp = dh * s * (1 + p (1 - s)), s = sigmoid(p), over (rows, F_pad) bf16
 * (rows < *n_rows_dev if given).                                               */
int kmoe_silu_rows(const void* p, int64_t rows, const int32_t* n_rows_dev, int F, void* h, void* stream);
int kmoe_silu_bwd(const void* dh, const void* p, int64_t rows, const int32_t* n_rows_dev, int F, void* dp,
                  void* stream);

/* Weight gradients read straight from row-major row buffers (no transposes):
 *   c_e[m, n] = sum over expert e's rows r of a[r, m] * b[r, n]
 * a (max_rows, lda) and b (max_rows, ldb) bf16, rows of expert e = [offsets[e],
 * offsets[e+1]); rows past an expert's end read as zero.  c: (E, M, ldc) bf16 (c_dtype
 * BF16) or f32 (F32: the raw fp32 sums, e.g. split-K partials over row segments),
 * columns < n_valid; with c2 (bf16 only; the dW1/dW2 split of the packed order) the
 * columns of 256-column tile nt go to c (first 128) and c2 (last 128) at column
 * nt*128.  N a multiple of 256; n_valid and ldc multiples of 8.  dW3 = h^T dyperm: a = h (lda F_pad), b = dyperm (ldb d), M = F,
 * N = round_up(d, 256);  dW1, dW2: a = the permuted x rows (kmoe_dispatch's xperm),
 * b = dgu (ldb 2*F_pad), M = d, N = 2*F_pad, c = dW1, c2 = dW2.                 */
int kmoe_gemm_wgrad_rows(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t max_rows,
                         const int32_t* offsets, int E, int M, int N, void* c, void* c2, int c_dtype, int64_t ldc,
                         int n_valid, void* stream);

/* out[i] = sum_p partial[p][i] (fp32, in a fixed order: 16 strided partial sums over
 * p = q, q + 16, ..., then those 16 in order; bit-reproducible), bf16 or f32 out. */
int kmoe_reduce_f32(const float* partial, int64_t n_parts, int64_t n, void* out, int out_dtype, void* stream);

/* Router logit gradient (f32, (T,E)): the top-k renormalisation's softmax-over-
 * the-selected backward, dl[i_j] += w_j (dw_j - sum_l w_l dw_l), plus the aux
 * losses scaled by *grad_aux (nullable = 0):
 *   dl += g (w_lb E/T p (f - p.f) + w_z 2/T lse p),  f_e = counts[e] / (T k).
 * k = 0 (topk_idx / topk_w / dw may be NULL): the aux part alone (the expert-choice
 * layer's z-loss, with counts NULL and w_lb 0).                                   */
int kmoe_router_dlogits(const float* logits, int64_t T, int E, const int64_t* topk_idx, const float* topk_w,
                        const float* dw, int k, const int32_t* counts, const float* grad_aux, float w_lb, float w_z,
                        float* dlogits, void* stream);

/* Expert-choice logit gradient added to dlogits (f32, (B*S, E)): the backward of
 * ExpertChoiceRouter.forward's softmax over each sequence's S tokens and per-expert
 * normalisation w = p / (sum_sel p + 1e-9) (moe.py:513-528), at the selection held by
 * the combine tables src_row / src_w (B*S, E) of kmoe_ec_select; dw (B*S, E) is the
 * gradient of each selected slot's weight (kmoe_combine_bwd over those tables).     */
int kmoe_ec_dlogits(const float* logits, int B, int S, int E, const int32_t* src_row, const float* src_w,
                    const float* dw, float* dlogits, void* stream);

/* Backward of MoDRouter.forward (mod.py:93-112) at its selection: with p = sel_w
 * (B, keep), the softmax over each sequence's kept logits, and dsel its gradient
 * (kmoe_combine_bwd_rows' dscale):
 *   dlog[i] = p_i (dsel_i - sum_l p_l dsel_l)     written at dlog[i * dlog_stride]
 *   dw_mod  = sum_i dlog[i] x_sel[i]              (logits = x . w_mod; nullable: skipped)
 * x_sel (B*keep, d) bf16: the kept rows in kmoe_mod_select's order.  Unkept tokens
 * get no logit gradient (top-k is piecewise constant; the MoD auxiliary BCE loss is
 * not part of this build).  workspace: kmoe_mod_bwd_workspace_bytes(B*keep, d).  */
size_t kmoe_mod_bwd_workspace_bytes(int64_t n_rows, int d);
int kmoe_mod_bwd(const float* sel_w, const float* dsel, int B, int64_t keep, const void* x_sel, int d, float* dlog,
                 int64_t dlog_stride, void* dw_mod, int dw_dtype, void* workspace, size_t workspace_bytes,
                 void* stream);

/* RMSNorm of the block boundary (RMSNorm.forward, embeddings.py:167-195; the
 * ffn_norm of TransformerBlock.forward, layers.py:142-147) for the training path:
 *   n[t] = bf16(g * x[t] * r_t),  rrms[t] = r_t = 1/sqrt(mean(x[t]^2) + eps)
 * x (T, d) bf16 or f32, g (d) bf16 or f32; d a multiple of 8, <= 8192.
 * w_mod (d) bf16 and mod_logits (T) f32, both or neither: also the MoD router
 * logits of the normalised rows, mod_logits[t] = n[t] . w_mod (mod.py:93), bit-identical
 * to those kmoe_mod_select computes from n (pass them to it with x = NULL).   */
int kmoe_rmsnorm(const void* x, int x_dtype, const void* weight, int w_dtype, float eps, int64_t T, int d, void* n,
                 float* rrms, const void* w_mod, float* mod_logits, void* stream);
/* Its backward from dn (T, d) bf16 (the gradient of n):
 *   dx[t] = dres[t] + r_t g*dn[t] - (r_t^3 / d) x[t] sum_c g_c dn[t,c] x[t,c]
 *   dweight = sum_t dn[t] * x[t] r_t  (fixed-order reduction)
 * dres (nullable; the residual's gradient of out = x + f(n)) and dx in x's dtype,
 * dweight in dw_dtype.  T = 0 writes dweight = 0 (the row buffers may be NULL).
 * workspace: kmoe_rmsnorm_bwd_workspace_bytes.                               */
size_t kmoe_rmsnorm_bwd_workspace_bytes(int64_t T, int d);
int kmoe_rmsnorm_bwd(const void* dn, const void* x, int x_dtype, const void* weight, int w_dtype, const float* rrms,
                     const void* dres, int64_t T, int d, void* dx, void* dweight, int dw_dtype, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Router MLP backward: da = (dl . w_out) * silu'(a) -> (T, 128) bf16 and
 * dw_out = dl^T silu(a) -> (E, 128) (bf16 or f32), reduced in a fixed order.
 * hidden_pre: a from kmoe_router_train.  workspace: kmoe_router_bwd_workspace_bytes.
 * dw_in = da^T x and dx += da . w_in follow with kmoe_gemm_wgrad_rows / kmoe_gemm_grouped
 * (w_in^T packed by kmoe_pack_w_in_t).                                       */
size_t kmoe_router_bwd_workspace_bytes(int64_t T, int E);
int kmoe_router_mlp_bwd(const float* dlogits, const float* hidden_pre, int64_t T, int E, const void* w_out,
                        void* da, void* dw_out, int dw_dtype, void* workspace, size_t workspace_bytes,
                        void* stream);
size_t kmoe_packed_w_in_t_bytes(int d);
int kmoe_pack_w_in_t(const void* w_in, int w_dtype, int d, void* out, void* stream);

/* ------------------------------------------------------------------------ */
/* Layer-boundary fusions: the FFN half of TransformerBlock.forward
 * (layers.py:142-147, 184-187), out = h + MoE(RMSNorm(h)), with RMSNorm
 * (embeddings.py:167-195: y = w_norm * x / sqrt(mean(x^2) + eps)) folded into the
 * router and the gate/up GEMM, and the residual add folded into the combine.
 * The caller folds the norm weight into the weights once per parameter version:
 *   w_in_g[j][i] = w_in[j][i] * w_norm[i];  w13 = kmoe_pack_weights(w1 * w_norm[:,None],
 *   w2 * w_norm[:,None], w3, ...).  x is then the un-normalised h.           */

/* kmoe_router_train (hidden_pre nullable) that also writes each block's per-expert
 * routed counts to block_counts (ceil(T/B) * E int32, B = kmoe_router_block_tokens(T);
 * k >= 1), the
 * histograms kmoe_dispatch_counted takes: the router already holds every token's
 * top-k, so the dispatch need not read topk_idx a second time to count them.      */
int kmoe_router_hist(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                     const void* w_out, int E, const float* logit_bias, int k, float* logits, int64_t* topk_idx,
                     float* topk_w, float* partials, float* hidden_pre, int32_t* block_counts, void* stream);

/* kmoe_router on RMSNorm(x): w_in_g carries the norm weight; the kernel computes
 * rscale[t] = 1/sqrt(mean(x[row(t)]^2) + eps) (f32, (T,)) from the x rows it reads and
 * scales the hidden pre-activation by it (replaces the separate norm pass).   */
int kmoe_router_rms(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in_g,
                    const void* w_out, int E, const float* logit_bias, int k, float* logits,
                    int64_t* topk_idx, float* topk_w, float* partials, float eps, float* rscale, void* stream);

/* kmoe_gemm_gate_up_rows on RMSNorm(x): the gate and up values of permuted row r are
 * scaled by rscale[row_token[r]] before the SiLU (w13 packed from the norm-folded
 * w1 / w2).  The normalised rows are never written.                           */
int kmoe_gemm_gate_up_rows_scaled(const void* x, const int32_t* row_index, int64_t n_x_rows,
                                  const int32_t* row_token, const int32_t* offsets, int E, int d, int F,
                                  int64_t max_rows, const void* w13_packed, const float* rscale, void* h,
                                  void* stream);

/* kmoe_combine plus a residual (y's dtype, (T_out, d)), added in f32 before the one
 * rounding: y[o] = residual[o] + scale[s] sum_j w[s,j] yperm[src[s,j]]; rows with
 * out_map[o] < 0 get residual[o].  residual may be NULL (= kmoe_combine).
 * residual and y must not overlap unless they are the same buffer.            */
int kmoe_combine_residual(const void* yperm, int d, const int32_t* src_row, const float* src_w, int fan,
                          const int32_t* out_map, const float* scale, const void* residual, int64_t T_out,
                          void* y, int y_dtype, void* stream);

/* kmoe_combine_residual with the block's residual dropout (replaces residual +
 * residual_dropout(ffn_output), moe_arch/model/layers.py:187-190, nn.Dropout(p) in
 * training): y[o] = residual[o] + keep[o] * keep_scale * scale[s] sum_j w[s,j]
 * yperm[src[s,j]], one rounding.  keep: (T_out, d) bytes, nonzero = kept (the
 * Bernoulli(1-p) draw); keep_scale = 1/(1-p) >= 1.  residual and keep are required. */
int kmoe_combine_residual_dropout(const void* yperm, int d, const int32_t* src_row, const float* src_w, int fan,
                                  const int32_t* out_map, const float* scale, const void* residual,
                                  const uint8_t* keep, float keep_scale, int64_t T_out, void* y, int y_dtype,
                                  void* stream);


#ifdef __cplusplus
}
#endif

#endif /* KMOE_H */
