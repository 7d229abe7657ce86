/*
 * octo_head.h — C ABI of libocto_head.so, the gfx950 (MI355X) LM-head logprob path.
 *
 * The path: for packed, prefix-deduplicated hidden rows h_r (d wide), labels y_r and the vocabulary
 * weight W [V, d], compute per row
 *     z = post(h_r . W^T),  s = z / T,  lse = log sum_j exp(s_j),
 *     logprob = s_y - lse,  entropy = lse - sum_j p_j s_j     (p = exp(s - lse), entropy detached)
 * without ever writing the [rows, V] logits, and the backward of a loss L(logprob):
 *     dL/dz_rj = g_r (1[j = y_r] - p_rj) / T * post'(z_rj),   g_r = dL/dlogprob_r
 *     grad_h = dz . W,   grad_W = dz^T . h.
 *
 * Every entry point
 *   - returns an int status (OCTO_OK or a negative OCTO_E* code) and never throws;
 *     octo_last_error() gives a message for the last failing call on the calling thread;
 *   - takes plain device pointers, element strides and sizes, and an explicit hipStream_t
 *     (passed as void* so that the header needs no HIP include); all work is queued on that stream.
 *     Outputs and the workspace are ordinary device memory (hipMalloc, coarse-grained): sums into
 *     fp32 outputs (the loss, grad_W accumulated across row passes or into the caller's fp32 gradient)
 *     use the GPU's hardware float atomics, which fine-grained (host-coherent) memory does not take;
 *   - allocates no device memory: scratch memory comes from a caller-provided workspace whose size the
 *     matching *_workspace_bytes query returns (the one exception is the timing hook below, which
 *     creates HIP events while it is enabled);
 *   - does no device-to-host synchronisation: row counts produced on the device (octo_compact_rows)
 *     are read by the kernels themselves.
 *
 * Reference interfaces replaced (shatianming5/octopus):
 *   octopus/rl/lm_head.py:102-105  _head_chunk      -> octo_head_fwd (GEMM + fused epilogue)
 *   octopus/rl/lm_head.py:108-112  _head_columns    -> octo_columns_fwd / octo_columns_bwd
 *   octopus/rl/lm_head.py:115-121  _chunked_rows    -> octo_head_fwd + octo_head_bwd (no chunk loop,
 *                                                     no checkpoint: the backward recomputes by design)
 *   octopus/rl/lm_head.py:124-130  _scored_rows     -> octo_compact_rows + OCTO_ROWS_VIA_IDX /
 *                                                     OCTO_OUT_SCATTER modes of octo_head_fwd
 *   octopus/rl/prefix_tree.py:416-421 tree_head_output -> octo_pairs_expand / octo_pairs_grad
 *   octopus/rl/prefix_tree.py:156-166 build_tree, label-pair section (np.unique over packed
 *                                     (position, label)) -> octo_label_pairs
 *   AReaL grpo_loss_fn (cited by docs/rl-plan-episodes.md:496-497, constants grpo.yaml:103-118)
 *                                                  -> octo_grpo_grad, or fused into the forward's
 *                                                     last step: octo_head_fwd_grpo
 *   octopus/rl/actor.py:343-347 (AReaL's grpo_loss_fn reads the head's columns, then loss.backward()
 *     runs lm_head.py:115-121's checkpoint recompute) -> octo_head_step_grpo (forward, GRPO loss and
 *                                                     backward in one call, the logits computed once per
 *                                                     row pass); over a tree's pair rows (tree_head_output,
 *                                                     prefix_tree.py:416-421): octo_head_step_grpo_pairs
 *   octopus/rl/actor.py:166-171, 343-347 unchanged (bind_head's own pre-hook binds the micro-batch's GRPO
 *     inputs; AReaL's loss.backward() reaches the head's backward) -> octo_head_step_grpo in the forward,
 *                                                     and in the backward octo_grpo_fit, octo_scale_add of
 *                                                     its gradients, and octo_head_bwd of the rest of
 *                                                     dL/dlogprob (its kernels end at once when that rest
 *                                                     is negligible)
 */
#ifndef OCTO_HEAD_H
#define OCTO_HEAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------------- */
#define OCTO_OK            0
#define OCTO_EINVAL       -1 /* bad shape, stride, pointer or dtype combination (ValueError)      */
#define OCTO_EWORKSPACE   -2 /* workspace smaller than the query returned (ValueError)             */
#define OCTO_EUNSUPPORTED -3 /* dtype or option the kernels do not implement (NotImplementedError) */
#define OCTO_EHIP         -4 /* HIP runtime error while queueing work (RuntimeError)               */

/* ---- element types ------------------------------------------------------------------------ */
#define OCTO_BF16   0
#define OCTO_F16    1
#define OCTO_F32    2
#define OCTO_FP8E4M3 3 /* OCP e4m3 (torch.float8_e4m3fn); weights only, with one fp32 scale per row */

/* ---- flags -------------------------------------------------------------------------------- */
#define OCTO_ROWS_VIA_IDX     1  /* labels[] are per hidden row: row r uses labels[idx[r]]            */
#define OCTO_OUT_SCATTER      2  /* out2 row for compact row r is idx[r] (else r)                     */
#define OCTO_GRADW_ACCUMULATE 4  /* grad_w += contribution (else grad_w = contribution)               */
#define OCTO_WS_BACKWARD      8  /* octo_head_workspace_bytes: size for octo_head_bwd                 */
#define OCTO_WS_NO_GRADW     16  /* octo_head_workspace_bytes: backward without grad_w                */
#define OCTO_WS_GATHER       32  /* octo_head_workspace_bytes: add a contiguous copy of the n_max rows  */
                                 /* read through idx; needed when h_rows * ldh * element bytes >= 2^31  */
#define OCTO_LSE_PAIR        64  /* head fwd/bwd: lse holds 2 floats per row, (m2, l2S): the row's       */
                                 /* base-2 maximum of s log2(e) and log2 of the shifted sum, lse =       */
                                 /* (m2 + l2S) ln 2; the backward then repeats the forward's rounding    */
                                 /* (exact dz row sums when the logits sit far from zero)                */
#define OCTO_WS_STEP        128  /* octo_head_workspace_bytes / octo_head_bwd_plan: for octo_head_step_grpo */
#define OCTO_WS_NO_GRADH    256  /* octo_head_workspace_bytes / octo_head_bwd_plan: without grad_h        */
#define OCTO_PAIRS_NONE_AS_COUNT 1 /* octo_label_pairs: positions without a pair get the pair count  */

const char *octo_version(void);
const char *octo_last_error(void);

/* Kernel timing hook (no counterpart in the reference: a measurement aid for benchmarks). While enabled,
 * every GEMM launch of octo_head_fwd / octo_head_bwd / octo_head_step_grpo is bracketed by HIP events on its
 * stream, under the names "gemm_stats", "gemm_dz", "gemm_store_grad_h" and "gemm_store_grad_w" (and the step's
 * "gemm_grads", "ex_fix" and, for f16 operands, "dz_scale"). octo_timing_read waits for
 * the recorded launches of one name and returns their count and summed duration. octo_timing_enable
 * (either value) discards what was recorded. Off by default; enabling it creates events (allocates). */
int octo_timing_enable(int on);
int octo_timing_read(const char *kernel, int *launches, double *total_ms);

/* Workspace bytes for octo_head_fwd (flags without OCTO_WS_BACKWARD) or octo_head_bwd
 * (OCTO_WS_BACKWARD [| OCTO_WS_NO_GRADW | OCTO_WS_NO_GRADH]) at n_max rows, width d, vocabulary V. With idx, a hidden matrix of
 * 2 GiB or more (h_rows * ldh * element bytes >= 2^31) is first gathered into the workspace (the GEMMs address
 * mapped rows with 32-bit offsets): add OCTO_WS_GATHER for those calls.
 * Backward: the size of its plan at a 2 GiB staging budget (see octo_head_bwd); a smaller workspace is accepted
 * down to the plan at a 1 MiB budget, a larger one may run fewer chunks. OCTO_WS_STEP [| OCTO_WS_NO_GRADW |
 * OCTO_WS_NO_GRADH]: for octo_head_step_grpo and octo_head_step_grpo_pairs (n_max = the pair rows), whose plan has
 * row passes only, each pass's [rows, V] exponentials within the 2 GiB staging budget (a larger workspace runs larger
 * passes); for fp32 operands the larger of the forward's and the backward's. */
int octo_head_workspace_bytes(int64_t n_max, int d, int V, int w_dtype, int flags, size_t *bytes);

/* The chunking octo_head_bwd runs in ws_bytes of workspace (a planning aid; no counterpart in the reference):
 * plan[0] rows per pass, plan[1] passes, plan[2] vocabulary columns per chunk, plan[3] chunks. flags as for
 * octo_head_workspace_bytes (OCTO_WS_NO_GRADW, OCTO_WS_NO_GRADH, OCTO_WS_GATHER). With OCTO_WS_STEP, the
 * fused step's plan: {rows per pass, passes, V rounded up to 256, 1}. OCTO_EWORKSPACE when no plan fits. */
int octo_head_bwd_plan(int64_t n_max, int d, int V, int w_dtype, int flags, size_t ws_bytes, int64_t plan[4]);

/* Masked-row compaction (lm_head.py:128 `scored.nonzero()[:, 0]`): idx[0..count) = the positions
 * r < n with mask[r] != 0, ascending; *count written on the device. idx must hold n entries;
 * entries at and after *count are left unspecified. */
int octo_compact_rows(const uint8_t *mask, int64_t n, int64_t *idx, int32_t *count, void *stream);

/* Forward: logprob, entropy and lse of each compact row r < *count (or n_max when count is NULL).
 *   hidden row of r  : h + (idx ? idx[r] : r) * ldh          (h_dtype BF16, F16 or F32);
 *                      h holds h_rows rows and every idx[r] must be below h_rows
 *   weight           : w [V, ldw] (w_dtype = h_dtype, or FP8E4M3 with w_scale[V] and BF16 h)
 *   label of r       : labels[(flags & OCTO_ROWS_VIA_IDX) ? idx[r] : r], int64 in [0, V)
 *   post-head logits : z' = use_tanh ? post * tanh(pre * z) : post * pre * z;  s = z' * inv_T
 *   outputs          : logp[r], ent[r], lse[r] (any may be NULL; lse[2 r], lse[2 r + 1] under
 *                      OCTO_LSE_PAIR) and, if out2 != NULL,
 *                      out2[row * ld_out2 + {0,1}] = {logp, entropy} with row = idx[r] under
 *                      OCTO_OUT_SCATTER, else r. Rows of out2 not written are left untouched.
 * Requires d % 8 == 0 (bf16/f16), d % 16 == 0 (fp8) or d % 4 == 0 (f32), inv_T > 0, pre * post > 0 when !use_tanh. */
int octo_head_fwd(const void *h, int64_t h_rows, int64_t ldh, int h_dtype,
                  const void *w, int64_t ldw, int w_dtype, const float *w_scale,
                  const int64_t *labels, const int64_t *idx, const int32_t *count,
                  int64_t n_max, int d, int V, int flags,
                  float inv_T, float pre, float post, int use_tanh,
                  float *logp, float *ent, float *lse, float *out2, int64_t ld_out2,
                  void *ws, size_t ws_bytes, void *stream);

/* octo_head_fwd without a workspace argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). No counterpart in the reference. Its workspace is
 * a 64 MiB device array inside the library, one copy per GPU, held until the process ends; the call allocates
 * nothing (no hipMalloc, no timing events). Limit: the forward's workspace for n_max, d, V (octo_head_workspace_bytes
 * with the same flags) must be at most 64 MiB, about 7,000 rows at V = 151,936, else OCTO_EINVAL before anything is
 * queued. Every call on one GPU uses the same array: calls that overlap on one GPU (other streams or threads) race;
 * calls on one stream are ordered. Nothing in the array needs clearing between calls. */
int octo_head_fwd_noalloc(const void *h, int64_t h_rows, int64_t ldh, int h_dtype,
                          const void *w, int64_t ldw, int w_dtype, const float *w_scale,
                          const int64_t *labels, const int64_t *idx, const int32_t *count,
                          int64_t n_max, int d, int V, int flags,
                          float inv_T, float pre, float post, int use_tanh,
                          float *logp, float *ent, float *lse, float *out2, int64_t ld_out2, void *stream);

/* Backward of octo_head_fwd's logprob column (the entropy column carries no gradient):
 *   g[r]   : dL/dlogprob of compact row r (fp32, compact order)
 *   lse[r] : from octo_head_fwd on the same inputs (the pair form under OCTO_LSE_PAIR, given to both calls)
 *   grad_h : NULL or [n_max, ld_gh] of gh_dtype (BF16, F16 or F32), compact order; rows at and
 *            after *count are left unspecified
 *   grad_w : NULL or [V, d] (row stride d) of gw_dtype (BF16, F16 or F32); = or += (OCTO_GRADW_ACCUMULATE),
 *            summed in fp32 and rounded once to gw_dtype. Not available for FP8E4M3 weights.
 * The logits are recomputed tile by tile; dz = g (onehot - p) / T is staged in the workspace (bf16 / f16 / f32)
 * one (row pass, vocabulary chunk) at a time: passes of at most 32,768 rows, chunks of a multiple of 256 columns
 * as wide as the staging budget allows. The staging (dz, fp32 grad_h partials across chunks, the chunk's W^T or
 * widened fp8 rows) stays within the budget; outside it are h^T of a pass [d, rows] and, over several passes with
 * a 16-bit grad_w, fp32 grad_w partials [V, d]. The plan is the largest that fits ws_bytes (octo_head_bwd_plan);
 * fp32 sums across chunks and passes follow it, so results are reproducible for a given workspace size. */
int octo_head_bwd(const void *h, int64_t h_rows, int64_t ldh, int h_dtype,
                  const void *w, int64_t ldw, int w_dtype, const float *w_scale,
                  const int64_t *labels, const int64_t *idx, const int32_t *count,
                  int64_t n_max, int d, int V, int flags,
                  float inv_T, float pre, float post, int use_tanh,
                  const float *lse, const float *g,
                  void *grad_h, int64_t ld_gh, int gh_dtype, void *grad_w, int gw_dtype,
                  void *ws, size_t ws_bytes, void *stream);

/* _head_columns on materialised logits [n, ld] (dtype BF16, F16 or F32):
 * out2[r] = {log_softmax(s)[y_r], entropy}, s = logits * inv_T; the row state saved (may be NULL) as two floats
 * per row, lse[2 r] = m2 (the row's maximum of s log2(e)) and lse[2 r + 1] = l2S (log2 of the shifted sum):
 * lse = (m2 + l2S) ln 2, and octo_columns_bwd repeats the forward's rounding with it. */
int octo_columns_fwd(const void *logits, int64_t ld, int dtype, const int64_t *labels,
                     int64_t n, int V, float inv_T, float *out2, float *lse, void *stream);
/* dlogits[r, j] = g[r] * (1[j = y_r] - p_rj) * inv_T, written in dtype at stride ld_d; lse: octo_columns_fwd's
 * row state (2 floats per row). */
int octo_columns_bwd(const void *logits, int64_t ld, int dtype, const int64_t *labels,
                     int64_t n, int V, float inv_T, const float *lse, const float *g,
                     void *dlogits, int64_t ld_d, void *stream);

/* Pair expansion (prefix_tree.py:419-421): out[t, :C] = pairs[flat_pair[t], :C] when
 * 0 <= flat_pair[t] < P, else 0. */
int octo_pairs_expand(const float *pairs, int64_t P, int C, const int64_t *flat_pair, int64_t T,
                      float *out, void *stream);
/* Its backward: grad_pairs[p, :C] = sum of grad_flat[t, :C] over t with flat_pair[t] == p
 * (grad_pairs is overwritten). */
int octo_pairs_grad(const float *grad_flat, int64_t T, int C, const int64_t *flat_pair, int64_t P,
                    float *grad_pairs, void *stream);

/* Label pairs of a prefix tree (prefix_tree.py:156-166), on the device. Flat position p asks when
 * scored[p] != 0 (scored NULL: every p), p + 1 < T_flat and p is not the last position of its
 * sequence (p != cu[s + 1] - 1 for any s < n_seq; cu holds n_seq + 1 device offsets, a -1 read as the
 * last flat position); its ask is (flat_to_tree[p], flat[p + 1]). Distinct asks are the pairs, numbered in
 * ascending (tree position, label) order:
 *   pair_pos[i], pair_label[i]  for i < P (both hold at least T_flat entries; later ones unspecified);
 *   flat_pair[p]                the pair of p's ask, else -1 (OCTO_PAIRS_NONE_AS_COUNT: P, the index of the
 *                               appended zero row of prefix_tree.py:203-205);
 *   count[0] = P, count[1] = asks whose flat_to_tree entry lies outside [0, T_tree) (ignored; 0 for a
 *                               valid tree). Both written on the device.
 * flat and flat_to_tree hold T_flat entries; T_flat, T_tree < 2^31. ws: octo_label_pairs_workspace_bytes. */
int octo_label_pairs_workspace_bytes(int64_t T_flat, int64_t T_tree, size_t *bytes);
int octo_label_pairs(const int64_t *flat, int64_t T_flat, const int64_t *cu, int64_t n_seq,
                     const int64_t *flat_to_tree, int64_t T_tree, const uint8_t *scored,
                     int64_t *pair_pos, int64_t *pair_label, int64_t *flat_pair, int32_t *count,
                     int flags, void *ws, size_t ws_bytes, void *stream);

/* dst[idx[r], :d] (+)= src[r, :d] for r < *count, with idx ascending (repeats allowed: the rows of
 * one run are summed in fp32 first). dst rows not named by idx are untouched; accumulate != 0 adds
 * to dst. src/dst dtypes BF16, F16 or F32. */
int octo_rows_scatter(const void *src, int64_t ld_src, int src_dtype, const int64_t *idx,
                      const int32_t *count, int64_t n_max, int d,
                      void *dst, int64_t ld_dst, int dst_dtype, int accumulate, void *stream);

/* y[i] = c y[i] + x[i] for i < n, with c = *c read on the device, formed in fp32 and rounded once to dtype (BF16, F16
 * or F32); while skip_x is given and *skip_x != 0, or x is NULL, x counts as zero and is not read (c = 1 then leaves y
 * as it is at once). y and x 16-byte aligned. No counterpart in the reference, whose autograd sums the chunks' gradients: the
 * backward of the bound GRPO step (octopus_amd/head_op.py) uses it to scale the gradients its forward computed by the
 * incoming gradient's multiple of the head's own GRPO weight and add the backward of the rest. */
int octo_scale_add(void *y, const void *x, int dtype, int64_t n, const float *c, const int32_t *skip_x,
                   void *stream);

/* The bound GRPO step's fit of the incoming dL/dlogprob, on the device: a[r] = src[idx[r] * ld_src] (src[r * ld_src]
 * without idx) for r < *count (all n without count), 0 past it; c = <a, g_head> / <g_head, g_head> (0 when g_head is
 * 0); rest[r] = a[r] - c g_head[r] for r < n; and when ||rest|| <= tol ||a||, *count_rest = 0 and *skip = 1 (the
 * rest's octo_head_bwd then ends at once), else *count_rest = the row count and *skip = 0. One workgroup, sums in a
 * fixed order. No counterpart in the reference: the backward of the bound GRPO step (octopus_amd/head_op.py) runs it
 * in place of a dozen small tensor operations. */
int octo_grpo_fit(const float *src, int64_t ld_src, const int64_t *idx, const float *g_head, int64_t n,
                  const int32_t *count, float tol, float *c, float *rest, int32_t *count_rest, int32_t *skip,
                  void *stream);

/* out[r] = src[idx[r] * ld_src] (fp32) for r < *count, 0 for count <= r < n_max. */
int octo_gather_f32(const float *src, int64_t ld_src, const int64_t *idx, const int32_t *count,
                    int64_t n_max, float *out, void *stream);

/* Per-row e4m3 quantisation of a weight matrix w [V, ldw] (BF16, F16 or F32) into the fp8 weight format that
 * octo_head_fwd / octo_head_bwd take (FP8E4M3 with w_scale):
 *   scale[v] = max(max_k |w[v, k]| / 448, 1e-12)                               (fp32; 448 = largest e4m3)
 *   q[v * ldq + k] = e4m3(clamp(w[v, k] / scale[v], -448, 448))               (nearest, ties to even)
 * for k < d; d % 4 == 0, rows and q aligned to 4 elements. The reference has no quantiser: this produces the
 * weight format of its fp8-weight configuration (per-row scale = absmax / 448) on the device. */
int octo_quantise_fp8_rows(const void *w, int64_t ldw, int w_dtype, int64_t V, int d,
                           uint8_t *q, int64_t ldq, float *scale, void *stream);

/* octo_head_fwd followed, in its last kernel, by the GRPO weight of each compact row: what octo_grpo_grad computes
 * for the row's flat token t = (idx ? idx[r] : r) from the row's logprob (the same per-token formula), written in
 * compact order, so octo_head_bwd can take g directly. Replaces lm_head.py:102-112 (_head_chunk + _head_columns,
 * as octo_head_fwd) plus the consumer of the head's column 0, AReaL's grpo_loss_fn (docs/rl-plan-episodes.md:
 * 496-497, grpo.yaml:103-118): dL/dlogprob without a second pass over the tokens.
 *   grpo->prox, old      : [n_tokens] or NULL (as octo_grpo_grad); adv, mask: [n_tokens]
 *   Z                    : max(1, count of mask[t] != 0 over all n_tokens) (not only the compact rows)
 *   grpo->g              : [n_max] fp32, g[r] = dL/dlogp of row r's token (0 when mask[t] == 0 or t >= n_tokens);
 *                          rows at and after *count are left untouched
 *   grpo->loss           : NULL or one float, L over the compact rows (the tokens with mask != 0 must be among
 *                          them for L to be the whole objective); summed with atomics, so its last bits may vary
 * Workspace as octo_head_fwd. */
typedef struct octo_grpo_tail {
  const float *prox, *old, *adv, *mask;
  int64_t n_tokens;
  float eps_lo, eps_hi, reject_upper;
  float *g, *loss;
} octo_grpo_tail;
int octo_head_fwd_grpo(const void *h, int64_t h_rows, int64_t ldh, int h_dtype,
                       const void *w, int64_t ldw, int w_dtype, const float *w_scale,
                       const int64_t *labels, const int64_t *idx, const int32_t *count,
                       int64_t n_max, int d, int V, int flags,
                       float inv_T, float pre, float post, int use_tanh,
                       float *logp, float *ent, float *lse, float *out2, int64_t ld_out2,
                       const octo_grpo_tail *grpo, void *ws, size_t ws_bytes, void *stream);

/* The GRPO training step of the head in one call: octo_head_fwd_grpo's outputs (logp, ent, lse, out2, grpo->g,
 * grpo->loss, with the same arguments and meaning) and octo_head_bwd's gradients for g = grpo->g (grad_h, grad_w,
 * ld_gh, gh_dtype, gw_dtype and OCTO_GRADW_ACCUMULATE as there; NULL skips one). lse must not be NULL (the pair
 * form under OCTO_LSE_PAIR, as for the backward). The gradients are those of grpo->loss; a caller whose loss is
 * c L scales them by c.
 * The rows run in passes of at most 32,768 (as many as the staging budget holds, balanced). The forward GEMM of a
 * pass stores each element's exponential [rows, V rounded up to 256] in the MFMA type. bf16 (and fp8 weights): as
 * exp2(s log2 e - o_r) x post'(z) (x the fp8 row scale) relative to a per-row offset o_r set before the pass, the
 * row's fp32 label logit (base 2) + 48, so that dz = -g exp2(o_r - m2 - l2S) / T x the stored value is one scale per
 * row: grad_h = dz . W takes it in its store and grad_W = dz^T . h through h^T scaled by it (rounded once to bf16);
 * the merge writes the label entry from the fp32 target logit, and a row whose maximum lies more than 112 (base 2)
 * above its label logit is rescaled to o_r = m2 after the merge. f16: relative to the maximum of each 128-column half
 * tile, then scaled into dz by -g exp2(m_h - m2 - l2S) / T once the merge has the rows' (m2, l2S) and g. grad_h and
 * grad_W run as in octo_head_bwd (both in one launch per pass). The logits are computed once instead of twice; dz
 * differs from octo_head_bwd's by the rounding of the stored value (bf16: 2^-9 relative, in place of the backward's
 * rounding of dz; f16: 2^-11 relative, besides it), and bf16 grad_W by the rounding of the scaled h^T as well.
 * Workspace: octo_head_workspace_bytes with OCTO_WS_STEP [| OCTO_WS_NO_GRADW | OCTO_WS_NO_GRADH | OCTO_WS_GATHER],
 * matching the gradients asked for, the plan at a
 * 2 GiB staging budget ([rows, V] of one pass); outside the staging are the pass's statistics per vocabulary tile,
 * h^T of a pass, fp32 grad_w partials [V, d] over several passes, and once per call W widened to bf16 (fp8 weights)
 * and W^T (16-bit weights with V % 64 or d % 256 not 0; and, for speed, when grad_h is the only gradient and
 * n_max >= 16,384). A smaller workspace is accepted down to the plan at a 1 MiB budget (without the optional W^T
 * first, before smaller passes); octo_head_bwd_plan with OCTO_WS_STEP gives {rows per pass, passes, V rounded up
 * to 256, 1}.
 * fp32 operands run octo_head_fwd_grpo, then octo_head_bwd, in the same workspace. With grad_h and grad_w both
 * NULL the call is octo_head_fwd_grpo (whose workspace size then suffices). */
int octo_head_step_grpo(const void *h, int64_t h_rows, int64_t ldh, int h_dtype,
                        const void *w, int64_t ldw, int w_dtype, const float *w_scale,
                        const int64_t *labels, const int64_t *idx, const int32_t *count,
                        int64_t n_max, int d, int V, int flags,
                        float inv_T, float pre, float post, int use_tanh,
                        float *logp, float *ent, float *lse, float *out2, int64_t ld_out2,
                        const octo_grpo_tail *grpo,
                        void *grad_h, int64_t ld_gh, int gh_dtype, void *grad_w, int gw_dtype,
                        void *ws, size_t ws_bytes, void *stream);

/* octo_head_step_grpo over a prefix tree's deduplicated (position, label) pair rows (prefix_tree.py:156-166,
 * 416-421: the rows tree_head_output runs the head on): compact row r is hidden row pair_pos[r] with label
 * pair_label[r], r < *pair_count (or n_pairs); flat token t takes pair row flat_pair[t] (none when negative or at or
 * past the row count). The GRPO tail's arrays (prox, old, adv, mask; n_tokens of them) are per flat token, so a pair
 * row's g is the sum of its flat tokens' dL/dlogprob and the loss sums over the flat tokens. out_flat [n_flat,
 * ld_out] receives each flat token's (logprob, entropy), 0 for a token with no pair (a masked one adds its loss term
 * at logprob 0, as the objective over the expanded columns does); lse and grpo->g are per pair row
 * (grpo->g complete, also past the count: 0); grad_h [n_pairs, ld_gh] per pair row (rows of one tree position are
 * summed by the caller's scatter). g and the loss are sums of float atomics: their last bits may vary run to run.
 * flags: OCTO_LSE_PAIR only (labels are per pair row). 16-bit operands; workspace as octo_head_step_grpo. */
int octo_head_step_grpo_pairs(const void *h, int64_t h_rows, int64_t ldh, int h_dtype,
                              const void *w, int64_t ldw, int w_dtype, const float *w_scale,
                              const int64_t *pair_label, const int64_t *pair_pos, const int32_t *pair_count,
                              int64_t n_pairs, int d, int V, int flags,
                              float inv_T, float pre, float post, int use_tanh, float *lse,
                              const int64_t *flat_pair, int64_t n_flat, float *out_flat, int64_t ld_out,
                              const octo_grpo_tail *grpo,
                              void *grad_h, int64_t ld_gh, int gh_dtype, void *grad_w, int gw_dtype,
                              void *ws, size_t ws_bytes, void *stream);

/* GRPO/PPO policy-gradient weight per token (AReaL grpo_loss_fn semantics):
 *   ratio r = exp(logp - prox)          (prox == NULL: prox = logp, i.e. reuse_train_logp)
 *   behaviour weight w = exp(prox - old) when old != NULL (decoupled loss), else 1;
 *                    w = 0 where reject_upper > 0 and w > reject_upper
 *   L = sum_t mask_t * w_t * max(-A_t r_t, -A_t clip(r_t, 1 - eps_lo, 1 + eps_hi)) / Z,
 *   Z = max(1, count of mask_t != 0)
 *   g[t] = dL/dlogp[t] (ties of the max split evenly, as torch.maximum's backward)
 * loss (NULL or one float) receives L. ws needs octo_grpo_workspace_bytes() bytes. */
int octo_grpo_workspace_bytes(size_t *bytes);
int octo_grpo_grad(const float *logp, const float *prox, const float *old, const float *adv,
                   const float *mask, int64_t n, float eps_lo, float eps_hi, float reject_upper,
                   float *g, float *loss, void *ws, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* OCTO_HEAD_H */
