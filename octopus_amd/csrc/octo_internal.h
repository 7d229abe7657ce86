// Internal interfaces between the C ABI (head_abi.hip) and the kernel translation units.
#pragma once

#include "octo_common.h"

namespace octo {

struct Operand;
struct GemmShape;

// gemm_stats epilogue arguments: part[row * mtiles + mt] = (m_a, S, U, m_b) of row over vocab tile mt: m_a and m_b
// the base-2 maxima of the tile's first and last 128 vocabulary rows (m_b = -inf when none of those is below V), S and
// U the online-softmax sums relative to max(m_a, m_b). The GEMM's first operand holds the vocabulary rows v0 .. (a
// chunk of W starting at row v0, a multiple of 256): its tile mt is vocab tile v0 / 256 + mt.
//
// With ex != NULL (16-bit operands) the epilogue also stores, per element, its exponential relative to its half
// tile's maximum (m_h = m_a or m_b),
//   ex[token][v] = exp2(c t - m_h) x post'(z)
// token-major in f16 (columns v of the vocabulary, rows = the GEMM's tokens, ldx elements apart; zero past V and past
// the tile's valid tokens), the same exp2 the sums use. Once the row's (m2, l2S) and g are known, dz = -g gmul
// exp2(m_h - m2 - l2S) ex x (fp8 row scale) (the fused step, launch_dz_scale). f16 for any MFMA type: the values lie
// in [0, 1], where f16 keeps 11 bits to bf16's 8; what it rounds in its subnormal range, below 2^-14 of the half
// tile's largest probability, errs by at most 2^-25 of it per element.
//
// With xoff != NULL as well (bf16 operands, the fused step's row-offset form) the stored value is bf16 and relative to
// a per-token offset xoff[token] (base-2 units) chosen before the GEMM, instead of the half tile's maximum:
//   ex[token][v] = exp2(c t - m_h) x exp2(min(m_h - xoff[token], kExClamp)) x post'(z) (x fp8 row scale of v),
// which is exp2(c t - xoff) x post'(z) (x scale) for every element of a token whose maximum m2 lies at most kExClamp
// above its offset. dz is then one scale per token times the stored value: dz = s[token] ex, s = -g gmul exp2(xoff
// - m2 - l2S), except at the label (launch_merge writes that entry); a token whose maximum lies further above its
// offset is rescaled by launch_ex_fix. bf16 keeps 8 exponent bits: with the offset kExAbove above the label's own
// logit (<= m2), every element within 2^-40 of the row's largest stays a normal number.
struct StatsArgs {
  f32x4 *part;
  int64_t mtiles;
  int64_t v0;
  int64_t V;
  const float *wscale;  // per-vocab-row scale (fp8 weights) or NULL
  float c;              // base-2 softmax scale of the (transformed) logit
  float pre;            // tanh argument scale (softcap)
  void *ex = nullptr;
  int64_t ldx = 0;
  const float *xoff = nullptr;  // per-token base-2 offsets of the stored exponentials (tokens of this GEMM), or NULL
};

// The row-offset form's constants (base-2 units): the offset sits kExAbove above the label's logit, and a half tile's
// factor exp2(m_h - offset) is clamped at 2^kExClamp (past it the row is flagged and rescaled).
constexpr float kExAbove = 48.f;
constexpr float kExClamp = 64.f;

// The backward's per-row softmax state. Paired (OCTO_LSE_PAIR): lse[2 r] = m2, the row's base-2 maximum exactly as
// the statistics epilogue subtracts it (t = fma(x, c, -m2)), and lse[2 r + 1] = log2 of the shifted sum, so that
// p = exp2(fma(x, c, -m2) - l2S) repeats the forward's rounding: a plain fp32 lse of a row whose logits sit far from
// zero carries an absolute rounding error that scales every p of the row alike, and the row's dz then no longer sums
// to zero (at logits near -1,400 nats, 3% off in grad_h when the weights share a large component). Plain: m2 =
// lse[r] log2(e), l2S = 0.
__device__ __forceinline__ void row_state(const float *lse, int pair, int64_t r, float &m2, float &l2s) {
  if (pair) {
    m2 = lse[2 * r];
    l2s = lse[2 * r + 1];
  } else {
    m2 = lse[r] * OCTO_LOG2E;
    l2s = 0.f;
  }
}

// gemm_dz epilogue arguments (tokens are pass-local; compact row = row_off + token). The GEMM's first operand holds
// the vocabulary rows v0 .. v0 + its M (a chunk of W; v0 a multiple of 256); dz columns are chunk-local.
struct DzArgs {
  void *dzA;  // [tokens, ldA] chunk columns contiguous, staged MFMA type, or NULL
  int64_t ldA;
  void *dzB;  // [chunk columns, ldB] tokens contiguous, fp32 only, or NULL
  int64_t ldB;
  int64_t v0;
  const float *lse;
  const float *g;
  const int64_t *labels;
  const int64_t *label_idx;  // labels[label_idx[r]] when set
  int64_t row_off;
  int64_t V;
  const float *wscale;
  const float *hit;  // 16-bit dz: the pass's label entries, hit[token] (launch_hit), written over the dense values
  float c, pre, gmul;
  int lse_pair;      // lse holds (m2, l2S) per row (row_state)
};

// The label entry of each row's dz, g (1 - p_y) / T x post'(z_y) (x the fp8 row scale), from an fp32 target logit:
// hit[r - r0] for the compact rows r0 .. r0 + rows of a backward pass (0 past the count or for a label outside [0, V)).
struct HitArgs {
  const void *h;
  int64_t ldh;
  int h_dtype;
  const int64_t *idx;        // compact row -> hidden row, or NULL
  const void *w;
  int64_t ldw;
  int w_dtype;
  const float *wscale;
  const int64_t *labels;
  const int64_t *label_idx;  // labels[label_idx[r]] when set
  const float *lse, *g;
  const int32_t *count;
  int64_t r0, rows, n_max;
  int d, V;
  float c, pre, gmul;
  int use_tanh;
  float *hit;
  int lse_pair;  // lse holds (m2, l2S) per row (row_state)
};
int launch_hit(const HitArgs &a, hipStream_t st);

struct StoreArgs {
  void *C = nullptr;
  const float *addend = nullptr;  // optional fp32 term added before the store, [M, ld_add]
  int64_t ldc = 0;                // elements
  int64_t ld_add = 0;             // elements
  int dtype = OCTO_F32;
  int accumulate = 0;
  // A GEMM of one row pass of several (K = the pass's rows), with the row count on the device (pass_count != NULL):
  // a pass that starts at or past the count (pass_r0 > 0) stores nothing. With fp32 partials (part != NULL, laid out
  // as C with row stride ldc), the pass whose end reaches the count (count <= pass_end) stores the final C as above
  // (addend = the earlier passes' partials); an earlier pass stores its sum to part instead (= or += by
  // part_accumulate). No count: C as above, the host having chosen the destination.
  const int32_t *pass_count = nullptr;
  int64_t pass_r0 = 0, pass_end = 0;
  float *part = nullptr;
  int part_accumulate = 0;
  // part_blocked: the fp32 partials (part, and the addend of the pass that stores C) laid out tile by tile in the
  // 8-wave accumulator order, [tile mt * (ldc / 256) + nt][wave][i][j][v][lane], so that each 4-byte store or atomic
  // of a wave covers 256 contiguous bytes; needs ldc a multiple of 256 and M rounded up to 256 rows of room.
  int part_blocked = 0;
  // row_scale: C's row m takes row_scale[m] x acc (before any addend); the final store only (not the partials)
  const float *row_scale = nullptr;
};

int launch_gemm_stats(int dt, bool a_fp8, bool tanh, const Operand &A, const Operand &B, const GemmShape &s,
                      const StatsArgs &e, hipStream_t st);
int launch_gemm_dz(int dt, bool a_fp8, bool tanh, const Operand &A, const Operand &B, const GemmShape &s,
                   const DzArgs &e, hipStream_t st);
// kmajor: which operand, if any, is a plain K-major matrix (element (k, m) at base + k ld + 2 m; 16-bit types)
enum { KM_NONE = 0, KM_A = 1, KM_B = 2 };
int launch_gemm_store(int dt, const Operand &A, const Operand &B, const GemmShape &s, const StoreArgs &e,
                      hipStream_t st, int kmajor = KM_NONE);
// grad_h (Ah = dz K-contiguous, Bh = W K-major as stored when wh_kmajor, else W^T K-contiguous) and grad_W (Aw = dz
// K-major, Bw = h^T) of one row pass in one launch, each with its own shape and store (16-bit operands).
int launch_gemm_grads(int dt, const Operand &Ah, const Operand &Bh, const GemmShape &sh, const StoreArgs &eh,
                      bool wh_kmajor, const Operand &Aw, const Operand &Bw, const GemmShape &sw, const StoreArgs &ew,
                      hipStream_t st);

// ---- small kernels (head_aux.hip) ---------------------------------------------------------------
struct MergeArgs {
  const f32x4 *part;
  int64_t mtiles;
  const void *h;
  int64_t ldh;  // elements
  int h_dtype;
  const void *w;
  int64_t ldw;  // elements
  int w_dtype;
  const float *wscale;
  const int64_t *labels;
  const int64_t *idx;
  const int32_t *count;
  int64_t n_max;
  int d;
  int64_t V;
  int flags;
  float inv_T, pre, post;
  int use_tanh;
  float *logp, *ent, *lse, *out2;
  int lse_pair;  // lse gets (m2, l2S) per row (row_state) instead of the natural-log lse
  int64_t ld_out2;
  // GRPO weight of each compact row (g != NULL): per-token arrays indexed by the row's flat token
  const float *gprox, *gold, *gadv, *gmask;
  int64_t n_tokens;
  float eps_lo, eps_hi, reject_upper;
  const float *z;  // max(1, masked-token count), from launch_grpo_count
  float *g, *loss;
  // Rows row_off .. row_off + rows of the compact order (rows < 0: all n_max), part indexed from row_off. With hit
  // != NULL, hit[r - row_off] = the row's dz at its label per unit of g gmul, (1 - p_y) post'(z_y) x (fp8 row scale)
  // (launch_hit's formula without g gmul); 0 past the count or for a label outside [0, V). zero_g: g_zero[r] = 0 for
  // the launch's rows (rows whose g a later kernel accumulates).
  int64_t row_off = 0, rows = -1;
  float c = 0.f;
  float *hit = nullptr;
  int zero_g = 0;
  float *g_zero = nullptr;
  // tdot: the rows' raw target dot products h . W_y from launch_row_offsets (compact rows), used in place of the
  // merge's own (the same computation). exs (the row-offset exponentials, StatsArgs::xoff; needs hit): a row whose
  // maximum m2 lies at most kExClamp above its offset xoff[r] gets its label entry written into exs[r - row_off][y],
  // -hit exp2(m2 + l2S - xoff) (so that the row's dz scale times it is the label's dz), and xuse[r - row_off] =
  // xoff[r]; any other row (its offset too low, or -inf for a label outside [0, V)) is listed in flag_rows (local
  // rows, flag_cnt of them) with xuse = m2, for launch_ex_fix.
  const float *tdot = nullptr;
  void *exs = nullptr;
  int64_t ldx = 0;
  const float *xoff = nullptr;
  float *xuse = nullptr;
  int32_t *flag_cnt = nullptr;
  int32_t *flag_rows = nullptr;
};
int launch_merge(const MergeArgs &a, hipStream_t st);

// The fused step's per-row offsets, before its passes: for compact rows r < min(count, n_max), tdot[r] = the raw
// fp32 dot h_r . W_y (the merge's target-logit product) and xoff[r] = the label's base-2 logit as the statistics
// epilogue forms it (c x the transformed logit) + kExAbove, -inf for a label outside [0, V); flag_cnt[0 .. nflag) = 0.
struct RowOffArgs {
  const void *h;
  int64_t ldh;  // elements
  int h_dtype;
  const int64_t *idx;  // compact row -> hidden row, or NULL
  const void *w;
  int64_t ldw;  // elements
  int w_dtype;
  const float *wscale;
  const int64_t *labels;
  int label_via_idx;  // labels indexed by the hidden row (OCTO_ROWS_VIA_IDX)
  const int32_t *count;
  int64_t n_max;
  int d;
  int64_t V;
  float c, pre;
  int use_tanh;
  float *tdot, *xoff;
  int32_t *flag_cnt;
  int nflag;
};
int launch_row_offsets(const RowOffArgs &a, hipStream_t st);

// After a pass's merge (and its pair-row GRPO tail): the rows' dz scales s[i] = -g[r] gmul exp2(xuse[i] - m2 - l2S)
// for local rows i < rows with r = r0 + i below the count (0 otherwise), and the flagged rows' exponentials rescaled
// in place to their new offset xuse = m2: per half tile h, by exp2(m_h - m2 - min(m_h - xoff[r], kExClamp)), the
// label entry written as the merge writes it.
struct ExFixArgs {
  void *ex;  // [rows, ldx] bf16
  int64_t ldx, V_pad;
  const f32x4 *part;  // [rows, mtiles], local rows
  int64_t mtiles;
  const float *xoff;  // compact rows
  const float *xuse;  // local rows
  const float *lse;   // compact rows
  int lse_pair;
  const float *g;  // compact rows
  float gmul;
  const float *hit;  // local rows
  const int64_t *labels;
  const int64_t *label_idx;  // labels[label_idx[r]] when set
  const int32_t *count;
  const int32_t *flag_cnt, *flag_rows;
  int64_t r0, rows, n_max, V;
  float *scale;  // local rows
};
int launch_ex_fix(const ExFixArgs &a, hipStream_t st);

// dz of compact rows r0 .. r0 + rows (local row i = r - r0) from the exponentials a stats GEMM stored (StatsArgs::ex,
// f16), in place: dz[i][v] = -g[r] gmul exp2(m_h - m2 - l2S) ex[i][v] (x wscale[v] for fp8 weights, 0 past V) for
// v < V_pad, m_h the maximum of v's half tile in part[i][v / 256], then dz[i][y] = g[r] gmul hit[i] (the merge's
// label entry per unit of g gmul), in the MFMA type. Rows at or past the count are left as they are (the GEMMs that
// read dz stop at the count).
struct DzScaleArgs {
  void *dz;  // [rows, ld] 16-bit: f16 exponentials in, dz in dtype (bf16 / f16) out
  int64_t ld, V_pad;
  int dtype;
  const f32x4 *part;  // [rows, mtiles], local rows
  int64_t mtiles;
  const float *lse;  // (m2, l2S) pairs or lse, global rows
  int lse_pair;
  const float *g;  // global rows
  float gmul;
  const float *wscale;  // [V] fp8 row scales, or NULL
  const int64_t *labels;
  const int64_t *label_idx;  // labels[label_idx[r]] when set
  const float *hit;          // local rows
  const int32_t *count;
  int64_t r0, rows, n_max;
  int64_t V;
};
int launch_dz_scale(const DzScaleArgs &a, hipStream_t st);

// The GRPO tail of the fused step over prefix-tree pair rows: flat token t reads its pair row p = flat_pair[t]; for
// the pass's rows (r0 <= p < r0 + rows, below the row count) it takes the row's (logprob, entropy) from rowout (2
// floats per compact row) into out2[t] and, when mask[t] != 0, adds its GRPO weight to g[p] and its loss term to the
// loss (atomics: the last bits of both sums may vary). Tokens with no pair (p < 0 or past the count) get out2 = 0
// in the first pass and, when masked, their loss term at logprob 0 (as the objective over the expanded columns).
struct PairsGrpoArgs {
  const int64_t *flat_pair;
  int64_t n_flat;
  int64_t r0, rows, n_max;
  const int32_t *count;
  const float *rowout;
  const float *prox, *old, *adv, *mask;
  int64_t n_tokens;
  float eps_lo, eps_hi, reject_upper;
  const float *z;
  float *g, *loss, *out2;
  int64_t ld_out2;
  int first_pass;
};
int launch_pairs_grpo(const PairsGrpoArgs &a, hipStream_t st);
// dst row r (row_bytes, contiguous) = src row idx[r] (ld_src_bytes apart) for r < *count; 16-byte aligned rows
int launch_rows_gather(const void *src, int64_t ld_src_bytes, const int64_t *idx, const int32_t *count,
                       int64_t n_max, int64_t row_bytes, void *dst, hipStream_t st);
// z[0] = max(1, count of mask[t] != 0, t < n); *loss = 0 when loss != NULL. One workgroup.
int launch_grpo_count(const float *mask, int64_t n, float *z, float *loss, hipStream_t st);

// dst[r * d + c] = bf16(e4m3 w[r * ldw + c]) for r < V, c < d (exact).
int launch_widen_fp8(const void *w, int64_t ldw, int64_t V, int d, void *dst, hipStream_t st);
// dst[c * ld_dst + r] = src row map[r] (or r), element c, for r < rows_pad, c < cols; rows at or past the valid
// count (count - count_off, capped at rows) read 0; dst holds the staged MFMA type (bf16/f16/f32). row_scale (16-bit
// source and destination of one type only): row r is multiplied by row_scale[r] in fp32 and rounded once.
int launch_transpose(const void *src, int64_t ld_src, int src_dtype, const float *row_scale,
                     const int64_t *map, const int32_t *count, int64_t count_off, int64_t rows,
                     int64_t rows_pad, int64_t cols, void *dst, int64_t ld_dst, int dst_dtype, hipStream_t st);

}  // namespace octo
