// C-ABI entry points of the fused head (octo_head_fwd / octo_head_bwd), the workspace query and the
// status plumbing. Argument checks happen here, on the host, before anything is queued.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "gemm_nt.h"
#include "octo_internal.h"
#include "plan.h"

static thread_local char g_err[512] = "";

void octo_set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int octo_fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

using namespace octo;
using namespace octo_plan;
static_assert(TM == kTile && TN == kTile, "the planner's tile is the GEMM tile");
static_assert(sizeof(f32x4) == kStat4, "the planner's statistics partial");

namespace {

// ---- kernel timing hook (octo_timing_enable / octo_timing_read) ----------------------------------
// When enabled, each GEMM launch of octo_head_fwd / octo_head_bwd is bracketed by a pair of HIP events on
// its stream; octo_timing_read waits for the recorded pairs of one kernel name and sums their durations.
struct TimedPair {
  const char *name;
  hipEvent_t a, b;
};
std::mutex g_timing_mu;
bool g_timing = false;
std::vector<TimedPair> g_timed;

struct TimedLaunch {
  hipEvent_t a = nullptr, b = nullptr;
  const char *name;
  hipStream_t st;
  TimedLaunch(const char *n, hipStream_t s, bool allowed = true) : name(n), st(s) {
    if (!g_timing || !allowed) return;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess || hipEventRecord(a, st) != hipSuccess) {
      if (a) (void)hipEventDestroy(a);
      if (b) (void)hipEventDestroy(b);
      a = b = nullptr;
    }
  }
  void done() {
    if (!a) return;
    if (hipEventRecord(b, st) == hipSuccess) {
      std::lock_guard<std::mutex> lk(g_timing_mu);
      g_timed.push_back({name, a, b});
    } else {
      (void)hipEventDestroy(a);
      (void)hipEventDestroy(b);
    }
    a = b = nullptr;
  }
  ~TimedLaunch() { done(); }
};

#ifndef OCTO_GROUP_M
#define OCTO_GROUP_M 4
#endif
constexpr int kGroupM = OCTO_GROUP_M;  // M-tiles per L2 group of the tile order (gemm_nt.h tile_of)


struct Common {
  int hesz, wesz, dt;
  bool fp8;
  float c, pre, gmul;
  uint32_t h_extent;
  bool gather;  // idx over a hidden matrix of 2 GiB or more: the GEMMs read a contiguous copy of the rows
};

int check_common(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw, int w_dtype,
                 const float *w_scale, const int64_t *labels, const int64_t *idx, int64_t n_max, int d, int V,
                 int flags, float inv_T, float pre, float post, int use_tanh, Common &cm) {
  OCTO_CHECK_ARG(n_max >= 0 && d > 0 && V > 0, "head: bad sizes n_max=%lld d=%d V=%d", (long long)n_max, d, V);
  OCTO_CHECK_ARG(h && w && labels, "head: null h, w or labels");
  const bool fp8 = w_dtype == OCTO_FP8E4M3;
  if (fp8) {
    if (h_dtype != OCTO_BF16) return octo_fail(OCTO_EUNSUPPORTED, "head: fp8 weights need bf16 hidden rows");
    OCTO_CHECK_ARG(w_scale != nullptr, "head: fp8 weights need per-row scales");
  } else {
    if (!(h_dtype == OCTO_BF16 || h_dtype == OCTO_F16 || h_dtype == OCTO_F32))
      return octo_fail(OCTO_EUNSUPPORTED, "head: hidden dtype %d", h_dtype);
    if (w_dtype != h_dtype)
      return octo_fail(OCTO_EUNSUPPORTED, "head: weight dtype %d differs from hidden dtype %d", w_dtype, h_dtype);
  }
  cm.hesz = elem_bytes(h_dtype);
  cm.wesz = elem_bytes(w_dtype);
  cm.dt = staged_dtype(w_dtype);
  cm.fp8 = fp8;
  const int kq = (h_dtype == OCTO_F32) ? 4 : (fp8 ? 16 : 8);
  OCTO_CHECK_ARG(d % kq == 0, "head: d=%d must be a multiple of %d", d, kq);
  OCTO_CHECK_ARG(ldh >= d && ldw >= d, "head: row strides below d");
  OCTO_CHECK_ARG((ldh * cm.hesz) % 16 == 0 && ((uintptr_t)h) % 16 == 0, "head: hidden rows must be 16-byte aligned");
  OCTO_CHECK_ARG((ldw * cm.wesz) % 16 == 0 && ((uintptr_t)w) % 16 == 0,
                 "head: weight rows must be 16-byte aligned");
  OCTO_CHECK_ARG(!fp8 || ((uintptr_t)w_scale) % 16 == 0, "head: w_scale must be 16-byte aligned");
  OCTO_CHECK_ARG(256 * ldh * cm.hesz < (int64_t)0x7fffffff && 256 * ldw * cm.wesz < (int64_t)0x7fffffff,
                 "head: row stride too large");
  if (idx) {
    OCTO_CHECK_ARG(h_rows > 0, "head: h_rows must be positive with idx");
    const int64_t ext = h_rows * ldh * cm.hesz;
    cm.gather = ext >= (int64_t)0x7fffffff;  // past the 32-bit offsets of a mapped GEMM operand
    cm.h_extent = cm.gather ? 0 : (uint32_t)ext;
  } else {
    OCTO_CHECK_ARG(h_rows >= n_max, "head: h_rows %lld < n_max %lld", (long long)h_rows, (long long)n_max);
    cm.h_extent = 0;
    cm.gather = false;
    OCTO_CHECK_ARG(!(flags & (OCTO_ROWS_VIA_IDX | OCTO_OUT_SCATTER)), "head: idx-based flags without idx");
  }
  OCTO_CHECK_ARG(inv_T > 0.f, "head: temperature must be positive");
  if (use_tanh) {
    OCTO_CHECK_ARG(post > 0.f && pre != 0.f, "head: softcap needs post > 0 and pre != 0");
    cm.c = post * inv_T * OCTO_LOG2E;
  } else {
    OCTO_CHECK_ARG(pre * post > 0.f, "head: logit scale must be positive");
    cm.c = pre * post * inv_T * OCTO_LOG2E;
  }
  cm.pre = pre;
  cm.gmul = inv_T * pre * post;
  return OCTO_OK;
}

Operand weight_operand(const void *w, int64_t ldw, const Common &cm, int V) {
  Operand A;
  A.base = (const char *)w;
  A.ld = ldw * cm.wesz;
  A.map = nullptr;
  A.rows = V;
  A.count = nullptr;
  A.count_off = 0;
  A.extent = 0;
  return A;
}

// The GEMMs' weight operand for the vocabulary rows [v0, v0 + vc): W as stored, or for fp8 weights those rows widened
// to bf16 into `wide` (queued on st).
Operand gemm_weight(const void *w, int64_t ldw, const Common &cm, int64_t v0, int64_t vc, int d, void *wide,
                    hipStream_t st, int &rc) {
  rc = OCTO_OK;
  if (!cm.fp8) return weight_operand((const char *)w + v0 * ldw * cm.wesz, ldw, cm, (int)vc);
  rc = launch_widen_fp8((const uint8_t *)w + v0 * ldw, ldw, vc, d, wide, st);
  Operand A = weight_operand(wide, d, cm, (int)vc);
  A.ld = (int64_t)d * 2;
  return A;
}

// Hidden rows [r0, r0 + rows) of the compact order.
// Hidden rows [r0, r0 + rows) of the compact order: through idx, or (gathered != NULL) from the contiguous copy
// [n_max, d] of them that launch_rows_gather wrote.
Operand hidden_operand(const void *h, int64_t ldh, const int64_t *idx, const int32_t *count, int64_t r0,
                       int64_t rows, const Common &cm, const void *gathered = nullptr, int d = 0) {
  Operand B;
  B.ld = ldh * cm.hesz;
  if (gathered) {
    B.ld = (int64_t)d * cm.hesz;
    B.base = (const char *)gathered + r0 * B.ld;
    B.map = nullptr;
    B.extent = 0;
  } else if (idx) {
    B.base = (const char *)h;
    B.map = idx + r0;
    B.extent = cm.h_extent;
  } else {
    B.base = (const char *)h + r0 * B.ld;
    B.map = nullptr;
    B.extent = 0;
  }
  B.rows = rows;
  B.count = count;
  B.count_off = r0;
  return B;
}

Operand plain_operand(const void *base, int64_t ld_bytes, int64_t rows, const int32_t *count, int64_t count_off) {
  Operand X;
  X.base = (const char *)base;
  X.ld = ld_bytes;
  X.map = nullptr;
  X.rows = rows;
  X.count = count;
  X.count_off = count_off;
  X.extent = 0;
  return X;
}

GemmShape shape(int64_t M, int64_t N, int64_t K, int group_m, int count_on, const int32_t *count, int64_t count_off) {
  GemmShape s;
  s.M = M;
  s.N = N;
  s.K = K;
  s.mtiles = (int)cdiv(M, TM);
  s.ntiles = (int)cdiv(N, TN);
  s.group_m = group_m;
  s.count_on = count_on;
  s.count = count;
  s.count_off = count_off;
  return s;
}

// grad_W[v0 .. v0 + vc) of row pass p (rows r0 .. r0 + rows, K = rows) from the pass's dz A3 and h^T B3: stored in
// gw_dtype when the pass is the only one or the last (adding the fp32 partials of the earlier passes when gacc_on),
// else as fp32 partials (gacc_on) or added to the output. With a device row count the count decides which pass is
// the last (passes at or past it store nothing). gacc and gw point at row v0.
StoreArgs grad_w_store(int d, int64_t r0, int64_t rows, int64_t p, int64_t passes, bool gacc_on, float *gacc, void *gw,
                       int gw_dtype, int flags, const int32_t *count, bool blocked = false) {
  const bool last_pass = p + 1 == passes;
  StoreArgs o;
  const bool acc_out = flags & OCTO_GRADW_ACCUMULATE;
  if (gacc_on && !last_pass && !count) {  // fp32 partial sums of the passes so far
    o.C = gacc;
    o.addend = nullptr;
    o.dtype = OCTO_F32;
    o.accumulate = p > 0 ? 1 : 0;
  } else {
    o.C = gw;
    o.addend = (gacc_on && p > 0) ? gacc : nullptr;
    o.dtype = gw_dtype;
    o.accumulate = (acc_out || (!gacc_on && p > 0)) ? 1 : 0;
  }
  if (count && p > 0) {  // passes at or past the device row count store nothing
    o.pass_count = count;
    o.pass_r0 = r0;
    o.pass_end = r0 + rows;
  }
  if (count && gacc_on && !last_pass) {
    // the device count decides: the pass that reaches it stores grad_W (adding the earlier passes' partials), an
    // earlier one stores its fp32 partials
    o.pass_count = count;
    o.pass_r0 = r0;
    o.pass_end = r0 + rows;
    o.part = gacc;
    o.part_accumulate = p > 0 ? 1 : 0;
  }
  // with a device count every pass reaches the partials through part / addend, so their layout may be blocked
  o.part_blocked = (blocked && count && gacc_on && d % TN == 0) ? 1 : 0;
  o.ldc = d;
  o.ld_add = d;
  return o;
}
int grad_w_pass(int dt, const Operand &A3, int kmajor, const Operand &B3, int64_t vc, int d, int64_t r0, int64_t rows,
                int64_t p, int64_t passes, bool gacc_on, float *gacc, void *gw, int gw_dtype, int flags,
                const int32_t *count, hipStream_t st, bool blocked = false) {
  const StoreArgs o = grad_w_store(d, r0, rows, p, passes, gacc_on, gacc, gw, gw_dtype, flags, count, blocked);
  TimedLaunch t("gemm_store_grad_w", st);
  return launch_gemm_store(dt, A3, B3, shape(vc, d, rows, kGroupM, 3, count, r0), o, st, kmajor);
}

// The merge's arguments for every row of the call (row_off 0, all n_max rows) with the GRPO tail gt, if any.
MergeArgs merge_args(const f32x4 *part, int64_t mtiles, const void *h, int64_t ldh, int h_dtype, const void *w,
                     int64_t ldw, int w_dtype, const float *w_scale, const int64_t *labels, const int64_t *idx,
                     const int32_t *count, int64_t n_max, int d, int V, int flags, float inv_T, float pre, float post,
                     int use_tanh, float *logp, float *ent, float *lse, float *out2, int64_t ld_out2,
                     const octo_grpo_tail *gt, const float *z) {
  MergeArgs m;
  m.part = part;
  m.mtiles = mtiles;
  m.h = h;
  m.ldh = ldh;
  m.h_dtype = h_dtype;
  m.w = w;
  m.ldw = ldw;
  m.w_dtype = w_dtype;
  m.wscale = w_scale;
  m.labels = labels;
  m.idx = idx;
  m.count = count;
  m.n_max = n_max;
  m.d = d;
  m.V = V;
  m.flags = flags;
  m.inv_T = inv_T;
  m.pre = pre;
  m.post = post;
  m.use_tanh = use_tanh;
  m.logp = logp;
  m.ent = ent;
  m.lse = lse;
  m.lse_pair = (flags & OCTO_LSE_PAIR) != 0;
  m.out2 = out2;
  m.ld_out2 = ld_out2;
  m.gprox = gt ? gt->prox : nullptr;
  m.gold = gt ? gt->old : nullptr;
  m.gadv = gt ? gt->adv : nullptr;
  m.gmask = gt ? gt->mask : nullptr;
  m.n_tokens = gt ? gt->n_tokens : 0;
  m.eps_lo = gt ? gt->eps_lo : 0.f;
  m.eps_hi = gt ? gt->eps_hi : 0.f;
  m.reject_upper = gt ? gt->reject_upper : 0.f;
  m.z = z;
  m.g = gt ? gt->g : nullptr;
  m.loss = gt ? gt->loss : nullptr;
  return m;
}

int head_fwd(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw, int w_dtype,
             const float *w_scale, const int64_t *labels, const int64_t *idx, const int32_t *count, int64_t n_max,
             int d, int V, int flags, float inv_T, float pre, float post, int use_tanh, float *logp, float *ent,
             float *lse, float *out2, int64_t ld_out2, const octo_grpo_tail *gt, void *ws, size_t ws_bytes,
             void *stream, bool timed = true) {
  Common cm;
  int rc = check_common(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, n_max, d, V, flags, inv_T,
                        pre, post, use_tanh, cm);
  if (rc) return rc;
  OCTO_CHECK_ARG(!out2 || ld_out2 >= 2, "head_fwd: ld_out2 < 2");
  if (gt) {
    OCTO_CHECK_ARG(gt->n_tokens >= 0, "head_fwd_grpo: n_tokens < 0");
    OCTO_CHECK_ARG(gt->g && gt->adv && gt->mask, "head_fwd_grpo: null g, adv or mask");
  }
  if (n_max == 0) return OCTO_OK;
  const FwdLayout L = fwd_layout(n_max, d, V, w_dtype, cm.gather);
  if (!ws || ws_bytes < L.total)
    return octo_fail(OCTO_EWORKSPACE, "head_fwd: workspace %zu < %zu bytes%s", ws_bytes, L.total,
                     cm.gather ? " (hidden of 2 GiB or more through idx: query with OCTO_WS_GATHER)" : "");
  hipStream_t st = (hipStream_t)stream;
  float *z = (float *)((char *)ws + L.z);
  if (gt) {  // Z (and the loss zeroed) ahead of the merge
    rc = launch_grpo_count(gt->mask, gt->n_tokens, z, gt->loss, st);
    if (rc) return rc;
  }

  void *gathered = cm.gather ? (char *)ws + L.rows : nullptr;
  if (gathered) {
    rc = launch_rows_gather(h, ldh * cm.hesz, idx, count, n_max, (int64_t)d * cm.hesz, gathered, st);
    if (rc) return rc;
  }
  const Operand B = hidden_operand(h, ldh, idx, count, 0, n_max, cm, gathered, d);
  StatsArgs e;
  e.part = (f32x4 *)((char *)ws + L.part);
  e.mtiles = L.mtiles;
  e.V = V;
  e.wscale = w_scale;
  e.c = cm.c;
  e.pre = cm.pre;
  for (int64_t c = 0; c < L.chunks; ++c) {  // one chunk covering V, except for fp8 weights (widened chunk by chunk)
    e.v0 = c * L.Vc;
    const int64_t vc = (V - e.v0) < L.Vc ? (V - e.v0) : L.Vc;
    const Operand A = gemm_weight(w, ldw, cm, e.v0, vc, d, (char *)ws + L.wide, st, rc);
    if (rc) return rc;
    const GemmShape s = shape(vc, n_max, d, kGroupM, 2, count, 0);
    {
      TimedLaunch t("gemm_stats", st, timed);
      rc = launch_gemm_stats(cm.dt, cm.fp8, use_tanh != 0, A, B, s, e, st);
    }
    if (rc) return rc;
  }

  const MergeArgs m = merge_args(e.part, L.mtiles, h, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count,
                                 n_max, d, V, flags, inv_T, pre, post, use_tanh, logp, ent, lse, out2, ld_out2, gt, z);
  return launch_merge(m, st);
}


// ---- the fused GRPO step (octo_head_step_grpo) ---------------------------------------------------------
// Forward, GRPO weight and backward of the compact rows in one call, pass by pass (StepLayout). The logits are
// computed once per pass: the forward GEMM leaves each element's exponential (from the same exp2 its statistics sum)
// in the staging area; the merge gives the rows' outputs, row state, g and label entry; bf16: launch_ex_fix sets each
// row's dz scale (and rescales the rows flagged by the merge), which grad_h's store and the scaled h^T of grad_W
// apply; f16: launch_dz_scale scales the exponentials into dz. grad_h = dz . W, grad_W = dz^T . h follow as in the
// backward. fp32 operands run head_fwd, then octo_head_bwd.
// Prefix-tree pair rows (octo_head_step_grpo_pairs): the compact rows are the tree's (position, label) pairs, the
// GRPO tail's arrays are per flat token, and flat token t reads pair row flat_pair[t]; its columns go to out_flat.
struct StepPairs {
  const int64_t *flat_pair;
  int64_t n_flat;
  float *out_flat;
  int64_t ld_out;
};

int head_step(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw, int w_dtype,
              const float *w_scale, const int64_t *labels, const int64_t *idx, const int32_t *count, int64_t n_max,
              int d, int V, int flags, float inv_T, float pre, float post, int use_tanh, float *logp, float *ent,
              float *lse, float *out2, int64_t ld_out2, const octo_grpo_tail *gt, void *grad_h, int64_t ld_gh,
              int gh_dtype, void *grad_w, int gw_dtype, void *ws, size_t ws_bytes, void *stream,
              const StepPairs *pm = nullptr) {
  Common cm;
  int rc = check_common(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, n_max, d, V, flags, inv_T,
                        pre, post, use_tanh, cm);
  if (rc) return rc;
  OCTO_CHECK_ARG(gt != nullptr, "head_step_grpo: null grpo");
  OCTO_CHECK_ARG(gt->n_tokens >= 0, "head_step_grpo: n_tokens < 0");
  OCTO_CHECK_ARG(gt->g && gt->adv && gt->mask, "head_step_grpo: null g, adv or mask");
  OCTO_CHECK_ARG(lse != nullptr, "head_step_grpo: null lse");
  OCTO_CHECK_ARG(!out2 || ld_out2 >= 2, "head_step_grpo: ld_out2 < 2");
  if (grad_h) {
    OCTO_CHECK_ARG(gh_dtype == OCTO_BF16 || gh_dtype == OCTO_F16 || gh_dtype == OCTO_F32, "head_step_grpo: grad_h dtype");
    OCTO_CHECK_ARG(ld_gh >= d, "head_step_grpo: ld_gh < d");
  }
  if (grad_w) {
    if (cm.fp8) return octo_fail(OCTO_EUNSUPPORTED, "head_step_grpo: grad_w of fp8 weights");
    OCTO_CHECK_ARG(gw_dtype == OCTO_BF16 || gw_dtype == OCTO_F16 || gw_dtype == OCTO_F32, "head_step_grpo: grad_w dtype");
  }
  const bool need_gh = grad_h != nullptr, need_gw = grad_w != nullptr;
  if (pm) {
    OCTO_CHECK_ARG(!(flags & (OCTO_ROWS_VIA_IDX | OCTO_OUT_SCATTER)), "head_step_grpo_pairs: labels are per pair row");
    OCTO_CHECK_ARG(pm->n_flat >= 0 && (pm->n_flat == 0 || (pm->flat_pair && pm->out_flat)) && pm->ld_out >= 2,
                   "head_step_grpo_pairs: flat_pair, out_flat or ld_out");
    if (cm.dt == OCTO_F32) return octo_fail(OCTO_EUNSUPPORTED, "head_step_grpo_pairs: fp32 operands");
  }
  if (n_max == 0 && !pm) return OCTO_OK;
  if (!need_gh && !need_gw && !pm)  // no gradient asked for: the forward with its GRPO tail (its own workspace size)
    return head_fwd(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags, inv_T,
                    pre, post, use_tanh, logp, ent, lse, out2, ld_out2, gt, ws, ws_bytes, stream);
  if (cm.dt == OCTO_F32) {  // fp32: the forward, then the backward
    if (!ws || ws_bytes < step_fallback_bytes(n_max, d, V, w_dtype, need_gw, cm.gather))
      return octo_fail(OCTO_EWORKSPACE, "head_step_grpo: workspace %zu < %zu bytes", ws ? ws_bytes : (size_t)0,
                       step_fallback_bytes(n_max, d, V, w_dtype, need_gw, cm.gather));
    rc = head_fwd(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags, inv_T,
                  pre, post, use_tanh, logp, ent, lse, out2, ld_out2, gt, ws, ws_bytes, stream);
    if (rc || (!need_gh && !need_gw)) return rc;
    return octo_head_bwd(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags,
                         inv_T, pre, post, use_tanh, lse, gt->g, grad_h, ld_gh, gh_dtype, grad_w, gw_dtype, ws,
                         ws_bytes, stream);
  }
  StepLayout L;
  if (!ws || !step_plan_for(n_max, d, V, w_dtype, need_gh, need_gw, cm.gather, ws_bytes, L)) {
    StepLayout Lmin;
    size_t least = 0;
    for (int q = kBudgetQMin; q <= kBudgetQMax && !least; ++q)
      if (step_plan(n_max, d, V, w_dtype, need_gh, need_gw, cm.gather, staging_candidate(q), Lmin, false))
        least = Lmin.total;
    return octo_fail(OCTO_EWORKSPACE, "head_step_grpo: workspace %zu bytes, below the smallest plan's %zu%s",
                     ws ? ws_bytes : (size_t)0, least,
                     cm.gather ? " (hidden of 2 GiB or more through idx: query with OCTO_WS_GATHER)" : "");
  }
  hipStream_t st = (hipStream_t)stream;
  char *wsb = (char *)ws;
  f32x4 *part = (f32x4 *)(wsb + L.part);
  float *z = (float *)(wsb + L.z), *hit = (float *)(wsb + L.hit), *gacc = (float *)(wsb + L.gacc);
  void *ht = wsb + L.ht, *dz = wsb + L.dz, *wt = wsb + L.wt;
  const int esz = L.esz;

  rc = launch_grpo_count(gt->mask, gt->n_tokens, z, gt->loss, st);  // Z, and the loss zeroed
  if (rc) return rc;
  const bool grads = need_gh || need_gw;
  float *rowout = (float *)(wsb + L.rowout);
  if (pm && L.passes == 0) {  // no pair row: every flat token's columns are 0
    PairsGrpoArgs pa{};
    pa.flat_pair = pm->flat_pair;
    pa.n_flat = pm->n_flat;
    pa.count = count;
    pa.rowout = rowout;
    pa.prox = gt->prox;
    pa.old = gt->old;
    pa.adv = gt->adv;
    pa.mask = gt->mask;
    pa.n_tokens = gt->n_tokens;
    pa.z = z;
    pa.g = gt->g;
    pa.out2 = pm->out_flat;
    pa.ld_out2 = pm->ld_out;
    pa.first_pass = 1;
    return launch_pairs_grpo(pa, st);
  }
  void *gathered = cm.gather ? wsb + L.rows : nullptr;
  if (gathered) {
    rc = launch_rows_gather(h, ldh * cm.hesz, idx, count, n_max, (int64_t)d * cm.hesz, gathered, st);
    if (rc) return rc;
  }
  // the GEMMs' weight operand: W as stored, or fp8 weights widened to bf16 once for every pass
  Operand Aw = weight_operand(w, ldw, cm, V);
  if (L.wide_on) {
    rc = launch_widen_fp8(w, ldw, V, d, wsb + L.wide, st);
    if (rc) return rc;
    Aw = weight_operand(wsb + L.wide, d, cm, V);
    Aw.ld = (int64_t)d * 2;
  }
  if (L.wt_on) {  // W^T [d, V_pad] in the staged type, zero past V
    rc = launch_transpose(Aw.base, Aw.ld / esz, cm.dt, nullptr, nullptr, nullptr, 0, V, L.V_pad, d, wt, L.V_pad,
                          cm.dt, st);
    if (rc) return rc;
  }
  // bf16 operands: the exponentials are stored relative to per-row offsets (StatsArgs::xoff), so dz is one scale per
  // row times the stored value: grad_h takes the scale in its store, grad_W through the scaled h^T, and no pass of its
  // own turns the exponentials into dz. f16 (5 exponent bits) keeps the half-tile form and launch_dz_scale.
  const bool rowoff = grads && cm.dt == OCTO_BF16 && cm.c > 0.f;
  float *xoff = (float *)(wsb + L.xoff), *tdot = (float *)(wsb + L.tdot);
  float *xuse = (float *)(wsb + L.xuse), *rscale = (float *)(wsb + L.scale);
  int32_t *flag_cnt = (int32_t *)(wsb + L.flags), *flag_rows = flag_cnt + L.passes;
  if (rowoff) {
    RowOffArgs ro{};
    ro.h = h;
    ro.ldh = ldh;
    ro.h_dtype = h_dtype;
    ro.idx = idx;
    ro.w = w;
    ro.ldw = ldw;
    ro.w_dtype = w_dtype;
    ro.wscale = w_scale;
    ro.labels = labels;
    ro.label_via_idx = (flags & OCTO_ROWS_VIA_IDX) != 0;
    ro.count = count;
    ro.n_max = n_max;
    ro.d = d;
    ro.V = V;
    ro.c = cm.c;
    ro.pre = cm.pre;
    ro.use_tanh = use_tanh;
    ro.tdot = tdot;
    ro.xoff = xoff;
    ro.flag_cnt = flag_cnt;
    ro.nflag = (int)L.passes;
    rc = launch_row_offsets(ro, st);
    if (rc) return rc;
  }

  for (int64_t p = 0; p < L.passes; ++p) {
    const int64_t r0 = p * L.P;
    const int64_t rows = (n_max - r0) < L.P ? (n_max - r0) : L.P;
    const Operand Bh = hidden_operand(h, ldh, idx, count, r0, rows, cm, gathered, d);

    // logits once: statistics per (row, vocabulary tile) and each element's exponential
    StatsArgs e;
    e.part = part;
    e.mtiles = L.mtiles;
    e.v0 = 0;
    e.V = V;
    e.wscale = w_scale;
    e.c = cm.c;
    e.pre = cm.pre;
    e.ex = grads ? dz : nullptr;
    e.ldx = L.V_pad;
    e.xoff = rowoff ? xoff + r0 : nullptr;
    {
      TimedLaunch t("gemm_stats", st);
      rc = launch_gemm_stats(cm.dt, cm.fp8, use_tanh != 0, Aw, Bh, shape(V, rows, d, kGroupM, 2, count, r0), e, st);
    }
    if (rc) return rc;

    // the pass's outputs, row state, GRPO weight g (the loss summed) and dz at each label per unit of g; pair rows:
    // the rows' columns to rowout, then each flat token's columns and GRPO weight, summed into its pair's g
    MergeArgs m = pm ? merge_args(part, L.mtiles, h, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count,
                                  n_max, d, V, flags, inv_T, pre, post, use_tanh, logp, ent, lse, rowout, 2, nullptr,
                                  z)
                     : merge_args(part, L.mtiles, h, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count,
                                  n_max, d, V, flags, inv_T, pre, post, use_tanh, logp, ent, lse, out2, ld_out2, gt, z);
    m.row_off = r0;
    m.rows = rows;
    m.c = cm.c;
    m.hit = hit;
    if (rowoff) {
      m.tdot = tdot;
      m.exs = dz;
      m.ldx = L.V_pad;
      m.xoff = xoff;
      m.xuse = xuse;
      m.flag_cnt = flag_cnt + p;
      m.flag_rows = flag_rows;
    }
    if (pm) {
      m.zero_g = 1;
      m.g_zero = gt->g;
    }
    rc = launch_merge(m, st);
    if (rc) return rc;
    if (pm) {
      PairsGrpoArgs pa{};
      pa.flat_pair = pm->flat_pair;
      pa.n_flat = pm->n_flat;
      pa.r0 = r0;
      pa.rows = rows;
      pa.n_max = n_max;
      pa.count = count;
      pa.rowout = rowout;
      pa.prox = gt->prox;
      pa.old = gt->old;
      pa.adv = gt->adv;
      pa.mask = gt->mask;
      pa.n_tokens = gt->n_tokens;
      pa.eps_lo = gt->eps_lo;
      pa.eps_hi = gt->eps_hi;
      pa.reject_upper = gt->reject_upper;
      pa.z = z;
      pa.g = gt->g;
      pa.loss = gt->loss;
      pa.out2 = pm->out_flat;
      pa.ld_out2 = pm->ld_out;
      pa.first_pass = p == 0;
      rc = launch_pairs_grpo(pa, st);
      if (rc) return rc;
    }
    if (!grads) continue;

    if (rowoff) {  // the rows' dz scales, and any flagged row's exponentials rescaled
      ExFixArgs fx{};
      fx.ex = dz;
      fx.ldx = L.V_pad;
      fx.V_pad = L.V_pad;
      fx.part = part;
      fx.mtiles = L.mtiles;
      fx.xoff = xoff;
      fx.xuse = xuse;
      fx.lse = lse;
      fx.lse_pair = (flags & OCTO_LSE_PAIR) != 0;
      fx.g = gt->g;
      fx.gmul = cm.gmul;
      fx.hit = hit;
      fx.labels = labels;
      fx.label_idx = (flags & OCTO_ROWS_VIA_IDX) ? idx : nullptr;
      fx.count = count;
      fx.flag_cnt = flag_cnt + p;
      fx.flag_rows = flag_rows;
      fx.r0 = r0;
      fx.rows = rows;
      fx.n_max = n_max;
      fx.V = V;
      fx.scale = rscale;
      {
        TimedLaunch t("ex_fix", st);
        rc = launch_ex_fix(fx, st);
      }
      if (rc) return rc;
    } else {
      DzScaleArgs sa;
      sa.dz = dz;
      sa.ld = L.V_pad;
      sa.V_pad = L.V_pad;
      sa.dtype = cm.dt;
      sa.part = part;
      sa.mtiles = L.mtiles;
      sa.lse = lse;
      sa.lse_pair = (flags & OCTO_LSE_PAIR) != 0;
      sa.g = gt->g;
      sa.gmul = cm.gmul;
      sa.wscale = cm.fp8 ? w_scale : nullptr;
      sa.labels = labels;
      sa.label_idx = (flags & OCTO_ROWS_VIA_IDX) ? idx : nullptr;
      sa.hit = hit;
      sa.count = count;
      sa.r0 = r0;
      sa.rows = rows;
      sa.n_max = n_max;
      sa.V = V;
      {
        TimedLaunch t("dz_scale", st);
        rc = launch_dz_scale(sa, st);
      }
      if (rc) return rc;
    }

    // grad_h[rows] = dz . W   (K = V, or V_pad through the staged W^T)
    const Operand A2 = plain_operand(dz, L.V_pad * esz, rows, count, r0);
    const Operand B2 = L.wt_on ? plain_operand(wt, L.V_pad * esz, d, nullptr, 0) : plain_operand(Aw.base, Aw.ld, d, nullptr, 0);
    const GemmShape s2 = shape(rows, d, L.wt_on ? L.V_pad : V, kGroupM, 1, count, r0);
    StoreArgs o2;
    o2.C = (char *)grad_h + r0 * ld_gh * elem_bytes(gh_dtype);
    o2.ldc = ld_gh;
    o2.dtype = gh_dtype;
    o2.row_scale = rowoff ? rscale : nullptr;
    // grad_W (+)= dz^T . h   (K = this pass's rows)
    const Operand A3 = plain_operand(dz, L.V_pad * esz, L.P, nullptr, 0);
    const Operand B3 = plain_operand(ht, L.P * esz, d, nullptr, 0);
    if (need_gw) {  // h^T [d, P] of the pass's rows, zero past the count
      const int64_t rows_pad = round_up(rows, TN);
      rc = launch_transpose(idx ? h : (const char *)h + r0 * ldh * cm.hesz, ldh, h_dtype, rowoff ? rscale : nullptr,
                            idx ? idx + r0 : nullptr, count, r0, rows, rows_pad, d, ht, L.P, cm.dt, st);
      if (rc) return rc;
    }
    if (need_gh && need_gw) {  // both in one launch
      const StoreArgs o3 = grad_w_store(d, r0, rows, p, L.passes, L.gacc_on, gacc, grad_w, gw_dtype, flags, count,
                                        true);
      TimedLaunch t("gemm_grads", st);
      rc = launch_gemm_grads(cm.dt, A2, B2, s2, o2, !L.wt_on, A3, B3, shape(V, d, rows, kGroupM, 3, count, r0), o3,
                             st);
    } else if (need_gh) {
      TimedLaunch t("gemm_store_grad_h", st);
      rc = launch_gemm_store(cm.dt, A2, B2, s2, o2, st, L.wt_on ? KM_NONE : KM_B);
    } else if (need_gw) {
      rc = grad_w_pass(cm.dt, A3, KM_A, B3, V, d, r0, rows, p, L.passes, L.gacc_on, gacc, grad_w, gw_dtype, flags,
                       count, st, true);
    }
    if (rc) return rc;
  }
  return OCTO_OK;
}

// ---- the allocation-free forward (octo_head_fwd_noalloc) ----------------------------------------
// Its workspace is this file-scope device array: one copy on each GPU the library runs on, held until the process
// ends. In host code the array's name stands for a host-side shadow, not a device address, so it is never passed to
// a kernel: each device's address comes from hipGetSymbolAddress, taken once per device with that device current,
// and kept in g_scratch_ptr.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __attribute__((aligned(256))) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on the device that runs `stream` (the current device for the null stream).
int scratch_on(hipStream_t stream, void **ptr) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return octo_fail(OCTO_EHIP, "head_fwd_noalloc: stream device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return octo_fail(OCTO_EUNSUPPORTED, "head_fwd_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void *p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = (cur >= 0 && cur != dev) ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || p == nullptr)
      return octo_fail(OCTO_EHIP, "head_fwd_noalloc: scratch address on device %d: %s", dev,
                       e != hipSuccess ? hipGetErrorString(e) : "null");
    if (back != hipSuccess)
      return octo_fail(OCTO_EHIP, "head_fwd_noalloc: restoring device %d: %s", cur, hipGetErrorString(back));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return OCTO_OK;
}

}  // namespace

extern "C" {

int octo_head_fwd_noalloc(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw,
                          int w_dtype, const float *w_scale, const int64_t *labels, const int64_t *idx,
                          const int32_t *count, int64_t n_max, int d, int V, int flags, float inv_T, float pre,
                          float post, int use_tanh, float *logp, float *ent, float *lse, float *out2,
                          int64_t ld_out2, void *stream) {
  Common cm;
  int rc = check_common(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, n_max, d, V, flags, inv_T,
                        pre, post, use_tanh, cm);
  if (rc) return rc;
  const size_t need = fwd_layout(n_max, d, V, w_dtype, cm.gather).total;
  if (need > kScratchBytes)
    return octo_fail(OCTO_EINVAL, "head_fwd_noalloc: n_max=%lld d=%d V=%d needs %zu bytes of scratch, above its %zu",
                     (long long)n_max, d, V, need, kScratchBytes);
  if (n_max == 0) return OCTO_OK;
  void *ptr = nullptr;
  rc = scratch_on((hipStream_t)stream, &ptr);
  if (rc) return rc;
  return head_fwd(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags, inv_T,
                  pre, post, use_tanh, logp, ent, lse, out2, ld_out2, nullptr, ptr, kScratchBytes, stream,
                  /*timed=*/false);
}

const char *octo_version(void) { return "octo_head 0.1 (gfx950)"; }
const char *octo_last_error(void) { return g_err; }

int octo_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (auto &t : g_timed) {
    (void)hipEventDestroy(t.a);
    (void)hipEventDestroy(t.b);
  }
  g_timed.clear();
  g_timing = on != 0;
  return OCTO_OK;
}

int octo_timing_read(const char *kernel, int *launches, double *total_ms) {
  OCTO_CHECK_ARG(kernel && launches && total_ms, "timing_read: null argument");
  std::lock_guard<std::mutex> lk(g_timing_mu);
  int n = 0;
  double ms = 0.0;
  for (auto &t : g_timed) {
    if (strcmp(t.name, kernel) != 0) continue;
    float x = 0.f;
    hipError_t e = hipEventSynchronize(t.b);
    if (e == hipSuccess) e = hipEventElapsedTime(&x, t.a, t.b);
    if (e != hipSuccess) return octo_fail(OCTO_EHIP, "timing_read: %s", hipGetErrorString(e));
    ++n;
    ms += x;
  }
  *launches = n;
  *total_ms = ms;
  return OCTO_OK;
}

int octo_head_workspace_bytes(int64_t n_max, int d, int V, int w_dtype, int flags, size_t *bytes) {
  OCTO_CHECK_ARG(bytes != nullptr, "workspace_bytes: null pointer");
  OCTO_CHECK_ARG(n_max >= 0 && d > 0 && V > 0, "workspace_bytes: bad sizes");
  OCTO_CHECK_ARG(w_dtype >= OCTO_BF16 && w_dtype <= OCTO_FP8E4M3, "workspace_bytes: dtype %d", w_dtype);
  const bool need_gh = !(flags & OCTO_WS_NO_GRADH), need_gw = !(flags & OCTO_WS_NO_GRADW);
  const bool gather = flags & OCTO_WS_GATHER;
  if (flags & OCTO_WS_STEP) {
    StepLayout L;
    if (step_plan(n_max, d, V, w_dtype, need_gh, need_gw, gather, kStagingBudget, L)) {
      *bytes = L.total;
    } else {
      if (elem_bytes(staged_dtype(w_dtype)) == 2)
        return octo_fail(OCTO_EINVAL, "workspace_bytes: no step plan for V=%d in the default budget", V);
      *bytes = step_fallback_bytes(n_max, d, V, w_dtype, need_gw, gather);
    }
  } else if (flags & OCTO_WS_BACKWARD) {
    BwdLayout L;
    if (!bwd_plan(n_max, d, V, w_dtype, need_gh, need_gw, gather, kStagingBudget, L))
      return octo_fail(OCTO_EINVAL, "workspace_bytes: no backward plan for d=%d", d);
    *bytes = L.total;
  } else {
    *bytes = fwd_layout(n_max, d, V, w_dtype, flags & OCTO_WS_GATHER).total;
  }
  return OCTO_OK;
}

int octo_head_bwd_plan(int64_t n_max, int d, int V, int w_dtype, int flags, size_t ws_bytes, int64_t plan[4]) {
  OCTO_CHECK_ARG(plan != nullptr, "bwd_plan: null pointer");
  OCTO_CHECK_ARG(n_max >= 0 && d > 0 && V > 0, "bwd_plan: bad sizes");
  OCTO_CHECK_ARG(w_dtype >= OCTO_BF16 && w_dtype <= OCTO_FP8E4M3, "bwd_plan: dtype %d", w_dtype);
  const bool need_gh = !(flags & OCTO_WS_NO_GRADH), need_gw = !(flags & OCTO_WS_NO_GRADW);
  const bool gather = flags & OCTO_WS_GATHER;
  if ((flags & OCTO_WS_STEP) && elem_bytes(staged_dtype(w_dtype)) == 2) {
    StepLayout S;
    if (!step_plan_for(n_max, d, V, w_dtype, need_gh, need_gw, gather, ws_bytes, S))
      return octo_fail(OCTO_EWORKSPACE, "bwd_plan: no step plan fits %zu bytes", ws_bytes);
    plan[0] = S.P;
    plan[1] = S.passes;
    plan[2] = S.V_pad;
    plan[3] = 1;
    return OCTO_OK;
  }
  BwdLayout L;
  if (!bwd_plan_for(n_max, d, V, w_dtype, need_gh, need_gw, gather, ws_bytes, L))
    return octo_fail(OCTO_EWORKSPACE, "bwd_plan: no plan fits %zu bytes", ws_bytes);
  plan[0] = L.P;
  plan[1] = L.passes;
  plan[2] = L.Vc;
  plan[3] = L.chunks;
  return OCTO_OK;
}

int octo_head_fwd(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw, int w_dtype,
                  const float *w_scale, const int64_t *labels, const int64_t *idx, const int32_t *count,
                  int64_t n_max, int d, int V, int flags, float inv_T, float pre, float post, int use_tanh,
                  float *logp, float *ent, float *lse, float *out2, int64_t ld_out2, void *ws, size_t ws_bytes,
                  void *stream) {
  return head_fwd(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags, inv_T,
                  pre, post, use_tanh, logp, ent, lse, out2, ld_out2, nullptr, ws, ws_bytes, stream);
}

int octo_head_fwd_grpo(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw,
                       int w_dtype, const float *w_scale, const int64_t *labels, const int64_t *idx,
                       const int32_t *count, int64_t n_max, int d, int V, int flags, float inv_T, float pre,
                       float post, int use_tanh, float *logp, float *ent, float *lse, float *out2, int64_t ld_out2,
                       const octo_grpo_tail *grpo, void *ws, size_t ws_bytes, void *stream) {
  OCTO_CHECK_ARG(grpo != nullptr, "head_fwd_grpo: null grpo");
  return head_fwd(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags, inv_T,
                  pre, post, use_tanh, logp, ent, lse, out2, ld_out2, grpo, ws, ws_bytes, stream);
}

int octo_head_step_grpo(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw,
                        int w_dtype, const float *w_scale, const int64_t *labels, const int64_t *idx,
                        const int32_t *count, int64_t n_max, int d, int V, int flags, float inv_T, float pre,
                        float post, int use_tanh, float *logp, float *ent, float *lse, float *out2, int64_t ld_out2,
                        const octo_grpo_tail *grpo, void *grad_h, int64_t ld_gh, int gh_dtype, void *grad_w,
                        int gw_dtype, void *ws, size_t ws_bytes, void *stream) {
  return head_step(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, count, n_max, d, V, flags, inv_T,
                   pre, post, use_tanh, logp, ent, lse, out2, ld_out2, grpo, grad_h, ld_gh, gh_dtype, grad_w,
                   gw_dtype, ws, ws_bytes, stream);
}

int octo_head_step_grpo_pairs(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw,
                              int w_dtype, const float *w_scale, const int64_t *pair_label, const int64_t *pair_pos,
                              const int32_t *pair_count, int64_t n_pairs, int d, int V, int flags, float inv_T,
                              float pre, float post, int use_tanh, float *lse, const int64_t *flat_pair,
                              int64_t n_flat, float *out_flat, int64_t ld_out, const octo_grpo_tail *grpo,
                              void *grad_h, int64_t ld_gh, int gh_dtype, void *grad_w, int gw_dtype, void *ws,
                              size_t ws_bytes, void *stream) {
  OCTO_CHECK_ARG(pair_pos != nullptr, "head_step_grpo_pairs: null pair_pos");
  const StepPairs pm{flat_pair, n_flat, out_flat, ld_out};
  return head_step(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, pair_label, pair_pos, pair_count, n_pairs, d,
                   V, flags, inv_T, pre, post, use_tanh, nullptr, nullptr, lse, nullptr, 2, grpo, grad_h, ld_gh,
                   gh_dtype, grad_w, gw_dtype, ws, ws_bytes, stream, &pm);
}

int octo_head_bwd(const void *h, int64_t h_rows, int64_t ldh, int h_dtype, const void *w, int64_t ldw, int w_dtype,
                  const float *w_scale, const int64_t *labels, const int64_t *idx, const int32_t *count,
                  int64_t n_max, int d, int V, int flags, float inv_T, float pre, float post, int use_tanh,
                  const float *lse, const float *g, void *grad_h, int64_t ld_gh, int gh_dtype, void *grad_w,
                  int gw_dtype, void *ws, size_t ws_bytes, void *stream) {
  Common cm;
  int rc = check_common(h, h_rows, ldh, h_dtype, w, ldw, w_dtype, w_scale, labels, idx, n_max, d, V, flags, inv_T,
                        pre, post, use_tanh, cm);
  if (rc) return rc;
  OCTO_CHECK_ARG(lse && g, "head_bwd: null lse or g");
  if (grad_h) {
    OCTO_CHECK_ARG(gh_dtype == OCTO_BF16 || gh_dtype == OCTO_F16 || gh_dtype == OCTO_F32, "head_bwd: grad_h dtype");
    OCTO_CHECK_ARG(ld_gh >= d, "head_bwd: ld_gh < d");
  }
  if (grad_w) {
    if (cm.fp8) return octo_fail(OCTO_EUNSUPPORTED, "head_bwd: grad_w of fp8 weights");
    OCTO_CHECK_ARG(gw_dtype == OCTO_BF16 || gw_dtype == OCTO_F16 || gw_dtype == OCTO_F32, "head_bwd: grad_w dtype");
  }
  const bool need_gh = grad_h != nullptr, need_gw = grad_w != nullptr;
  if (n_max == 0 || (!need_gh && !need_gw)) return OCTO_OK;
  BwdLayout L;
  if (!ws || !bwd_plan_for(n_max, d, V, w_dtype, need_gh, need_gw, cm.gather, ws_bytes, L)) {
    BwdLayout Lmin;
    size_t least = 0;
    for (int q = kBudgetQMin; q <= kBudgetQMax; ++q)
      if (bwd_plan(n_max, d, V, w_dtype, need_gh, need_gw, cm.gather, staging_candidate(q), Lmin) &&
          (!least || Lmin.total < least))
        least = Lmin.total;
    return octo_fail(OCTO_EWORKSPACE, "head_bwd: workspace %zu bytes, below the smallest plan's %zu%s",
                     ws ? ws_bytes : (size_t)0, least,
                     cm.gather ? " (hidden of 2 GiB or more through idx: query with OCTO_WS_GATHER)" : "");
  }
  if (need_gw && L.passes > 1 && gw_dtype != OCTO_F32 && w_dtype == OCTO_F32)
    return octo_fail(OCTO_EUNSUPPORTED, "head_bwd: 16-bit grad_w of fp32 weights over several passes");
  hipStream_t st = (hipStream_t)stream;
  char *wsb = (char *)ws;
  void *wt = wsb + L.wt, *ht = wsb + L.ht, *dza = wsb + L.dza, *dzb = wsb + L.dzb;
  float *gacc = (float *)(wsb + L.gacc), *hacc = (float *)(wsb + L.hacc);
  const int esz = L.esz;

  void *gathered = cm.gather ? wsb + L.rows : nullptr;
  if (gathered) {
    rc = launch_rows_gather(h, ldh * cm.hesz, idx, count, n_max, (int64_t)d * cm.hesz, gathered, st);
    if (rc) return rc;
  }
  // grad_h reads the chunk's W rows (or their bf16 widening) K-major as stored, or else their staged W^T [d, Vc]
  const bool wk = gh_reads_w(d, V, w_dtype);

  for (int64_t p = 0; p < L.passes; ++p) {
    const int64_t r0 = p * L.P;
    const int64_t rows = (n_max - r0) < L.P ? (n_max - r0) : L.P;

    const Operand Bh = hidden_operand(h, ldh, idx, count, r0, rows, cm, gathered, d);
    DzArgs e;
    e.dzA = (need_gh || (need_gw && esz == 2)) ? dza : nullptr;
    e.ldA = L.Vc;
    e.dzB = (need_gw && esz == 4) ? dzb : nullptr;
    e.ldB = L.P;
    e.lse = lse;
    e.lse_pair = (flags & OCTO_LSE_PAIR) != 0;
    e.g = g;
    e.labels = labels;
    e.label_idx = (flags & OCTO_ROWS_VIA_IDX) ? idx : nullptr;
    e.row_off = r0;
    e.V = V;
    e.wscale = w_scale;
    e.c = cm.c;
    e.pre = cm.pre;
    e.gmul = cm.gmul;
    e.hit = nullptr;
    if (esz == 2) {  // the label entries of this pass's dz, written by the dz epilogue over its dense values
      HitArgs ha;
      ha.h = h;
      ha.ldh = ldh;
      ha.h_dtype = h_dtype;
      ha.idx = idx;
      ha.w = w;
      ha.ldw = ldw;
      ha.w_dtype = w_dtype;
      ha.wscale = w_scale;
      ha.labels = labels;
      ha.label_idx = e.label_idx;
      ha.lse = lse;
      ha.lse_pair = e.lse_pair;
      ha.g = g;
      ha.count = count;
      ha.r0 = r0;
      ha.rows = rows;
      ha.n_max = n_max;
      ha.d = d;
      ha.V = V;
      ha.c = cm.c;
      ha.pre = cm.pre;
      ha.gmul = cm.gmul;
      ha.use_tanh = use_tanh;
      ha.hit = (float *)(wsb + L.hit);
      rc = launch_hit(ha, st);
      if (rc) return rc;
      e.hit = ha.hit;
    }
    if (need_gw) {  // h^T [d, P] of the pass's rows, zero past the count (grad_W's K-contiguous operand)
      const int64_t rows_pad = round_up(rows, TN);
      rc = launch_transpose(idx ? h : (const char *)h + r0 * ldh * cm.hesz, ldh, h_dtype, nullptr,
                            idx ? idx + r0 : nullptr, count, r0, rows, rows_pad, d, ht, L.P, cm.dt, st);
      if (rc) return rc;
    }

    for (int64_t c = 0; c < L.chunks; ++c) {
      const int64_t v0 = c * L.Vc;
      const int64_t vc = (V - v0) < L.Vc ? (V - v0) : L.Vc;           // vocabulary rows of the chunk
      const int64_t vc_pad = (L.V_pad - v0) < L.Vc ? (L.V_pad - v0) : L.Vc;  // dz columns written (zero past V)
      const bool first_chunk = c == 0, last_chunk = c + 1 == L.chunks;

      // dz of the pass's rows over the chunk, recomputed tile by tile
      const Operand Aw = gemm_weight(w, ldw, cm, v0, vc, d, wsb + L.wide, st, rc);
      if (rc) return rc;
      e.v0 = v0;
      {
        TimedLaunch t("gemm_dz", st);
        rc = launch_gemm_dz(cm.dt, cm.fp8, use_tanh != 0, Aw, Bh, shape(vc, rows, d, kGroupM, 2, count, r0), e, st);
      }
      if (rc) return rc;

      if (need_gh) {  // grad_h[rows] (+)= dz . W[v0 .. v0 + vc)   (K = vc, or vc_pad through the staged W^T)
        if (!wk) {  // W^T [d, Vc] of the chunk's rows in the staged type (fp8: from the widened rows), zero past vc
          rc = launch_transpose(Aw.base, Aw.ld / esz, cm.dt, nullptr, nullptr, nullptr, 0, vc, L.Vc, d, wt, L.Vc,
                                cm.dt, st);
          if (rc) return rc;
        }
        const Operand A2 = plain_operand(dza, L.Vc * esz, rows, count, r0);
        const Operand B2 = wk ? plain_operand(Aw.base, Aw.ld, d, nullptr, 0) : plain_operand(wt, L.Vc * esz, d, nullptr, 0);
        const GemmShape s2 = shape(rows, d, wk ? vc : vc_pad, kGroupM, 1, count, r0);
        StoreArgs o;
        o.ld_add = d;
        if (L.chunks > 1 && !last_chunk) {  // fp32 partial sums of the chunks so far
          o.C = hacc;
          o.addend = nullptr;
          o.ldc = d;
          o.dtype = OCTO_F32;
          o.accumulate = first_chunk ? 0 : 1;
        } else {
          o.C = (char *)grad_h + r0 * ld_gh * elem_bytes(gh_dtype);
          o.addend = L.chunks > 1 ? hacc : nullptr;
          o.ldc = ld_gh;
          o.dtype = gh_dtype;
          o.accumulate = 0;
        }
        {
          TimedLaunch t("gemm_store_grad_h", st);
          rc = launch_gemm_store(cm.dt, A2, B2, s2, o, st, wk ? KM_B : KM_NONE);
        }
        if (rc) return rc;
      }
      if (need_gw) {  // grad_W[v0 .. v0 + vc) (+)= dz^T . h   (K = this pass's rows)
        const int kmajor = esz == 2 ? KM_A : KM_NONE;  // dz token-major read K-major, else the fp32 chunk-major copy
        const Operand A3 = kmajor ? plain_operand(dza, L.Vc * esz, L.P, nullptr, 0)
                                  : plain_operand(dzb, L.P * esz, L.Vc, nullptr, 0);
        const Operand B3 = plain_operand(ht, L.P * esz, d, nullptr, 0);
        rc = grad_w_pass(cm.dt, A3, kmajor, B3, vc, d, r0, rows, p, L.passes, L.gacc_on, gacc + v0 * d,
                         (char *)grad_w + v0 * d * elem_bytes(gw_dtype), gw_dtype, flags, count, st);
        if (rc) return rc;
      }
    }
  }
  return OCTO_OK;
}

}  // extern "C"
