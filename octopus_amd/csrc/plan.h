// Host-side planning of the LM-head workspaces: the forward's statistics and fp8 widening area, the backward's
// (row pass, vocabulary chunk) staging, the fused GRPO step's row passes, and the byte offset of every region inside
// the caller's workspace. Plain C++ (no HIP types), so the same code builds into libocto_head.so and, with g++ under
// -fsanitize=address,undefined, into the planner check that sweeps sizes on the CPU.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/octo_head.h"

namespace octo_plan {

constexpr int64_t kTile = 256;   // GEMM tile rows and columns (gemm_nt.h TM, TN)
constexpr size_t kStat4 = 16;    // bytes of one (m, S, U, m_b) fp32 partial per (row, vocabulary tile)

inline int64_t ceil_div(int64_t x, int64_t m) { return (x + m - 1) / m; }
inline int64_t round_to(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// The backward stages dz = g (onehot - p) / T per (row pass, vocabulary chunk): [P rows, Vc columns] in the MFMA
// type. Per chunk, grad_W rows v0 .. v0 + Vc are complete once every pass has run, and grad_h of the pass's rows sums
// over the chunks. Rows that carry across chunks (grad_h) or passes (grad_W) are summed in fp32: grad_h partials
// [P, d], grad_W partials [V, d]. For a fixed staging area P x Vc the partial round trips cost in proportion to
// 1 / Vc + 1 / P, so rows per pass are capped where the chunk is about square at the default budget.
constexpr int64_t kPassRowsMax = 32768;
// Default budget of the chunk-sized staging (dz, grad_h partials, the chunk's W^T or widened fp8 rows): 2 GiB, against
// 2 V bytes per row for the whole dz (7.5 GB at 24,576 rows and V = 151,936).
constexpr size_t kStagingBudget = (size_t)2 << 30;
// The forward widens fp8 weights to bf16 one vocabulary chunk at a time, at most this many bytes of them.
constexpr size_t kFwdWideBytes = (size_t)256 << 20;
constexpr size_t kAlign = 256;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

inline int elem_bytes(int dt) { return dt == OCTO_F32 ? 4 : (dt == OCTO_FP8E4M3 ? 1 : 2); }
// MFMA operand type for a weight dtype: fp8 weights are widened to bf16 (exactly) in the workspace, one vocabulary
// chunk at a time, and run the bf16 GEMMs with their row scale applied in the epilogues.
inline int staged_dtype(int w_dtype) { return w_dtype == OCTO_FP8E4M3 ? OCTO_BF16 : w_dtype; }

// Vocabulary chunks of Vc columns (a multiple of 256) covering V_pad: the smallest count whose chunks fit vmax, then
// balanced, then the count recomputed so that no chunk is empty.
inline void vocab_chunks(int64_t V_pad, int64_t vmax, int64_t &Vc, int64_t &chunks) {
  chunks = ceil_div(V_pad, vmax);
  Vc = round_to(ceil_div(V_pad, chunks), kTile);
  chunks = ceil_div(V_pad, Vc);
}

// Rounds of tiles (32 CUs per XCD, tiles dealt evenly to the 8 XCDs) that grad_W = dz^T . h takes over the chunks: a
// chunk of m vocabulary tiles has m x d/256 tiles of K = all the pass's rows each, so its last round, when partial,
// idles CUs for a whole long tile.
inline int64_t gradw_rounds(int64_t V_pad, int d, int64_t Vc) {
  const int64_t nd = ceil_div(d, kTile);
  int64_t rounds = 0;
  for (int64_t v0 = 0; v0 < V_pad; v0 += Vc) {
    const int64_t m = ((V_pad - v0) < Vc ? (V_pad - v0) : Vc) / kTile;
    rounds += ceil_div(ceil_div(m * nd, 8), 32);
  }
  return rounds;
}
// With grad_W asked for: of the chunk counts from the fewest that fit up to 3 more, the one whose grad_W takes the
// fewest rounds (the fewest chunks on a tie). At d 4096, V 128,256: 8 chunks of 63 vocabulary tiles, 32 rounds, where
// 5 chunks of 101 take 35 (202 tiles per XCD in each: 6.3 rounds of 32).
inline void gradw_rounds_chunks(int64_t V_pad, int d, int64_t &Vc, int64_t &chunks) {
  int64_t best = gradw_rounds(V_pad, d, Vc);
  const int64_t c0 = chunks;
  for (int64_t c = c0 + 1; c <= c0 + 3; ++c) {
    const int64_t vc = round_to(ceil_div(V_pad, c), kTile);
    const int64_t r = gradw_rounds(V_pad, d, vc);
    if (r < best) {
      best = r;
      Vc = vc;
      chunks = ceil_div(V_pad, vc);
    }
  }
}

struct FwdLayout {
  int64_t mtiles, Vc, chunks;
  size_t part, wide, z, rows, total;
};
// Bytes of the contiguous copy of the n_max gathered hidden rows [n_max, d] (OCTO_WS_GATHER).
inline size_t gather_bytes(int64_t n_max, int d, int h_dtype) {
  return align_up((size_t)n_max * d * elem_bytes(h_dtype));
}

// part: (m, S, U) per (row, vocab tile). wide: one chunk of fp8 weights widened to bf16 [Vc, d] (the forward GEMM runs
// once per chunk; one chunk covering V for 16-bit weights). z: the GRPO tail's token count. rows: the gathered hidden
// rows, when asked for (last, so the other offsets do not depend on it).
inline FwdLayout fwd_layout(int64_t n_max, int d, int V, int w_dtype, bool gather) {
  FwdLayout L;
  L.mtiles = ceil_div(V, kTile);
  const int64_t V_pad = L.mtiles * kTile;
  if (w_dtype == OCTO_FP8E4M3) {
    const int64_t vmax = (int64_t)(kFwdWideBytes / ((size_t)d * 2)) / kTile * kTile;
    vocab_chunks(V_pad, vmax < kTile ? kTile : vmax, L.Vc, L.chunks);
  } else {
    L.Vc = V_pad;
    L.chunks = 1;
  }
  L.part = 0;
  size_t off = align_up((size_t)n_max * L.mtiles * kStat4);
  L.wide = off;
  if (w_dtype == OCTO_FP8E4M3) off += align_up((size_t)L.Vc * d * 2);
  L.z = off;
  off += kAlign;
  L.rows = off;
  if (gather) off += gather_bytes(n_max, d, w_dtype == OCTO_FP8E4M3 ? OCTO_BF16 : w_dtype);
  L.total = off;
  return L;
}

// The backward stages the gradient GEMMs' operands so each mainloop row fetch is whole cache lines: the pass's
// hidden rows transposed to h^T [d, P] for grad_W = dz^T . h, and dz token-major [P, Vc] per vocabulary chunk, which
// grad_h reads K-contiguous and 16-bit grad_W K-major (transposing LDS reads). 16-bit grad_h = dz . W reads the
// chunk's W rows K-major as stored when V is a multiple of 64 (the loader's K-row granule) and d of 256 (its column
// granule); otherwise, and for fp32, the chunk's W^T [d, Vc] is staged. fp32 dz is also written chunk-major [Vc, P]
// for the fp32 loop, which reads K-contiguous operands only.
inline bool gh_reads_w(int d, int V, int w_dtype) {
  return elem_bytes(staged_dtype(w_dtype)) == 2 && V % 64 == 0 && d % 256 == 0;
}
struct BwdLayout {
  int64_t P, passes, Vc, chunks, V_pad;
  int esz;
  bool hacc_on, gacc_on;
  size_t wt, ht, dza, dzb, hit, wide, hacc, gacc, rows, total;
};

// The plan for a staging budget (0: unbounded, one chunk). Rows per pass start at kPassRowsMax (balanced over the
// passes); the chunk width is the widest multiple of 256 whose staging fits the budget, and rows per pass halve
// while not even 256 columns fit. Returns false when no plan fits (a budget below one 256 x 256 chunk).
inline bool bwd_plan(int64_t n_max, int d, int V, int w_dtype, bool need_gh, bool need_gw, bool gather,
                     size_t budget, BwdLayout &L) {
  L.esz = elem_bytes(staged_dtype(w_dtype));
  L.V_pad = round_to(V, kTile);
  const bool dz_a = need_gh || (need_gw && L.esz == 2), dz_b = need_gw && L.esz == 4;
  const bool wt = need_gh && !gh_reads_w(d, V, w_dtype), wide = w_dtype == OCTO_FP8E4M3;
  L.P = L.passes = 0;
  L.Vc = L.V_pad;
  L.chunks = 1;
  if (n_max > 0) {
    int64_t passes = ceil_div(n_max, kPassRowsMax);
    for (;;) {
      const int64_t P = round_to(ceil_div(n_max, passes), kTile);
      const size_t per_col = (size_t)P * L.esz * ((dz_a ? 1 : 0) + (dz_b ? 1 : 0)) + (wt ? (size_t)d * L.esz : 0) +
                             (wide ? (size_t)d * 2 : 0);  // staging bytes per vocabulary column of a chunk
      int64_t Vc = 0, chunks = 0;
      if (budget == 0 || per_col * (size_t)L.V_pad <= budget) {
        Vc = L.V_pad;
        chunks = 1;
      } else {
        const size_t hb = need_gh ? (size_t)P * d * sizeof(float) : 0;  // grad_h partials, with more than one chunk
        if (budget > hb) {
          const int64_t vmax = (int64_t)((budget - hb) / per_col) / kTile * kTile;
          if (vmax >= kTile) vocab_chunks(L.V_pad, vmax, Vc, chunks);
          if (vmax >= kTile && need_gw) gradw_rounds_chunks(L.V_pad, d, Vc, chunks);
        }
      }
      if (chunks > 0) {
        L.P = P;
        L.passes = ceil_div(n_max, P);
        L.Vc = Vc;
        L.chunks = chunks;
        break;
      }
      if (P <= kTile) return false;
      passes = ceil_div(n_max, P / 2);
    }
  }
  L.hacc_on = need_gh && L.chunks > 1;
  L.gacc_on = need_gw && L.passes > 1 && w_dtype != OCTO_F32;
  size_t off = 0;
  L.wt = off;  // W^T [d, Vc] of the chunk (grad_h, unless it reads W K-major)
  if (wt) off += align_up((size_t)d * L.Vc * L.esz);
  L.ht = off;  // h^T [d, P] of the pass's rows (grad_W)
  if (need_gw) off += align_up((size_t)d * L.P * L.esz);
  L.dza = off;  // dz [P, Vc], token-major (grad_h; 16-bit grad_W)
  if (dz_a) off += align_up((size_t)L.P * L.Vc * L.esz);
  L.dzb = off;  // dz [Vc, P], chunk-major (fp32 grad_W)
  if (dz_b) off += align_up((size_t)L.Vc * L.P * L.esz);
  L.hit = off;  // dz at each row's label [P] fp32 (16-bit dz epilogue)
  if (L.esz == 2) off += align_up((size_t)L.P * sizeof(float));
  L.wide = off;  // the chunk's fp8 weights widened to bf16 [Vc, d] (the dz recompute's and grad_h's operand)
  if (wide) off += align_up((size_t)L.Vc * d * 2);
  L.hacc = off;  // fp32 grad_h partial sums across chunks [P, d]
  if (L.hacc_on) off += align_up((size_t)L.P * d * sizeof(float));
  L.gacc = off;  // fp32 grad_W partial sums across passes, for a 16-bit grad_W
  if (L.gacc_on) off += align_up((size_t)V * d * sizeof(float));
  L.rows = off;  // the gathered hidden rows (OCTO_WS_GATHER), last
  if (gather) off += gather_bytes(n_max, d, w_dtype == OCTO_FP8E4M3 ? OCTO_BF16 : w_dtype);
  L.total = off;
  return true;
}

// Candidate staging budgets, largest first: 2^(q / 4) bytes for q = 160 .. 80 (2^40 down to 2^20 in steps of 2^(1/4),
// 2^31 among them).
inline size_t staging_candidate(int q) {
  static const uint32_t frac[4] = {4096, 4871, 5793, 6889};  // 2^(j / 4) x 4096
  return ((size_t)1 << (q / 4 - 12)) * frac[q % 4];
}
constexpr int kBudgetQMax = 160, kBudgetQMin = 80;

// The plan the backward runs in ws_bytes of workspace: unbounded if it fits, else the largest candidate staging
// budget whose plan fits. With the queried size (the plan at kStagingBudget = 2^31, a candidate) this is that plan or
// one with fewer chunks in no more bytes. Returns false when none fits.
inline bool bwd_plan_for(int64_t n_max, int d, int V, int w_dtype, bool need_gh, bool need_gw, bool gather,
                         size_t ws_bytes, BwdLayout &L) {
  if (bwd_plan(n_max, d, V, w_dtype, need_gh, need_gw, gather, 0, L) && L.total <= ws_bytes) return true;
  for (int q = kBudgetQMax; q >= kBudgetQMin; --q)
    if (bwd_plan(n_max, d, V, w_dtype, need_gh, need_gw, gather, staging_candidate(q), L) && L.total <= ws_bytes)
      return true;
  return false;
}

// ---- the fused GRPO step's plan (octo_head_step_grpo) ----------------------------------------------------
// The step runs the rows in passes of P; per pass its forward GEMM stores, besides the statistics, every element's
// exponential (StatsArgs::ex) into a [P, V_pad] staging area: bf16, relative to the row's offset (StatsArgs::xoff),
// so that dz is one scale per row times it (launch_ex_fix sets the scales); f16, relative to its half tile's maximum,
// turned into dz by launch_dz_scale once the merge has the rows' (m2, l2S) and g. The gradient GEMMs read it as the
// backward's read their dz. Rows per pass: the most that fit the staging budget (at most kPassRowsMax), balanced over
// the passes.
// The staging is the only part that grows with the budget; outside it sit the pass's statistics [P, V / 256], h^T
// [d, P], the label entries [P], fp32 grad_W partials [V, d] over several passes, and, once per call, W widened to
// bf16 (fp8 weights) or staged as W^T (16-bit weights that grad_h cannot read K-major as stored).
struct StepLayout {
  int64_t P, passes, mtiles, V_pad;
  int esz;
  bool gacc_on, wide_on, wt_on;
  size_t part, z, hit, rowout, xoff, tdot, xuse, scale, flags, ht, dz, wide, wt, gacc, rows, total;
};

// Rows per pass when grad_h is asked for: each pass's grad_h is one tile per CU per round of long tiles (K = V), so
// a pass whose tiles overrun a multiple of the 256 CUs pays a whole extra round for the overrun, with or without
// grad_W's short tiles beside them in the same launch (those fill the CUs the long tiles leave, but cannot start the
// overrun early). Of the pass sizes up to pmax (multiples of 256), the one whose passes take the fewest grad_h rounds
// in total, the largest (up to the rows there are) on a tie: at d 2560 and 131,072 rows, 25 x 256 rows (250 tiles,
// 21 passes, 21 rounds) against 27 x 256 (270 tiles, 19 passes, 38 rounds); at 32,768 rows, 25 x 256 (6 passes,
// 6 rounds) against 26 x 256 (260 tiles: 5 passes, 9 rounds).
inline int64_t gradh_pass_rows(int64_t n_max, int d, int64_t pmax) {
  const int64_t nt = ceil_div(n_max, kTile), nd = ceil_div(d, kTile), cus = 256;
  int64_t best_p = 0, best_r = 0;
  for (int64_t p = (pmax / kTile < nt ? pmax / kTile : nt); p >= 1; --p) {
    const int64_t passes = ceil_div(nt, p), last = nt - (passes - 1) * p;
    const int64_t r = (passes - 1) * ceil_div(p * nd, cus) + ceil_div(last * nd, cus);
    if (!best_p || r < best_r) {
      best_p = p;
      best_r = r;
    }
  }
  return best_p * kTile;
}

// grad_h reads W^T K-contiguous faster than W K-major (its B fragments one ds_read_b128 each rather than two
// transposing reads): 57.3 against 60.3 ms per step at 114,688 rows, d 2560, V 151,936 (grad_h alone, fp8 weights
// widened), for a transpose of the weight once per call (about 0.3 ms at 0.78 GB). Beside grad_W in the same launch
// the gain is smaller (24,576 rows: the launches 0.4 ms faster, the step equal), so W^T is staged by choice only when
// grad_h is the only gradient and the rows reach kWtRows.
constexpr int64_t kWtRows = 16384;

// False when the budget holds fewer than 256 rows, or for fp32 operands (the step then runs the forward and the
// backward: step_fallback). opt_wt: stage W^T where it pays (kWtRows); it is staged regardless where grad_h cannot
// read W as stored.
inline bool step_plan(int64_t n_max, int d, int V, int w_dtype, bool need_gh, bool need_gw, bool gather,
                      size_t budget, StepLayout &L, bool opt_wt = true) {
  L.esz = elem_bytes(staged_dtype(w_dtype));
  if (L.esz != 2) return false;
  L.mtiles = ceil_div(V, kTile);
  L.V_pad = L.mtiles * kTile;
  int64_t pmax = kPassRowsMax;
  if (budget) {
    const int64_t fit = (int64_t)(budget / ((size_t)L.V_pad * L.esz)) / kTile * kTile;
    if (fit < kTile) return false;
    if (fit < pmax) pmax = fit;
  }
  L.passes = n_max > 0 ? ceil_div(n_max, pmax) : 0;
  L.P = n_max > 0 ? round_to(ceil_div(n_max, L.passes), kTile) : 0;
  if (n_max > 0 && need_gh) L.P = gradh_pass_rows(n_max, d, pmax);
  L.passes = n_max > 0 ? ceil_div(n_max, L.P) : 0;
  L.gacc_on = need_gw && L.passes > 1;
  L.wide_on = w_dtype == OCTO_FP8E4M3;
  L.wt_on = need_gh && (!gh_reads_w(d, V, w_dtype) || (opt_wt && !need_gw && n_max >= kWtRows));
  size_t off = 0;
  L.part = off;  // (m, S, U) per (row of the pass, vocabulary tile)
  off += align_up((size_t)L.P * L.mtiles * kStat4);
  L.z = off;  // the GRPO tail's token count
  off += kAlign;
  L.hit = off;  // dz at each row's label per unit of g gmul [P] fp32
  off += align_up((size_t)L.P * sizeof(float));
  L.rowout = off;  // (logprob, entropy) per compact row [n_max, 2] fp32, for the pair-row GRPO tail
  off += align_up((size_t)n_max * 2 * sizeof(float));
  // bf16 operands, the row-offset exponentials: each compact row's offset and target dot [n_max] fp32; per pass row
  // the offset in use and the dz scale [P] fp32, the flagged rows [P] int32; a flag count per pass
  L.xoff = off;
  off += align_up((size_t)n_max * sizeof(float));
  L.tdot = off;
  off += align_up((size_t)n_max * sizeof(float));
  L.xuse = off;
  off += align_up((size_t)L.P * sizeof(float));
  L.scale = off;
  off += align_up((size_t)L.P * sizeof(float));
  L.flags = off;  // flag counts [passes], then the flagged rows [P]
  off += align_up((size_t)(L.passes + L.P) * sizeof(int32_t));
  L.ht = off;  // h^T [d, P] of the pass's rows (grad_W)
  if (need_gw) off += align_up((size_t)d * L.P * L.esz);
  L.dz = off;  // the exponentials, then dz [P, V_pad], token-major
  off += align_up((size_t)L.P * L.V_pad * L.esz);
  L.wide = off;  // fp8 weights widened to bf16 [V, d]
  if (L.wide_on) off += align_up((size_t)V * d * 2);
  L.wt = off;  // W^T [d, V_pad] (grad_h: when it cannot read W K-major, or by choice)
  if (L.wt_on) off += align_up((size_t)d * L.V_pad * L.esz);
  L.gacc = off;  // fp32 grad_W partial sums across passes (tile-blocked over V_pad rows when d % 256 == 0)
  if (L.gacc_on) off += align_up((size_t)(d % kTile == 0 ? L.V_pad : V) * d * sizeof(float));
  L.rows = off;  // the gathered hidden rows (OCTO_WS_GATHER), last
  if (gather) off += gather_bytes(n_max, d, w_dtype == OCTO_FP8E4M3 ? OCTO_BF16 : w_dtype);
  L.total = off;
  return true;
}

// The plan the step runs in ws_bytes: unbounded if it fits, else the largest candidate staging budget that fits; at
// each budget the optional W^T first, then without it (a workspace short of the W^T keeps the larger passes).
inline bool step_plan_for(int64_t n_max, int d, int V, int w_dtype, bool need_gh, bool need_gw, bool gather,
                          size_t ws_bytes, StepLayout &L) {
  for (int q = kBudgetQMax + 1; q >= kBudgetQMin; --q) {
    const size_t budget = q > kBudgetQMax ? 0 : staging_candidate(q);
    for (int opt = 1; opt >= 0; --opt)
      if (step_plan(n_max, d, V, w_dtype, need_gh, need_gw, gather, budget, L, opt != 0) && L.total <= ws_bytes)
        return true;
  }
  return false;
}

// Workspace of the step for fp32 operands: the forward's, then the backward's (at the default budget), in turn.
inline size_t step_fallback_bytes(int64_t n_max, int d, int V, int w_dtype, bool need_gw, bool gather) {
  const size_t f = fwd_layout(n_max, d, V, w_dtype, gather).total;
  BwdLayout B;
  const size_t b = bwd_plan(n_max, d, V, w_dtype, true, need_gw, gather, kStagingBudget, B) ? B.total : 0;
  return f > b ? f : b;
}

}  // namespace octo_plan
