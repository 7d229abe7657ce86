// CPU check of the host-side workspace planners (octopus_amd/csrc/plan.h) and of the GEMMs' workgroup -> tile order
// (octopus_amd/csrc/tile_order.h), built by tests/test_plan_sanitized.py with g++ -fsanitize=address,undefined so
// that any out-of-bounds access, overflow or undefined shift in that code stops the run.
//
// Over a sweep of row counts, widths, vocabulary sizes, weight types, gradient sets, gathers and budgets it checks
// that every region a plan carves lies inside the workspace total, that no two regions overlap, that each K-major
// read of a gradient GEMM (the loader fetches K-rows up to the next multiple of 64) stays inside its buffer, that a
// plan fits the workspace it was chosen for, and that the tile order visits every tile of a grid exactly once.
// Prints "ok" and returns 0, or the first failures and returns 1.
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "../octopus_amd/csrc/plan.h"
#include "../octopus_amd/csrc/tile_order.h"

using namespace octo_plan;

static int failures = 0;
static long checks = 0;

#define CHECK(cond, ...)                                        \
  do {                                                          \
    ++checks;                                                   \
    if (!(cond)) {                                              \
      if (failures++ < 20) {                                    \
        fprintf(stderr, "FAIL line %d: %s: ", __LINE__, #cond); \
        fprintf(stderr, __VA_ARGS__);                           \
        fprintf(stderr, "\n");                                  \
      }                                                         \
    }                                                           \
  } while (0)

struct Region {
  const char *name;
  size_t off, bytes;
};

// Every region within [0, total), 256-byte aligned, and no two non-empty regions overlapping.
static void check_regions(std::vector<Region> r, size_t total, const char *what, long long n, int d, int V) {
  for (const Region &x : r) {
    CHECK(x.off % kAlign == 0, "%s %s: offset %zu unaligned (n %lld d %d V %d)", what, x.name, x.off, n, d, V);
    CHECK(x.off + x.bytes <= total, "%s %s: [%zu, %zu) past total %zu (n %lld d %d V %d)", what, x.name, x.off,
          x.off + x.bytes, total, n, d, V);
  }
  r.erase(std::remove_if(r.begin(), r.end(), [](const Region &x) { return x.bytes == 0; }), r.end());
  std::sort(r.begin(), r.end(), [](const Region &a, const Region &b) { return a.off < b.off; });
  for (size_t i = 1; i < r.size(); ++i)
    CHECK(r[i - 1].off + r[i - 1].bytes <= r[i].off, "%s: %s [%zu, +%zu) overlaps %s at %zu (n %lld d %d V %d)", what,
          r[i - 1].name, r[i - 1].off, r[i - 1].bytes, r[i].name, r[i].off, n, d, V);
}

// The bytes each kernel of the step touches in each region (the sizes the kernels index up to), from the conditions
// under which the step's code uses each region, not from the plan's own flags.
static void check_step(const StepLayout &L, int64_t n_max, int d, int V, int w_dtype, bool need_gh, bool need_gw,
                       bool gather) {
  const size_t esz = L.esz, hesz = w_dtype == OCTO_FP8E4M3 ? 2 : elem_bytes(w_dtype);
  std::vector<Region> r = {
      {"part", L.part, (size_t)L.P * L.mtiles * kStat4},
      {"z", L.z, 4},
      {"hit", L.hit, (size_t)L.P * 4},
      {"rowout", L.rowout, (size_t)n_max * 8},
      {"xoff", L.xoff, (size_t)n_max * 4},
      {"tdot", L.tdot, (size_t)n_max * 4},
      {"xuse", L.xuse, (size_t)L.P * 4},
      {"scale", L.scale, (size_t)L.P * 4},
      {"flags", L.flags, (size_t)(L.passes + L.P) * 4},
      {"ht", L.ht, need_gw ? (size_t)d * L.P * esz : 0},
      {"dz", L.dz, (size_t)L.P * L.V_pad * esz},
      {"wide", L.wide, w_dtype == OCTO_FP8E4M3 ? (size_t)V * d * 2 : 0},
      {"wt", L.wt, L.wt_on || (need_gh && !gh_reads_w(d, V, w_dtype)) ? (size_t)d * L.V_pad * esz : 0},
      {"gacc", L.gacc, need_gw && L.passes > 1 ? (size_t)(d % kTile == 0 ? L.V_pad : V) * d * 4 : 0},
      {"rows", L.rows, gather ? (size_t)n_max * d * hesz : 0},
  };
  check_regions(r, L.total, "step", n_max, d, V);
  CHECK(L.P % kTile == 0 && L.P * L.passes >= n_max && (L.passes == 0 || L.P * (L.passes - 1) < n_max),
        "step passes: P %lld passes %lld n %lld", (long long)L.P, (long long)L.passes, (long long)n_max);
  CHECK(L.V_pad % kTile == 0 && L.V_pad >= V && L.V_pad - V < kTile, "step V_pad %lld V %d", (long long)L.V_pad, V);
  for (int64_t p = 0; p < L.passes; ++p) {  // grad_W reads dz [rows, V_pad] K-major: K-rows up to round_to(rows, 64)
    const int64_t rows = std::min(L.P, n_max - p * L.P);
    CHECK((size_t)round_to(rows, 64) * L.V_pad * esz <= (size_t)L.P * L.V_pad * esz, "step dz K-major pass %lld",
          (long long)p);
  }
  if (need_gh && !L.wt_on)  // grad_h reads W [V, d] K-major as stored: K-rows up to round_to(V, 64) must exist
    CHECK(round_to(V, 64) == V && d % kTile == 0, "step W K-major: V %d d %d", V, d);
}

static void check_bwd(const BwdLayout &L, int64_t n_max, int d, int V, int w_dtype, bool need_gh, bool need_gw,
                      bool gather) {
  const size_t esz = L.esz, hesz = w_dtype == OCTO_FP8E4M3 ? 2 : elem_bytes(w_dtype);
  const bool dz_a = need_gh || (need_gw && esz == 2), dz_b = need_gw && esz == 4;
  const bool wt = need_gh && !gh_reads_w(d, V, w_dtype);
  std::vector<Region> r = {
      {"wt", L.wt, wt ? (size_t)d * L.Vc * esz : 0},
      {"ht", L.ht, need_gw ? (size_t)d * L.P * esz : 0},
      {"dza", L.dza, dz_a ? (size_t)L.P * L.Vc * esz : 0},
      {"dzb", L.dzb, dz_b ? (size_t)L.Vc * L.P * esz : 0},
      {"hit", L.hit, esz == 2 ? (size_t)L.P * 4 : 0},
      {"wide", L.wide, w_dtype == OCTO_FP8E4M3 ? (size_t)L.Vc * d * 2 : 0},
      {"hacc", L.hacc, need_gh && L.chunks > 1 ? (size_t)L.P * d * 4 : 0},
      {"gacc", L.gacc, need_gw && L.passes > 1 && esz == 2 ? (size_t)V * d * 4 : 0},
      {"rows", L.rows, gather ? (size_t)n_max * d * hesz : 0},
  };
  check_regions(r, L.total, "bwd", n_max, d, V);
  if (n_max > 0) {
    CHECK(L.P % kTile == 0 && L.P * L.passes >= n_max && L.P * (L.passes - 1) < n_max, "bwd passes");
    CHECK(L.Vc % kTile == 0 && L.Vc * L.chunks >= L.V_pad && L.Vc * (L.chunks - 1) < L.V_pad, "bwd chunks: Vc %lld",
          (long long)L.Vc);
  }
  for (int64_t p = 0; p < L.passes && dz_a; ++p) {  // grad_W reads the chunk's dz [rows, Vc] K-major
    const int64_t rows = std::min(L.P, n_max - p * L.P);
    CHECK((size_t)round_to(rows, 64) <= (size_t)L.P, "bwd dz K-major pass %lld", (long long)p);
  }
  if (need_gh && !wt) {  // grad_h reads each chunk's W rows [v0, v0 + vc) K-major: up to round_to(vc, 64) rows of W
    for (int64_t v0 = 0; v0 < V; v0 += L.Vc) {
      const int64_t vc = std::min<int64_t>(L.Vc, V - v0);
      CHECK(v0 + round_to(vc, 64) <= V, "bwd W K-major chunk at %lld (V %d)", (long long)v0, V);
    }
  }
}

static void check_fwd(int64_t n_max, int d, int V, int w_dtype, bool gather) {
  const FwdLayout L = fwd_layout(n_max, d, V, w_dtype, gather);
  const size_t hesz = w_dtype == OCTO_FP8E4M3 ? 2 : elem_bytes(w_dtype);
  std::vector<Region> r = {
      {"part", L.part, (size_t)n_max * L.mtiles * kStat4},
      {"wide", L.wide, w_dtype == OCTO_FP8E4M3 ? (size_t)L.Vc * d * 2 : 0},
      {"z", L.z, 4},
      {"rows", L.rows, gather ? (size_t)n_max * d * hesz : 0},
  };
  check_regions(r, L.total, "fwd", n_max, d, V);
  CHECK(L.Vc % kTile == 0 && L.Vc * L.chunks >= round_to(V, kTile), "fwd chunks");
}

// Every tile of an mtiles x ntiles grid visited exactly once by the 8 XCDs' tile lists, and the grid large enough.
static void check_tiles(int64_t mtiles, int64_t ntiles, int group_m) {
  std::vector<unsigned char> seen((size_t)(mtiles * ntiles), 0);
  int64_t most = 0, total = 0;
  for (int x = 0; x < 8; ++x) {
    const int64_t n = octo_tiles::xcd_tiles(x, mtiles, ntiles);
    most = std::max(most, n);
    total += n;
    for (int64_t k = 0; k <= n; ++k) {
      int mt = -1, nt = -1;
      const bool ok = octo_tiles::tile_at(group_m, x, k, mtiles, ntiles, mt, nt);
      if (k == n) {
        CHECK(!ok || k < (mtiles / 8) * ntiles, "tile %lld of XCD %d past its %lld (%lldx%lld g%d)", (long long)k, x,
              (long long)n, (long long)mtiles, (long long)ntiles, group_m);
        continue;
      }
      CHECK(ok && mt >= 0 && mt < mtiles && nt >= 0 && nt < ntiles, "tile %lld of XCD %d: (%d, %d) in %lldx%lld g%d",
            (long long)k, x, mt, nt, (long long)mtiles, (long long)ntiles, group_m);
      if (ok && mt >= 0 && mt < mtiles && nt >= 0 && nt < ntiles) {
        unsigned char &s = seen[(size_t)(mt * ntiles + nt)];
        CHECK(s == 0, "tile (%d, %d) visited twice (%lldx%lld g%d)", mt, nt, (long long)mtiles, (long long)ntiles,
              group_m);
        s = 1;
      }
    }
  }
  CHECK(total == mtiles * ntiles, "%lld tiles listed for %lldx%lld", (long long)total, (long long)mtiles,
        (long long)ntiles);
  CHECK(8 * most <= octo_tiles::tile_grid(mtiles, ntiles), "grid %lld for %lld per XCD",
        (long long)octo_tiles::tile_grid(mtiles, ntiles), (long long)most);
}

int main() {
  const int64_t ns[] = {0, 1, 255, 256, 257, 1000, 3000, 6400, 24576, 32768, 32769, 65536, 131072};
  const int ds[] = {8, 64, 136, 256, 2560, 4096};
  const int Vs[] = {100, 5000, 32000, 128256, 151936, 151937};
  const int dts[] = {OCTO_BF16, OCTO_F16, OCTO_F32, OCTO_FP8E4M3};
  const int qs[] = {kBudgetQMin, 100, 120, 124, 140, kBudgetQMax};
  for (int64_t n : ns)
    for (int d : ds)
      for (int V : Vs)
        for (int dt : dts) {
          if (dt == OCTO_FP8E4M3 && d % 16) continue;  // the head's argument checks: fp8 rows of 16 bytes
          for (int gather = 0; gather < 2; ++gather) {
            check_fwd(n, d, V, dt, gather);
            for (int gset = 1; gset < 4; ++gset) {
              const bool gh = gset & 1, gw = gset & 2;
              if (dt == OCTO_FP8E4M3 && gw) continue;  // no grad_W of fp8 weights
              for (int q : qs) {
                BwdLayout B;
                if (bwd_plan(n, d, V, dt, gh, gw, gather, staging_candidate(q), B))
                  check_bwd(B, n, d, V, dt, gh, gw, gather);
                StepLayout S;
                for (int opt = 0; opt < 2; ++opt)
                  if (step_plan(n, d, V, dt, gh, gw, gather, staging_candidate(q), S, opt != 0))
                    check_step(S, n, d, V, dt, gh, gw, gather);
              }
              // the plan chosen for a workspace fits it
              BwdLayout B0;
              if (n <= 32768 && bwd_plan(n, d, V, dt, gh, gw, gather, kStagingBudget, B0)) {
                for (size_t ws : {B0.total, B0.total / 3, (size_t)(64 << 20)}) {
                  BwdLayout B;
                  if (bwd_plan_for(n, d, V, dt, gh, gw, gather, ws, B)) {
                    CHECK(B.total <= ws, "bwd plan of %zu bytes in %zu", B.total, ws);
                    check_bwd(B, n, d, V, dt, gh, gw, gather);
                  }
                }
              }
              StepLayout S0;
              if (n <= 32768 && step_plan(n, d, V, dt, gh, gw, gather, kStagingBudget, S0)) {
                for (size_t ws : {S0.total, S0.total / 3, (size_t)(64 << 20)}) {
                  StepLayout S;
                  if (step_plan_for(n, d, V, dt, gh, gw, gather, ws, S)) {
                    CHECK(S.total <= ws, "step plan of %zu bytes in %zu", S.total, ws);
                    check_step(S, n, d, V, dt, gh, gw, gather);
                  }
                }
              }
            }
          }
        }
  for (int64_t m = 1; m <= 40; ++m)
    for (int64_t nn = 1; nn <= 30; ++nn)
      for (int g : {1, 2, 4, 8}) check_tiles(m, nn, g);
  for (int g : {1, 4}) {
    check_tiles(594, 25, g);   // the logits GEMM of a 6,400-row pass at V 151,936
    check_tiles(594, 10, g);   // grad_W at d 2560
    check_tiles(25, 10, g);    // grad_h of a pass
    check_tiles(99, 10, g);    // a vocabulary chunk of 99 tiles
    check_tiles(501, 16, g);   // d 4096, V 128,256
  }
  if (failures) {
    fprintf(stderr, "%d of %ld checks failed\n", failures, checks);
    return 1;
  }
  printf("ok %ld checks\n", checks);
  return 0;
}
