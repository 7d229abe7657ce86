// The label-pair section of a prefix tree on the device (octopus/rl/prefix_tree.py:156-166):
//
//   a flat position p "asks" when it is scored, and p is not the last position of its sequence;
//   its ask is (tree position flat_to_tree[p], label flat[p + 1]);
//   equal asks share one pair; pairs are numbered in ascending (tree position, label) order;
//   flat_pair[p] = the pair of p's ask, or "none" (-1, or the pair count: the appended zero row of
//   TreeMeta, prefix_tree.py:203-205).
//
// The reference packs (position, label) into one int64 and runs np.unique over the flat positions. Here the
// asks are bucketed by tree position instead (a counting sort: one atomic per ask, a scan over positions),
// each bucket sorted by label (buckets hold one ask per sequence through that position, so they are short),
// and the distinct labels per position scanned into pair numbers. Every output is independent of the
// order in which the atomics land: a bucket's content is sorted before it is numbered.
//
// Workspace (int32 unless noted): cnt, start, fill, distinct, base [T_tree]; lab [T_flat] int64; src [T_flat];
// ends [T_flat] uint8; a 16-byte header of totals.
#include "octo_common.h"

namespace octo {

struct PairsWs {
  int32_t *cnt, *start, *fill, *uniq, *base, *src, *tot;
  int64_t *lab;
  uint8_t *ends;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static size_t pairs_ws_layout(int64_t T_flat, int64_t T_tree, char *ws, PairsWs *w) {
  size_t off = 0;
  auto take = [&](size_t bytes) { char *p = ws ? ws + off : nullptr; off += align256(bytes); return p; };
  char *tot = take(16);
  char *cnt = take((size_t)T_tree * 4), *start = take((size_t)T_tree * 4), *fill = take((size_t)T_tree * 4);
  char *uniq = take((size_t)T_tree * 4), *base = take((size_t)T_tree * 4);
  char *lab = take((size_t)T_flat * 8), *src = take((size_t)T_flat * 4), *ends = take((size_t)T_flat);
  if (w) {
    w->tot = (int32_t *)tot;
    w->cnt = (int32_t *)cnt;
    w->start = (int32_t *)start;
    w->fill = (int32_t *)fill;
    w->uniq = (int32_t *)uniq;
    w->base = (int32_t *)base;
    w->lab = (int64_t *)lab;
    w->src = (int32_t *)src;
    w->ends = (uint8_t *)ends;
  }
  return off;
}

__global__ __launch_bounds__(256) void pairs_init_kernel(PairsWs w, int64_t T_flat, int64_t T_tree, int32_t *count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < T_tree) {
    w.cnt[i] = 0;
    w.fill[i] = 0;
  }
  if (i < T_flat) w.ends[i] = 0;
  if (i < 4) w.tot[i] = 0;
  if (i < 2) count[i] = 0;
}

// ends[cu[s + 1] - 1] = 1 for every sequence s (index -1 is the last flat position, as numpy reads it)
__global__ __launch_bounds__(256) void pairs_ends_kernel(const int64_t *cu, int64_t n_seq, int64_t T_flat, PairsWs w) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= n_seq) return;
  int64_t e = cu[s + 1] - 1;
  if (e < 0) e += T_flat;
  if (e >= 0 && e < T_flat) w.ends[e] = 1;
}

// The ask of flat position p, or -1: its tree position when in [0, T_tree); an out-of-range position is
// counted in count[1] (by pairs_count_kernel only) and treated as no ask.
__device__ __forceinline__ int64_t ask_pos(int64_t p, int64_t T_flat, const uint8_t *scored, const PairsWs &w,
                                           const int64_t *f2t, int64_t T_tree, bool &bad) {
  bad = false;
  if (p + 1 >= T_flat || w.ends[p] || (scored && !scored[p])) return -1;
  const int64_t pos = f2t[p];
  if (pos < 0 || pos >= T_tree) {
    bad = true;
    return -1;
  }
  return pos;
}

__global__ __launch_bounds__(256) void pairs_count_kernel(int64_t T_flat, const uint8_t *scored, const int64_t *f2t,
                                                          int64_t T_tree, PairsWs w, int32_t *count) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= T_flat) return;
  bool bad;
  const int64_t pos = ask_pos(p, T_flat, scored, w, f2t, T_tree, bad);
  if (pos >= 0) atomicAdd(&w.cnt[pos], 1);
  if (bad) atomicAdd(&count[1], 1);
}

// Exclusive scan of in[0, n) into out, total into *total. One workgroup of 16 waves, 1024 entries per sweep:
// a shuffle scan per wave, the wave totals through LDS.
__global__ __launch_bounds__(1024) void scan_i32_kernel(const int32_t *in, int64_t n, int32_t *out, int32_t *total) {
  __shared__ int wsum[16];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int carry = 0;
  for (int64_t s0 = 0; s0 < n; s0 += 1024) {
    const int64_t i = s0 + threadIdx.x;
    const int v = i < n ? in[i] : 0;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wv] = x;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int c = wsum[k];
      off += (k < wv) ? c : 0;
      tot += c;
    }
    if (i < n) out[i] = carry + off + x - v;
    carry += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) *total = carry;
}

__global__ __launch_bounds__(256) void pairs_fill_kernel(const int64_t *flat, int64_t T_flat, const uint8_t *scored,
                                                         const int64_t *f2t, int64_t T_tree, PairsWs w) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= T_flat) return;
  bool bad;
  const int64_t pos = ask_pos(p, T_flat, scored, w, f2t, T_tree, bad);
  if (pos < 0) return;
  const int slot = w.start[pos] + atomicAdd(&w.fill[pos], 1);
  w.lab[slot] = flat[p + 1];
  w.src[slot] = (int32_t)p;
}

// One thread per tree position: insertion sort of its bucket by label, then its distinct-label count.
__global__ __launch_bounds__(256) void pairs_sort_kernel(int64_t T_tree, PairsWs w) {
  const int64_t pos = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (pos >= T_tree) return;
  const int s = w.start[pos], k = w.cnt[pos];
  int64_t *lab = w.lab + s;
  int32_t *src = w.src + s;
  for (int j = 1; j < k; ++j) {
    const int64_t l = lab[j];
    const int32_t q = src[j];
    int i = j - 1;
    while (i >= 0 && lab[i] > l) {
      lab[i + 1] = lab[i];
      src[i + 1] = src[i];
      --i;
    }
    lab[i + 1] = l;
    src[i + 1] = q;
  }
  int u = 0;
  for (int j = 0; j < k; ++j) u += (j == 0 || lab[j] != lab[j - 1]) ? 1 : 0;
  w.uniq[pos] = u;
}

// One thread per tree position: number its distinct labels from base[pos]; every ask of the bucket gets its
// label's pair.
__global__ __launch_bounds__(256) void pairs_emit_kernel(int64_t T_tree, PairsWs w, int64_t *pair_pos,
                                                         int64_t *pair_label, int64_t *flat_pair) {
  const int64_t pos = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (pos >= T_tree) return;
  const int s = w.start[pos], k = w.cnt[pos];
  int64_t pair = (int64_t)w.base[pos] - 1;
  for (int j = 0; j < k; ++j) {
    const int64_t l = w.lab[s + j];
    if (j == 0 || l != w.lab[s + j - 1]) {
      ++pair;
      pair_pos[pair] = pos;
      pair_label[pair] = l;
    }
    flat_pair[w.src[s + j]] = pair;
  }
}

// flat positions without an ask: -1, or the pair count
__global__ __launch_bounds__(256) void pairs_none_kernel(int64_t T_flat, const uint8_t *scored, const int64_t *f2t,
                                                         int64_t T_tree, PairsWs w, int none_as_count,
                                                         int64_t *flat_pair, int32_t *count) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (blockIdx.x == 0 && threadIdx.x == 0) count[0] = w.tot[1];
  if (p >= T_flat) return;
  bool bad;
  if (ask_pos(p, T_flat, scored, w, f2t, T_tree, bad) < 0) flat_pair[p] = none_as_count ? (int64_t)w.tot[1] : -1;
}

}  // namespace octo

using namespace octo;

extern "C" {

int octo_label_pairs_workspace_bytes(int64_t T_flat, int64_t T_tree, size_t *bytes) {
  OCTO_CHECK_ARG(bytes != nullptr, "label_pairs_workspace_bytes: null pointer");
  OCTO_CHECK_ARG(T_flat >= 0 && T_tree >= 0 && T_flat < 0x7fffffff && T_tree < 0x7fffffff,
                 "label_pairs: T_flat=%lld T_tree=%lld out of range", (long long)T_flat, (long long)T_tree);
  *bytes = pairs_ws_layout(T_flat, T_tree, nullptr, nullptr);
  return OCTO_OK;
}

int octo_label_pairs(const int64_t *flat, int64_t T_flat, const int64_t *cu, int64_t n_seq,
                     const int64_t *flat_to_tree, int64_t T_tree, const uint8_t *scored, int64_t *pair_pos,
                     int64_t *pair_label, int64_t *flat_pair, int32_t *count, int flags, void *ws, size_t ws_bytes,
                     void *stream) {
  OCTO_CHECK_ARG(T_flat >= 0 && T_tree >= 0 && n_seq >= 0 && T_flat < 0x7fffffff && T_tree < 0x7fffffff,
                 "label_pairs: T_flat=%lld T_tree=%lld n_seq=%lld out of range", (long long)T_flat,
                 (long long)T_tree, (long long)n_seq);
  OCTO_CHECK_ARG((flags & ~OCTO_PAIRS_NONE_AS_COUNT) == 0, "label_pairs: unknown flags %d", flags);
  OCTO_CHECK_ARG(count != nullptr, "label_pairs: null count");
  OCTO_CHECK_ARG(T_flat == 0 || (flat && flat_to_tree && pair_pos && pair_label && flat_pair),
                 "label_pairs: null pointer");
  OCTO_CHECK_ARG(n_seq == 0 || cu != nullptr, "label_pairs: null cu");
  PairsWs w;
  const size_t need = pairs_ws_layout(T_flat, T_tree, (char *)ws, &w);
  if (!ws || ws_bytes < need) return octo_fail(OCTO_EWORKSPACE, "label_pairs: workspace %zu < %zu bytes", ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int64_t big = T_flat > T_tree ? T_flat : T_tree;
  hipLaunchKernelGGL(pairs_init_kernel, dim3((unsigned)cdiv(big > 4 ? big : 4, 256)), dim3(256), 0, st, w, T_flat,
                     T_tree, count);
  if (T_flat == 0) return OCTO_OK;
  if (n_seq > 0)
    hipLaunchKernelGGL(pairs_ends_kernel, dim3((unsigned)cdiv(n_seq, 256)), dim3(256), 0, st, cu, n_seq, T_flat, w);
  const dim3 gf((unsigned)cdiv(T_flat, 256)), gt((unsigned)cdiv(T_tree > 0 ? T_tree : 1, 256));
  hipLaunchKernelGGL(pairs_count_kernel, gf, dim3(256), 0, st, T_flat, scored, flat_to_tree, T_tree, w, count);
  hipLaunchKernelGGL(scan_i32_kernel, dim3(1), dim3(1024), 0, st, w.cnt, T_tree, w.start, w.tot + 0);
  hipLaunchKernelGGL(pairs_fill_kernel, gf, dim3(256), 0, st, flat, T_flat, scored, flat_to_tree, T_tree, w);
  hipLaunchKernelGGL(pairs_sort_kernel, gt, dim3(256), 0, st, T_tree, w);
  hipLaunchKernelGGL(scan_i32_kernel, dim3(1), dim3(1024), 0, st, w.uniq, T_tree, w.base, w.tot + 1);
  hipLaunchKernelGGL(pairs_emit_kernel, gt, dim3(256), 0, st, T_tree, w, pair_pos, pair_label, flat_pair);
  hipLaunchKernelGGL(pairs_none_kernel, gf, dim3(256), 0, st, T_flat, scored, flat_to_tree, T_tree, w,
                     (flags & OCTO_PAIRS_NONE_AS_COUNT) ? 1 : 0, flat_pair, count);
  OCTO_CHECK_LAUNCH("label_pairs");
  return OCTO_OK;
}

}  // extern "C"
