// GEMM kernels of the LM-head path, each the MFMA mainloop of gemm_nt.h with a fused epilogue:
//
//   gemm_stats : S^T = W . H^T tile -> per (row, vocab tile) online softmax statistics (m, S, U)
//                (forward; octopus/rl/lm_head.py:102-112 without the [rows, V] logits)
//   gemm_dz    : the same tile recomputed -> dz = g (onehot - p) / T * post'(z) of one vocabulary chunk, written
//                token-major [tokens, chunk columns] in the 16-bit MFMA type (fp32 inputs: also chunk-major)
//                (backward recompute, lm_head.py:118-121 under checkpoint)
//   gemm_store : plain C = A . B^T with fp32/bf16/f16 output, optionally accumulated or with an fp32 addend:
//                grad_h = dz . W (dz read K-contiguous, W read K-major as stored), grad_W = dz^T . h (dz read
//                K-major by transposing LDS reads, h^T staged K-contiguous)
//
// Orientation: the first operand (MFMA "A", tile rows) of gemm_stats / gemm_dz is the vocabulary, the second (tile
// columns) the tokens. The 16-bit kernels run v_mfma_f32_16x16x32 on 8 waves of 128 x 64 (Acc16N<4>): a lane holds
// 32 vocabulary rows of each of its 4 token columns, so the softmax reductions over the vocabulary are in registers
// plus a 4-lane shuffle and one LDS exchange between the two waves of a token column.
// fp32 operands run v_mfma_f32_32x32x2 on 4 waves (Acc32).
#include <type_traits>

#include "gemm_nt.h"
#include "octo_internal.h"

namespace octo {

// ---- 16-bit staging tiles ------------------------------------------------------------------------

typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack2(float lo, float hi, bf16x2 *) {
  bf16x2 p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}
__device__ __forceinline__ uint32_t pack2(float lo, float hi, f16x2_t *) {
  f16x2_t p;
  p[0] = (_Float16)lo;
  p[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

// A 16-bit tile staged in LDS for a token-major store (dz, or the fused step's exponentials) (the ring, free after
// the mainloop): T[t] holds token t (tile column) over the tile's 256 vocabulary rows, as 64 slots of 8 bytes (4
// consecutive rows); logical slot s of token t sits at physical slot s ^ swz(t), the swizzle chosen for the
// accumulator layout so that both accesses are free of bank conflicts:
//   - the accumulator writes (Acc16N: a half-wave = 16 consecutive tokens x 2 adjacent slots, for 4 and 8 waves);
//   - the token-major read-back (16 lanes: one token, 16 consecutive 16-byte pairs).
template <class L> struct DzSwz;
template <int NJ> struct DzSwz<Acc16N<NJ>> {
  static __device__ __forceinline__ int at(int t) { return (((t & 15) << 1) | ((t >> 4) & 1)) ^ (((t >> 5) & 1) << 3); }
};

// ---- epilogue: online softmax statistics ----------------------------------------------------

// The softcap's tanh of every accumulator in place, acc = tanh(pre z), with z = acc times its vocabulary row's scale for
// fp8 weights (the tile's scales staged in LDS at wsl, 0 past V). Without the softcap nothing is done here: stats_cols
// applies an fp8 row scale as it reads each accumulator (the same fp32 product; an in-place multiply here made the
// compiler spill accumulators: 112-136 bytes per lane against 24).
template <class L, bool A_FP8, bool TANH>
__device__ __forceinline__ void pre_transform(typename L::V (&acc)[L::NI][L::NJ], int wm, int lane, float pre,
                                              const __attribute__((address_space(3))) f32x4 *wsl = nullptr) {
  static_assert(!A_FP8 || L::NV == 4, "fp8 weights run the 16 x 16 accumulator layout");
  if constexpr (TANH) {
#pragma unroll
    for (int i = 0; i < L::NI; ++i) {
      f32x4 q;
      if constexpr (A_FP8) q = wsl[L::row(wm, i, 0, lane) >> 2];
#pragma unroll
      for (int j = 0; j < L::NJ; ++j)
#pragma unroll
        for (int v = 0; v < L::NV; ++v) {
          float x = acc[i][j][v];
          if constexpr (A_FP8) x *= q[v & 3];
          acc[i][j][v] = ftanh(pre * x);
        }
    }
  }
}

typedef __attribute__((address_space(3))) f32x4 lds_f32x4;

// The per-token softmax statistics of this wave's rows of the tile: red[wm * 256 + column] = (m2, S, U), m2 the
// base-2 maximum, S and U the sums of e = exp2(t - m2) and e t (0 past V). EXM (16-bit, the fused step): each e,
// times the softcap's derivative 1 - x^2 when TANH (acc holds x = tanh(pre z) then), is also written into the LDS
// staging tile, laid out as dz_stage lays out dz (zero past V and for tokens at or past nvalid). EXM 1: as f16,
// relative to the wave's own maximum, which the tile's part keeps. EXM 2: as bf16, times exp2(min(m2 - xoff[token],
// kExClamp)) (and the fp8 row scale when A_FP8, from the tile's 256 scales staged in LDS at wsl), i.e. relative to
// the token's offset (StatsArgs::xoff; xoff here points at the tile's first token). fp8 weights without the softcap:
// acc holds the raw e4m3 products, and each is multiplied by its row's scale (wsl) as it is read.
template <class L, bool MASK, int EXM = 0, bool TANH = false, bool A_FP8 = false>
__device__ __forceinline__ void stats_cols(const typename L::V (&acc)[L::NI][L::NJ], int64_t m0, int wm, int wn,
                                           int lane, int64_t V, float c, lds_f32x4 *red, lds_char *tile = nullptr,
                                           int64_t nvalid = 0, const float *xoff = nullptr,
                                           const lds_f32x4 *wsl = nullptr) {
  constexpr bool SCALE = A_FP8 && !TANH;  // the fp8 row scale applied here (with TANH, pre_transform applied it)
#pragma unroll
  for (int j = 0; j < L::NJ; ++j) {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < L::NI; ++i) {
      f32x4 q;
      if constexpr (SCALE) q = wsl[L::row(wm, i, 0, lane) >> 2];
#pragma unroll
      for (int v = 0; v < L::NV; ++v) {
        const bool ok = !MASK || (m0 + L::row(wm, i, v, lane) < V);
        float x = acc[i][j][v];
        if constexpr (SCALE) x *= q[v & 3];
        if (ok) mx = fmaxf(mx, x);
      }
    }
    mx = L::col_max(mx);
    const float m2 = mx * c;
    const int tt = L::col(wn, j, lane);
    // EXM 2: the half tile's factor to the token's offset (fminf also takes kExClamp for m2 - xoff = NaN, which needs
    // xoff = -inf and m2 = -inf: no element of the half lies below V, each e is 0)
    float f = 1.f;
    if constexpr (EXM == 2) f = tt < nvalid ? fexp2(fminf(m2 - xoff[tt], kExClamp)) : 0.f;
    float S = 0.f, U = 0.f;
#pragma unroll
    for (int i = 0; i < L::NI; ++i)
#pragma unroll
      for (int g4 = 0; g4 < L::NV / 4; ++g4) {
        f32x4 q;  // fp8 weights: the scales of this lane's 4 vocab rows (LDS, 0 past V)
        if constexpr (A_FP8) q = wsl[L::row(wm, i, 4 * g4, lane) >> 2];
        float x4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int v = 4 * g4 + u;
          float xs = acc[i][j][v];
          if constexpr (SCALE) xs *= q[u];
          const float t = __builtin_fmaf(xs, c, -m2);
          float e = fexp2(t);
          if (MASK) {
            const bool ok = m0 + L::row(wm, i, v, lane) < V;
            e = ok ? e : 0.f;
          }
          S += e;
          U = __builtin_fmaf(e, t, U);
          if constexpr (EXM != 0) {
            const float x = acc[i][j][v];
            const float ev = TANH ? e * (1.f - x * x) : e;
            x4[u] = EXM == 2 ? ev * f : (tt < nvalid ? ev : 0.f);
          }
        }
        if constexpr (EXM != 0) {
          const int rl = L::row(wm, i, 4 * g4, lane);  // first of this lane's 4 vocab rows in the tile
          if constexpr (EXM == 2 && A_FP8) {  // d/d(raw e4m3 product): times the rows' scales
#pragma unroll
            for (int u = 0; u < 4; ++u) x4[u] *= q[u];
          }
          i32x2 pk;
          if constexpr (EXM == 2) {
            pk[0] = (int)pack2(x4[0], x4[1], (bf16x2 *)nullptr);
            pk[1] = (int)pack2(x4[2], x4[3], (bf16x2 *)nullptr);
          } else {
            pk[0] = (int)pack2(x4[0], x4[1], (f16x2_t *)nullptr);
            pk[1] = (int)pack2(x4[2], x4[3], (f16x2_t *)nullptr);
          }
          *(lds_i32x2 *)(tile + tt * 512 + (((rl >> 2) ^ DzSwz<L>::at(tt)) << 3)) = pk;
        }
      }
    S = L::col_sum(S);
    U = L::col_sum(U);
    if (L::col_lane(lane)) {
      f32x4 o;
      o[0] = m2; o[1] = S; o[2] = U; o[3] = 0.f;
      red[wm * 256 + tt] = o;
    }
  }
}

// fp32 forward statistics (4-stage loop, 32 x 32 MFMAs); 16-bit operands run gemm_stats8_kernel.
template <int DT, bool A_FP8, bool TANH>
__global__ __launch_bounds__(NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_stats_kernel(Operand A, Operand B, GemmShape s, StatsArgs e) {
  static_assert(!ring5_ok(DT) && !A_FP8, "16-bit operands run gemm_stats8_kernel");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_BYTES];
  lds_char *smem = (lds_char *)smem_;
  int mt, nt;
  if (!tile_of(s, mt, nt)) return;
  const int64_t m0 = (int64_t)mt * TM, n0 = (int64_t)nt * TN;
  const int64_t nvalid = min(dev_count(s.count, s.count_off + n0, s.N - n0), (int64_t)TN);  // this tile's tokens
  if (nvalid <= 0) return;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
  lds_f32x4 *red = (lds_f32x4 *)smem;
  f32x16 acc[4][4];
  mainloop_dma<DT, OpRows, OpRows>(A, B, m0, n0, s.K, smem, acc);
  const int64_t ma = e.v0 + m0;  // first vocabulary row of the tile
  pre_transform<Acc32, false, TANH>(acc, wm, lane, e.pre);
  if (ma + TM > e.V) stats_cols<Acc32, true>(acc, ma, wm, wn, lane, e.V, e.c, red);
  else stats_cols<Acc32, false>(acc, ma, wm, wn, lane, e.V, e.c, red);
  __syncthreads();
  const int t = threadIdx.x;
  if (t < nvalid) {
    const f32x4 a = red[t], b = red[256 + t];
    Stat3 sa{a[0], a[1], a[2]}, sb{b[0], b[1], b[2]};
    Stat3 r = stat_merge(sa, sb);
    f32x4 o;
    o[0] = a[0]; o[1] = r.S; o[2] = r.U; o[3] = b[0];
    e.part[(n0 + t) * e.mtiles + e.v0 / TM + mt] = o;
  }
}

// ---- epilogue: dz recompute ------------------------------------------------------------------
//
// dz = g (onehot - p) / T x post'(z) of the 256 (vocab) x 256 (token) tile. 16-bit types write it token-major
// only (dzA [token][vocab]: grad_h reads it K-contiguous, grad_W K-major), through one LDS staging tile as whole
// 512-byte rows (dz_stage / dz_write below). fp32 is computed in place in the accumulators and stored directly in
// both layouts (dzB [vocab][token] for grad_W's K-contiguous fp32 loop).

// Stream a 256 x 512-byte LDS tile (rows stored with slot swizzle `s(row)` on 8-byte slots) to global
// rows dst + row * ld_bytes, 16 bytes per thread per row-eighth. Non-temporal stores: dz is read back only by the
// next kernels, after 7.5 GB more of it at 24,576 rows. Same box, 24,576 rows, d 2560, V 151,936: gemm_dz 14.9
// against 15.2 ms, grad_h 0.13 ms slower, the fused fwd+bwd step 0.15 ms faster.
template <int NT = NTHREADS, typename SWZ>
__device__ __forceinline__ void lds_tile_to_global(const lds_char *tile, char *dst, int64_t ld_bytes, SWZ swz) {
  constexpr int RPP = NT / 32;  // rows per pass
  const int t = threadIdx.x;
  const int c16 = t & 31;
#pragma unroll 4
  for (int p = 0; p < 256 / RPP; ++p) {
    const int row = p * RPP + (t >> 5);
    const int s = swz(row);
    // logical slots 2c, 2c+1 sit at physical (2c ^ s, (2c+1) ^ s): one aligned 16-byte pair, its halves
    // swapped when s is odd
    i32x4 v = *(const lds_i32x4 *)(tile + row * 512 + ((2 * c16) ^ (s & ~1)) * 8);
    if (s & 1) v = __builtin_shufflevector(v, v, 2, 3, 0, 1);
    __builtin_nontemporal_store(v, (i32x4 *)(dst + row * ld_bytes + c16 * 16));
  }
}

// dz = g (onehot - p) / T * post'(z) of every tile element, in place (fp32), zero outside V and the
// pass's valid tokens. The one-hot test compares the label, relative to this lane's first vocab row,
// with each register's compile-time row offset.
template <bool A_FP8, bool TANH>
__device__ __forceinline__ void dz_in_place(f32x16 (&acc)[4][4], const DzArgs &e, int64_t m0, int64_t n0,
                                            int64_t nvalid, int wm, int wn, int lane) {
  const int64_t lane_row0 = m0 + wm * 128 + 4 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = acc_col(wn, j, lane);
    const bool tok_ok = col < nvalid;
    const int64_t r = e.row_off + n0 + col;  // compact row
    float m2 = 0.f, l2s = 0.f, gs = 0.f;
    int yrel = -1;
    if (tok_ok) {
      row_state(e.lse, e.lse_pair, r, m2, l2s);
      gs = e.g[r] * e.gmul;
      const int64_t y = e.labels[e.label_idx ? e.label_idx[r] : r] - lane_row0;
      yrel = (y >= 0 && y < 256) ? (int)y : -1;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int roff = i * 32 + 8 * (v >> 2) + (v & 3);
        const float hit = (yrel == roff) ? gs : 0.f;
        const float x = acc[i][j][v];
        if constexpr (TANH) {
          const float th = ftanh(e.pre * x);
          const float p = fexp2(__builtin_fmaf(th, e.c, -m2) - l2s);
          acc[i][j][v] = __builtin_fmaf(-gs, p, hit) * (1.f - th * th);
        } else {
          const float p = fexp2(__builtin_fmaf(x, e.c, -m2) - l2s);
          acc[i][j][v] = __builtin_fmaf(-gs, p, hit);
        }
      }
  }
  if constexpr (A_FP8) {  // d/d(raw e4m3 product) = dz * row scale
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = lane_row0 + i * 32 + 8 * (v >> 2) + (v & 3);
        const float sc = row < e.V ? e.wscale[row] : 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j][v] *= sc;
      }
  }
  if (m0 + TM > e.V || nvalid < TN) {  // edge tile: zero rows past V and tokens past the pass's count
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool tok_ok = acc_col(wn, j, lane) < nvalid;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const bool ok = tok_ok && (lane_row0 + i * 32 + 8 * (v >> 2) + (v & 3) < e.V);
          acc[i][j][v] = ok ? acc[i][j][v] : 0.f;
        }
    }
  }
}

// fp32 dz (fp32 inputs): direct 16-byte stores to dzA, 4-byte stores to dzB.
__device__ __forceinline__ void dz_store_direct(const f32x16 (&acc)[4][4], const DzArgs &e, int64_t m0, int64_t n0,
                                                int wm, int wn, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t tk = n0 + acc_col(wn, j, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int64_t row0 = m0 + acc_row(wm, i, 4 * g4, lane);
        if (e.dzA) {
          f32x4 pk;
#pragma unroll
          for (int u = 0; u < 4; ++u) pk[u] = acc[i][j][4 * g4 + u];
          *(f32x4 *)((float *)e.dzA + tk * e.ldA + row0) = pk;
        }
        if (e.dzB) {
#pragma unroll
          for (int u = 0; u < 4; ++u) ((float *)e.dzB)[(row0 + u) * e.ldB + tk] = acc[i][j][4 * g4 + u];
        }
      }
  }
}

// (dz_stage below: the dense pass writes -g p / T x post' (x fp8 row scale) everywhere; after a barrier one thread per
// token writes the label entry (launch_hit's value) over it, so no element is compared against the label.)

typedef __attribute__((address_space(3))) short lds_short;

// fp8 weights: the accumulators are raw e4m3 products; z = acc x the row's scale (the forward's pre_transform, the same
// fp32 multiply, so the row state still matches), and d/d(raw product) = dz x that scale. A lane's 4 consecutive rows'
// scales are loaded once per (i, g4) and serve all its token columns (loaded per column, and once more to scale the
// accumulators: same box, 65,536-row passes of 114,688 rows, d 2560, V 151,936, gemm_dz 35.5-35.8 against 35.1-35.5 ms).
template <class L, typename P2, bool TANH, bool EDGE>
__device__ __forceinline__ void dz_stage_fp8(const typename L::V (&acc)[L::NI][L::NJ], const DzArgs &e, int64_t m0,
                                             int64_t n0, int64_t nvalid, int wm, int wn, int lane, lds_char *tile) {
  float m2[L::NJ], l2s[L::NJ], ngs[L::NJ];
  int tt[L::NJ], sw[L::NJ];
#pragma unroll
  for (int j = 0; j < L::NJ; ++j) {
    tt[j] = L::col(wn, j, lane);
    m2[j] = 0.f;
    l2s[j] = 0.f;
    ngs[j] = 0.f;  // -g / T (0 for tokens past the pass's count: dz 0, also in K-padding)
    if (tt[j] < nvalid) {
      const int64_t r = e.row_off + n0 + tt[j];
      row_state(e.lse, e.lse_pair, r, m2[j], l2s[j]);
      ngs[j] = -(e.g[r] * e.gmul);
    }
    sw[j] = DzSwz<L>::at(tt[j]);
  }
#pragma unroll
  for (int i = 0; i < L::NI; ++i)
#pragma unroll
    for (int g4 = 0; g4 < L::NV / 4; ++g4) {
      const int rl = L::row(wm, i, 4 * g4, lane);  // first of this lane's 4 vocab rows in the tile
      const int64_t row = m0 + rl;
      float sc[4];
      if (row + 3 < e.V) {
        const f32x4 q = *(const f32x4 *)(e.wscale + row);
#pragma unroll
        for (int u = 0; u < 4; ++u) sc[u] = q[u];
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) sc[u] = (row + u < e.V) ? e.wscale[row + u] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < L::NJ; ++j) {
        float d[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float x = acc[i][j][4 * g4 + u] * sc[u];
          if constexpr (TANH) {
            const float th = ftanh(e.pre * x);
            d[u] = ngs[j] * fexp2(__builtin_fmaf(th, e.c, -m2[j]) - l2s[j]) * (1.f - th * th) * sc[u];
          } else {
            d[u] = ngs[j] * fexp2(__builtin_fmaf(x, e.c, -m2[j]) - l2s[j]) * sc[u];
          }
          if constexpr (EDGE) d[u] = (row + u < e.V) ? d[u] : 0.f;
        }
        i32x2 pk;
        pk[0] = (int)pack2(d[0], d[1], (P2 *)nullptr);
        pk[1] = (int)pack2(d[2], d[3], (P2 *)nullptr);
        *(lds_i32x2 *)(tile + tt[j] * 512 + (((rl >> 2) ^ sw[j]) << 3)) = pk;
      }
    }
}

template <class L, typename P2, bool TANH, bool EDGE>
__device__ __forceinline__ void dz_stage(const typename L::V (&acc)[L::NI][L::NJ], const DzArgs &e, int64_t m0,
                                         int64_t n0, int64_t nvalid, int wm, int wn, int lane, lds_char *tile) {
#pragma unroll
  for (int j = 0; j < L::NJ; ++j) {
    const int tt = L::col(wn, j, lane);
    float m2 = 0.f, l2s = 0.f, ngs = 0.f;  // -g / T (0 for tokens past the pass's count: dz 0, also in K-padding)
    if (tt < nvalid) {
      const int64_t r = e.row_off + n0 + tt;
      row_state(e.lse, e.lse_pair, r, m2, l2s);
      ngs = -(e.g[r] * e.gmul);
    }
    const int sw = DzSwz<L>::at(tt);
#pragma unroll
    for (int i = 0; i < L::NI; ++i)
#pragma unroll
      for (int g4 = 0; g4 < L::NV / 4; ++g4) {
        const int rl = L::row(wm, i, 4 * g4, lane);  // first of this lane's 4 vocab rows in the tile
        float d[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float x = acc[i][j][4 * g4 + u];
          if constexpr (TANH) {
            const float th = ftanh(e.pre * x);
            d[u] = ngs * fexp2(__builtin_fmaf(th, e.c, -m2) - l2s) * (1.f - th * th);
          } else {
            d[u] = ngs * fexp2(__builtin_fmaf(x, e.c, -m2) - l2s);
          }
          if constexpr (EDGE) d[u] = (m0 + rl + u < e.V) ? d[u] : 0.f;
        }
        i32x2 pk;
        pk[0] = (int)pack2(d[0], d[1], (P2 *)nullptr);
        pk[1] = (int)pack2(d[2], d[3], (P2 *)nullptr);
        *(lds_i32x2 *)(tile + tt * 512 + (((rl >> 2) ^ sw) << 3)) = pk;
      }
  }
}

// ma: the tile's first vocabulary row; m0: its first dz column (ma - v0)
template <class L, typename P2, int NT = NTHREADS>
__device__ __forceinline__ void dz_write(const DzArgs &e, int64_t ma, int64_t m0, int64_t n0, int64_t nvalid,
                                         lds_char *tile) {
  typedef typename std::conditional<std::is_same<P2, bf16x2>::value, __bf16, _Float16>::type ET;
  const int t = threadIdx.x;
  // the label entry of token t (column t of the tile), loaded before the barrier that ends the dense pass
  int yl = -1;
  float hv = 0.f;
  if (t < nvalid) {
    const int64_t r = e.row_off + n0 + t;
    const int64_t y = e.labels[e.label_idx ? e.label_idx[r] : r] - ma;
    if (y >= 0 && y < TM && ma + y < e.V) {
      yl = (int)y;
      hv = e.hit[n0 + t];
    }
  }
  __syncthreads();  // dense pass written
  if (yl >= 0) {
    const ET v = (ET)hv;
    *(lds_short *)(tile + t * 512 + (((yl >> 2) ^ DzSwz<L>::at(t)) << 3) + (yl & 3) * 2) = __builtin_bit_cast(short, v);
  }
  __syncthreads();
  if (e.dzA)  // [token][vocab]: 512-byte rows
    lds_tile_to_global<NT>(tile, (char *)e.dzA + (n0 * e.ldA + m0) * 2, e.ldA * 2, [](int row) { return DzSwz<L>::at(row); });
}

// fp32 dz (4-stage loop, 32 x 32 MFMAs, both layouts stored directly); 16-bit operands run gemm_dz8_kernel.
template <int DT, bool A_FP8, bool TANH>
__global__ __launch_bounds__(NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_dz_kernel(Operand A, Operand B, GemmShape s, DzArgs e) {
  static_assert(!ring5_ok(DT) && !A_FP8, "16-bit operands run gemm_dz8_kernel");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_BYTES];
  lds_char *smem = (lds_char *)smem_;
  int mt, nt;
  if (!tile_of(s, mt, nt)) return;
  const int64_t m0 = (int64_t)mt * TM, n0 = (int64_t)nt * TN;
  const int64_t nvalid = min(dev_count(s.count, s.count_off + n0, s.N - n0), (int64_t)TN);  // this tile's tokens
  if (nvalid <= 0) return;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
  f32x16 acc[4][4];
  mainloop_dma<DT, OpRows, OpRows>(A, B, m0, n0, s.K, smem, acc);
  dz_in_place<false, TANH>(acc, e, e.v0 + m0, n0, nvalid, wm, wn, lane);  // vocabulary rows from v0 + m0
  dz_store_direct(acc, e, m0, n0, wm, wn, lane);                            // dz columns from m0
}

// ---- epilogue: plain store -------------------------------------------------------------------

#ifndef OCTO_PART_ATOMIC
#define OCTO_PART_ATOMIC 1
#endif
// C = rs[row] x acc (rs NULL: acc) (+ addend, fp32, row stride ld_add) (+ C when ACC), rounded once to OT. An fp32 C += acc is one no-return
// atomic add per element, performed in the L2, so the tile's epilogue does not wait for C to be read (grad_W's fp32
// partials of the fused step at 24,576 rows, d 2560, V 151,936: the gradient launches 28.35 against 28.65 ms per
// step, same box). A launch adds to each element once (one tile), so the sums keep launch order and are
// reproducible.
template <class L, typename OT, bool ACC, bool ADD, bool EDGE>
__device__ __forceinline__ void store_tile(const typename L::V (&acc)[L::NI][L::NJ], OT *C, const float *addend,
                                           int64_t ldc, int64_t ld_add, int64_t m0, int64_t n0, int64_t mvalid,
                                           int64_t nvalid, int wm, int wn, int lane, const float *rs) {
#pragma unroll
  for (int i = 0; i < L::NI; ++i)
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int rr = L::row(wm, i, v, lane);
      if (EDGE && rr >= mvalid) continue;
      OT *crow = C + (m0 + rr) * ldc + n0;
      const float *arow = ADD ? addend + (m0 + rr) * ld_add + n0 : nullptr;
      const float sc = rs ? rs[m0 + rr] : 1.f;
#pragma unroll
      for (int j = 0; j < L::NJ; ++j) {
        const int cc = L::col(wn, j, lane);
        if (EDGE && cc >= nvalid) continue;
        float x = acc[i][j][v] * sc;
        if (ADD) x += arow[cc];
        if constexpr (OCTO_PART_ATOMIC && ACC && std::is_same<OT, float>::value) {
          __hip_atomic_fetch_add(crow + cc, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          continue;
        }
        if (ACC) x += (float)crow[cc];
        crow[cc] = (OT)x;
      }
    }
}

template <class L, typename OT, bool ACC, bool ADD>
__device__ __forceinline__ void store_edge(const typename L::V (&acc)[L::NI][L::NJ], OT *C, const float *addend,
                                           int64_t ldc, int64_t ld_add, int64_t m0, int64_t n0, int64_t mvalid,
                                           int64_t nvalid, int wm, int wn, int lane, const float *rs) {
  if (mvalid < TM || nvalid < TN)
    store_tile<L, OT, ACC, ADD, true>(acc, C, addend, ldc, ld_add, m0, n0, mvalid, nvalid, wm, wn, lane, rs);
  else store_tile<L, OT, ACC, ADD, false>(acc, C, addend, ldc, ld_add, m0, n0, mvalid, nvalid, wm, wn, lane, rs);
}

template <class L, typename OT>
__device__ __forceinline__ void store_any(const typename L::V (&acc)[L::NI][L::NJ], const StoreArgs &e, int64_t m0,
                                          int64_t n0, int64_t mvalid, int64_t nvalid) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = L::wm(w), wn = L::wn(w);
  OT *c = (OT *)e.C;
  const float *rs = e.row_scale;
  if (e.accumulate) {
    if (e.addend) store_edge<L, OT, true, true>(acc, c, e.addend, e.ldc, e.ld_add, m0, n0, mvalid, nvalid, wm, wn, lane, rs);
    else store_edge<L, OT, true, false>(acc, c, e.addend, e.ldc, e.ld_add, m0, n0, mvalid, nvalid, wm, wn, lane, rs);
  } else {
    if (e.addend) store_edge<L, OT, false, true>(acc, c, e.addend, e.ldc, e.ld_add, m0, n0, mvalid, nvalid, wm, wn, lane, rs);
    else store_edge<L, OT, false, false>(acc, c, e.addend, e.ldc, e.ld_add, m0, n0, mvalid, nvalid, wm, wn, lane, rs);
  }
}

// True when a tile with no K to contract (a device count of 0 rows) would only add zeros to what C or the partials
// already hold: it can end before its mainloop. A store that overwrites, or adds an addend, still runs.
__device__ __forceinline__ bool adds_nothing(const StoreArgs &e, int which, int64_t K_eff) {
  if (K_eff > 0) return false;
  return which == 1 ? (e.accumulate && !e.addend) : (which == 2 && e.part_accumulate);
}

// Which store a row pass's GEMM makes (StoreArgs pass_count / part): 0 none, 1 the final C, 2 the fp32 partials.
__device__ __forceinline__ int pass_store(const StoreArgs &e) {
  if (!e.pass_count) return 1;
  const int64_t c = *e.pass_count;
  if (e.pass_r0 > 0 && c <= e.pass_r0) return 0;
  return (e.part && c > e.pass_end) ? 2 : 1;
}

// The tile's fp32 partials in the blocked layout (StoreArgs::part_blocked): this wave's 8192 values, element v of
// block (i, j) of lane l at ((i NJ + j) NV + v) 64 + l, stored or added (no-return atomics).
template <class L>
__device__ __forceinline__ float *blocked_part(float *base, int64_t ldc, int64_t m0, int64_t n0) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  return base + ((m0 / TM) * (ldc / TN) + n0 / TN) * (int64_t)(TM * TN) + w * (L::NI * L::NJ * L::NV * 64) + lane;
}

template <class L>
__device__ __forceinline__ void store_blocked(const typename L::V (&acc)[L::NI][L::NJ], const StoreArgs &e,
                                              int64_t m0, int64_t n0) {
  float *b = blocked_part<L>(e.part, e.ldc, m0, n0);
#pragma unroll
  for (int i = 0; i < L::NI; ++i)
#pragma unroll
    for (int j = 0; j < L::NJ; ++j)
#pragma unroll
      for (int v = 0; v < L::NV; ++v) {
        float *q = b + ((i * L::NJ + j) * L::NV + v) * 64;
        if (e.part_accumulate) __hip_atomic_fetch_add(q, acc[i][j][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else *q = acc[i][j][v];
      }
}

// acc += the blocked partials of the earlier passes (the pass that stores C).
template <class L>
__device__ __forceinline__ void add_blocked(typename L::V (&acc)[L::NI][L::NJ], const float *addend, int64_t ldc,
                                            int64_t m0, int64_t n0) {
  const float *b = blocked_part<L>((float *)addend, ldc, m0, n0);
#pragma unroll
  for (int i = 0; i < L::NI; ++i)
#pragma unroll
    for (int j = 0; j < L::NJ; ++j)
#pragma unroll
      for (int v = 0; v < L::NV; ++v) acc[i][j][v] += b[((i * L::NJ + j) * L::NV + v) * 64];
}

template <class L, typename OT>
__device__ __forceinline__ void store_pass(const typename L::V (&acc)[L::NI][L::NJ], const StoreArgs &e, int which,
                                           int64_t m0, int64_t n0, int64_t mvalid, int64_t nvalid) {
  if (which == 1) {
    store_any<L, OT>(acc, e, m0, n0, mvalid, nvalid);
  } else if (e.part_blocked) {
    store_blocked<L>(acc, e, m0, n0);
  } else {
    StoreArgs p = e;
    p.C = e.part;
    p.addend = nullptr;
    p.accumulate = e.part_accumulate;
    p.row_scale = nullptr;
    store_any<L, float>(acc, p, m0, n0, mvalid, nvalid);
  }
}

// The fp32 GEMMs' store: C = rs[row] x acc (+ addend) (+ C when accumulate), one loop with the run-time choices
// inside it. Separate loops per choice (store_any) made the compiler move all 256 accumulators out of the AGPRs into
// VGPRs ahead of the branches: 376 bytes of spills per lane, against none here. fp32 operands store no partials (their
// sums across passes accumulate into the fp32 output), so `which` is 1 here.
template <class L, typename OT>
__device__ __forceinline__ void store_rt(const typename L::V (&acc)[L::NI][L::NJ], const StoreArgs &e, int64_t m0,
                                         int64_t n0, int64_t mvalid, int64_t nvalid) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = L::wm(w), wn = L::wn(w);
  OT *C = (OT *)e.C;
  const bool acc_c = e.accumulate != 0, add = e.addend != nullptr;
  const bool atomic = OCTO_PART_ATOMIC && acc_c && std::is_same<OT, float>::value;
#pragma unroll
  for (int i = 0; i < L::NI; ++i)
#pragma unroll
    for (int v = 0; v < L::NV; ++v) {
      const int rr = L::row(wm, i, v, lane);
      if (rr >= mvalid) continue;
      OT *crow = C + (m0 + rr) * e.ldc + n0;
      const float *arow = add ? e.addend + (m0 + rr) * e.ld_add + n0 : nullptr;
      const float sc = e.row_scale ? e.row_scale[m0 + rr] : 1.f;
#pragma unroll
      for (int j = 0; j < L::NJ; ++j) {
        const int cc = L::col(wn, j, lane);
        if (cc >= nvalid) continue;
        float x = acc[i][j][v] * sc;
        if (add) x += arow[cc];
        if (atomic) {
          __hip_atomic_fetch_add((float *)crow + cc, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else {
          if (acc_c) x += (float)crow[cc];
          crow[cc] = (OT)x;
        }
      }
    }
}

// fp32 gradient GEMMs (4-stage loop, 32 x 32 MFMAs).
template <int DT, int OT>
__global__ __launch_bounds__(NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_store_kernel(Operand A, Operand B, GemmShape s, StoreArgs e) {
  static_assert(!ring5_ok(DT), "16-bit operands run gemm_store8_kernel");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_BYTES];
  lds_char *smem = (lds_char *)smem_;
  int mt, nt;
  if (!tile_of(s, mt, nt)) return;
  const int which = pass_store(e);
  if (which == 0) return;
  const int64_t m0 = (int64_t)mt * TM, n0 = (int64_t)nt * TN;
  int64_t mvalid = s.M - m0, nvalid = s.N - n0, K_eff = s.K;
  if (s.count_on == 1) mvalid = dev_count(s.count, s.count_off + m0, mvalid);
  if (s.count_on == 3) K_eff = round_up(dev_count(s.count, s.count_off, s.K), 64);
  if (mvalid <= 0 || nvalid <= 0 || adds_nothing(e, which, K_eff)) return;
  f32x16 acc[4][4];
  mainloop_dma<DT, OpRows, OpRows>(A, B, m0, n0, K_eff, smem, acc);
  store_rt<Acc32, typename Elem<OT>::T>(acc, e, m0, n0, mvalid, nvalid);
}

// The 16-bit gradient GEMMs' 8-wave form: 512 threads, two waves per SIMD, each 128 x 64 of the tile; the second
// wave on each SIMD issues MFMAs while one waits. KM selects the operand layouts: KM_A, grad_W (dz read K-major by
// transposing LDS reads), keeps one barrier per stage; KM_NONE (both K-contiguous) and KM_B, grad_h (W read K-major
// as stored, so no W^T is staged), wait for the next stage half-way through the K-step (SPLIT). Same box, 24,576
// rows, d 2560, V 151,936: grad_W 13.6 against 14.1 ms and grad_h 13.9 against 14.4 ms for the 4-wave form; grad_h
// reading W K-major without SPLIT 15.0 against 14.15 ms.
// One tile (mt, nt) of the 8-wave gradient GEMM; OT < 0: the output type is e.dtype, chosen after the mainloop.
template <int DT, int OT, int KM>
__device__ __forceinline__ void store8_tile(const Operand &A, const Operand &B, const GemmShape &s, const StoreArgs &e,
                                            int mt, int nt, int which, lds_char *smem) {
  const int64_t m0 = (int64_t)mt * TM, n0 = (int64_t)nt * TN;
  int64_t mvalid = s.M - m0, nvalid = s.N - n0, K_eff = s.K;
  if (s.count_on == 1) mvalid = dev_count(s.count, s.count_off + m0, mvalid);
  if (s.count_on == 3) K_eff = round_up(dev_count(s.count, s.count_off, s.K), 64);
  if (mvalid <= 0 || nvalid <= 0 || adds_nothing(e, which, K_eff)) return;
  f32x4 acc[8][4];
  if constexpr (KM == KM_A) mainloop_ring5<DT, OpColsN<8, 128>, OpRowsN<8, 64>>(A, B, m0, n0, K_eff, smem, acc);
  else if constexpr (KM == KM_B) mainloop_ring5<DT, OpRowsN<8, 128>, OpColsN<8, 64>, true>(A, B, m0, n0, K_eff, smem, acc);
  else mainloop_ring5<DT, OpRowsN<8, 128>, OpRowsN<8, 64>, true>(A, B, m0, n0, K_eff, smem, acc);
  StoreArgs eb = e;
  if (e.part_blocked && which == 1 && e.addend) {  // the blocked partials added here, C stored as usual
    add_blocked<Acc16N<4>>(acc, e.addend, e.ldc, m0, n0);
    eb.addend = nullptr;
  }
  if constexpr (OT >= 0) {
    store_pass<Acc16N<4>, typename Elem<OT>::T>(acc, eb, which, m0, n0, mvalid, nvalid);
  } else {
    switch (eb.dtype) {
      case OCTO_BF16: store_pass<Acc16N<4>, __bf16>(acc, eb, which, m0, n0, mvalid, nvalid); break;
      case OCTO_F16: store_pass<Acc16N<4>, _Float16>(acc, eb, which, m0, n0, mvalid, nvalid); break;
      default: store_pass<Acc16N<4>, float>(acc, eb, which, m0, n0, mvalid, nvalid); break;
    }
  }
}

template <int DT, int OT, int KM>
__global__ __launch_bounds__(2 * NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_store8_kernel(Operand A, Operand B, GemmShape s, StoreArgs e) {
  static_assert(ring5_ok(DT), "16-bit operands");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_RING5];
  lds_char *smem = (lds_char *)smem_;
  int mt, nt;
  if (!tile_of(s, mt, nt)) return;
  const int which = pass_store(e);
  if (which == 0) return;
  store8_tile<DT, OT, KM>(A, B, s, e, mt, nt, which, smem);
}

// Both gradient GEMMs of one row pass in one launch (the fused step): blocks [0, nh) run grad_h = dz . W (nh = its
// tile grid, a multiple of 8, so block b still runs on XCD b % 8 in either part), the rest grad_W = dz^T . h. The
// grad_h tiles, K = V long, are dispatched first; grad_W's, K = the pass's rows, fill the CUs its grid leaves idle
// and the rest of its last round (a pass of 6,656 rows at d 2560 has 260 grad_h tiles: alone, a second round for 4
// of them). KMH: grad_h reads W K-major as stored (KM_B) or a staged W^T (KM_NONE); grad_W reads dz K-major.
template <int DT, int KMH>
__global__ __launch_bounds__(2 * NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_grads8_kernel(Operand Ah, Operand Bh, GemmShape sh, StoreArgs eh, Operand Aw, Operand Bw, GemmShape sw, StoreArgs ew, unsigned nh) {
  static_assert(ring5_ok(DT), "16-bit operands");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_RING5];
  lds_char *smem = (lds_char *)smem_;
  const unsigned b = blockIdx.x;
  int64_t mtiles, ntiles;
  int mt, nt;
  if (b < nh) {
    bounded_tiles(sh, mtiles, ntiles);
    if (!tile_at(sh, (int)(b & 7), (int64_t)(b >> 3), mtiles, ntiles, mt, nt)) return;
    store8_tile<DT, -1, KMH>(Ah, Bh, sh, eh, mt, nt, 1, smem);
  } else {
    const unsigned c = b - nh;
    bounded_tiles(sw, mtiles, ntiles);
    if (!tile_at(sw, (int)(c & 7), (int64_t)(c >> 3), mtiles, ntiles, mt, nt)) return;
    const int which = pass_store(ew);
    if (which == 0) return;
    store8_tile<DT, -1, KM_A>(Aw, Bw, sw, ew, mt, nt, which, smem);
  }
}

// The logits-shaped GEMMs on the 8-wave loop (16-bit operands): 512 threads, two waves per SIMD, each 128 x 64, with
// the split stage barrier. Same box, 24,576 rows, d 2560, V 151,936 (against the 4-wave loop): gemm_stats 14.3
// against 15.1 ms, gemm_dz 15.3 against 16.5 ms; without the split barrier gemm_dz was 0.4 ms slower than the 4-wave
// loop.
// EX: also store the exponentials (StatsArgs::ex) through the LDS staging tile, as gemm_dz8 stores dz; the per-wave
// statistics then sit past that tile. EX 1: f16 relative to each half tile's maximum; EX 2: bf16 relative to each
// token's offset (StatsArgs::xoff).
template <int DT, bool A_FP8, bool TANH, int EX>
__global__ __launch_bounds__(2 * NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_stats8_kernel(Operand A, Operand B, GemmShape s, StatsArgs e) {
  static_assert(ring5_ok(DT), "16-bit operands");
  static_assert(256 * 512 + 512 * 16 + 256 * 4 <= SMEM_RING5, "staging tile, statistics and scales fit the LDS");
  typedef Acc16N<4> L;
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_RING5];
  lds_char *smem = (lds_char *)smem_;
  int mt, nt;
  if (!tile_of(s, mt, nt)) return;
  const int64_t m0 = (int64_t)mt * TM, n0 = (int64_t)nt * TN;
  const int64_t nvalid = min(dev_count(s.count, s.count_off + n0, s.N - n0), (int64_t)TN);  // this tile's tokens
  if (nvalid <= 0) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = L::wm(w), wn = L::wn(w);
  lds_f32x4 *red = (lds_f32x4 *)(smem + (EX ? 256 * 512 : 0));
  f32x4 acc[8][4];
  mainloop_ring5<DT, OpRowsN<8, 128>, OpRowsN<8, 64>, true>(A, B, m0, n0, s.K, smem, acc);
  const int64_t ma = e.v0 + m0;  // first vocabulary row of the tile
  lds_f32x4 *wsl = (lds_f32x4 *)(smem + 256 * 512 + 512 * 16);
  if constexpr (A_FP8) {  // the tile's row scales, read once (the ring is free now)
    if (threadIdx.x < 64) {
      const int64_t row = ma + 4 * threadIdx.x;
      f32x4 q;
      if (row + 3 < e.V) {
        q = *(const f32x4 *)(e.wscale + row);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) q[u] = (row + u < e.V) ? e.wscale[row + u] : 0.f;
      }
      wsl[threadIdx.x] = q;
    }
    __syncthreads();
  }
  pre_transform<L, A_FP8, TANH>(acc, wm, lane, e.pre, wsl);
  const float *xo = EX == 2 ? e.xoff + n0 : nullptr;
  if (ma + TM > e.V) stats_cols<L, true, EX, TANH, A_FP8>(acc, ma, wm, wn, lane, e.V, e.c, red, smem, nvalid, xo, wsl);
  else stats_cols<L, false, EX, TANH, A_FP8>(acc, ma, wm, wn, lane, e.V, e.c, red, smem, nvalid, xo, wsl);
  __syncthreads();  // per-wave statistics (and the staging tile) written
  const int t = threadIdx.x;
  if (t < nvalid) {  // (m_a, S, U, m_b): S and U relative to max(m_a, m_b), the halves' maxima kept
    const f32x4 a = red[t], b = red[256 + t];
    Stat3 sa{a[0], a[1], a[2]}, sb{b[0], b[1], b[2]};
    Stat3 r = stat_merge(sa, sb);
    f32x4 o;
    o[0] = a[0]; o[1] = r.S; o[2] = r.U; o[3] = b[0];
    e.part[(n0 + t) * e.mtiles + e.v0 / TM + mt] = o;
  }
  if constexpr (EX)
    lds_tile_to_global<2 * NTHREADS>(smem, (char *)e.ex + (n0 * e.ldx + ma) * 2, e.ldx * 2,
                                     [](int row) { return DzSwz<L>::at(row); });
}

template <int DT, bool A_FP8, bool TANH>
__global__ __launch_bounds__(2 * NTHREADS, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_dz8_kernel(Operand A, Operand B, GemmShape s, DzArgs e) {
  static_assert(ring5_ok(DT), "16-bit operands");
  typedef Acc16N<4> L;
  __shared__ __attribute__((aligned(16))) char smem_[SMEM_RING5];
  lds_char *smem = (lds_char *)smem_;
  int mt, nt;
  if (!tile_of(s, mt, nt)) return;
  const int64_t m0 = (int64_t)mt * TM, n0 = (int64_t)nt * TN;
  const int64_t nvalid = min(dev_count(s.count, s.count_off + n0, s.N - n0), (int64_t)TN);  // this tile's tokens
  if (nvalid <= 0) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = L::wm(w), wn = L::wn(w);
  typedef typename std::conditional<DT == OCTO_BF16, bf16x2, f16x2_t>::type P2;
  f32x4 acc[8][4];
  mainloop_ring5<DT, OpRowsN<8, 128>, OpRowsN<8, 64>, true>(A, B, m0, n0, s.K, smem, acc);
  const int64_t ma = e.v0 + m0;  // first vocabulary row of the tile; its dz columns start at m0
  if constexpr (A_FP8) {
    if (ma + TM > e.V) dz_stage_fp8<L, P2, TANH, true>(acc, e, ma, n0, nvalid, wm, wn, lane, smem);
    else dz_stage_fp8<L, P2, TANH, false>(acc, e, ma, n0, nvalid, wm, wn, lane, smem);
  } else {
    if (ma + TM > e.V) dz_stage<L, P2, TANH, true>(acc, e, ma, n0, nvalid, wm, wn, lane, smem);
    else dz_stage<L, P2, TANH, false>(acc, e, ma, n0, nvalid, wm, wn, lane, smem);
  }
  dz_write<L, P2, 2 * NTHREADS>(e, ma, m0, n0, nvalid, smem);
}

// ---- host launchers ----------------------------------------------------------------------------

static inline dim3 grid_of(const GemmShape &s) { return dim3((unsigned)tile_grid(s.mtiles, s.ntiles)); }

template <int DT, bool F8, bool TH>
static int go_stats(const Operand &A, const Operand &B, const GemmShape &s, const StatsArgs &e, hipStream_t st) {
  if constexpr (ring5_ok(DT)) {
    if (e.ex && e.xoff) {
      if constexpr (DT == OCTO_BF16)
        hipLaunchKernelGGL((gemm_stats8_kernel<DT, F8, TH, 2>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e);
      else
        return octo_fail(OCTO_EUNSUPPORTED, "gemm_stats: row-offset exponentials need bf16 operands");
    } else if (e.ex) {
      hipLaunchKernelGGL((gemm_stats8_kernel<DT, F8, TH, 1>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e);
    } else {
      hipLaunchKernelGGL((gemm_stats8_kernel<DT, F8, TH, 0>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e);
    }
  } else {
    if (e.ex) return octo_fail(OCTO_EUNSUPPORTED, "gemm_stats: exponentials of fp32 operands");
    hipLaunchKernelGGL((gemm_stats_kernel<DT, F8, TH>), grid_of(s), dim3(NTHREADS), 0, st, A, B, s, e);
  }
  OCTO_CHECK_LAUNCH("gemm_stats");
  return OCTO_OK;
}

template <int DT, bool F8, bool TH>
static int go_dz(const Operand &A, const Operand &B, const GemmShape &s, const DzArgs &e, hipStream_t st) {
  if constexpr (ring5_ok(DT))
    hipLaunchKernelGGL((gemm_dz8_kernel<DT, F8, TH>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e);
  else
    hipLaunchKernelGGL((gemm_dz_kernel<DT, F8, TH>), grid_of(s), dim3(NTHREADS), 0, st, A, B, s, e);
  OCTO_CHECK_LAUNCH("gemm_dz");
  return OCTO_OK;
}

int launch_gemm_stats(int dt, bool a_fp8, bool tanh, const Operand &A, const Operand &B, const GemmShape &s,
                      const StatsArgs &e, hipStream_t st) {
  if (a_fp8) {
    if (dt != OCTO_BF16) return octo_fail(OCTO_EUNSUPPORTED, "fp8 weights need bf16 hidden rows");
    return tanh ? go_stats<OCTO_BF16, true, true>(A, B, s, e, st) : go_stats<OCTO_BF16, true, false>(A, B, s, e, st);
  }
  switch (dt) {
    case OCTO_BF16: return tanh ? go_stats<OCTO_BF16, false, true>(A, B, s, e, st) : go_stats<OCTO_BF16, false, false>(A, B, s, e, st);
    case OCTO_F16: return tanh ? go_stats<OCTO_F16, false, true>(A, B, s, e, st) : go_stats<OCTO_F16, false, false>(A, B, s, e, st);
    case OCTO_F32: return tanh ? go_stats<OCTO_F32, false, true>(A, B, s, e, st) : go_stats<OCTO_F32, false, false>(A, B, s, e, st);
  }
  return octo_fail(OCTO_EUNSUPPORTED, "gemm_stats: dtype %d", dt);
}

int launch_gemm_dz(int dt, bool a_fp8, bool tanh, const Operand &A, const Operand &B, const GemmShape &s,
                   const DzArgs &e, hipStream_t st) {
  if (a_fp8) {
    if (dt != OCTO_BF16) return octo_fail(OCTO_EUNSUPPORTED, "fp8 weights need bf16 hidden rows");
    return tanh ? go_dz<OCTO_BF16, true, true>(A, B, s, e, st) : go_dz<OCTO_BF16, true, false>(A, B, s, e, st);
  }
  switch (dt) {
    case OCTO_BF16: return tanh ? go_dz<OCTO_BF16, false, true>(A, B, s, e, st) : go_dz<OCTO_BF16, false, false>(A, B, s, e, st);
    case OCTO_F16: return tanh ? go_dz<OCTO_F16, false, true>(A, B, s, e, st) : go_dz<OCTO_F16, false, false>(A, B, s, e, st);
    case OCTO_F32: return tanh ? go_dz<OCTO_F32, false, true>(A, B, s, e, st) : go_dz<OCTO_F32, false, false>(A, B, s, e, st);
  }
  return octo_fail(OCTO_EUNSUPPORTED, "gemm_dz: dtype %d", dt);
}

template <int DT, int KM>
static int go_store(const Operand &A, const Operand &B, const GemmShape &s, const StoreArgs &e, hipStream_t st) {
  if constexpr (ring5_ok(DT)) {
    switch (e.dtype) {
      case OCTO_BF16: hipLaunchKernelGGL((gemm_store8_kernel<DT, OCTO_BF16, KM>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e); break;
      case OCTO_F16: hipLaunchKernelGGL((gemm_store8_kernel<DT, OCTO_F16, KM>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e); break;
      case OCTO_F32: hipLaunchKernelGGL((gemm_store8_kernel<DT, OCTO_F32, KM>), grid_of(s), dim3(2 * NTHREADS), 0, st, A, B, s, e); break;
      default: return octo_fail(OCTO_EUNSUPPORTED, "gemm_store: output dtype %d", e.dtype);
    }
  } else {
    switch (e.dtype) {
      case OCTO_BF16: hipLaunchKernelGGL((gemm_store_kernel<DT, OCTO_BF16>), grid_of(s), dim3(NTHREADS), 0, st, A, B, s, e); break;
      case OCTO_F16: hipLaunchKernelGGL((gemm_store_kernel<DT, OCTO_F16>), grid_of(s), dim3(NTHREADS), 0, st, A, B, s, e); break;
      case OCTO_F32: hipLaunchKernelGGL((gemm_store_kernel<DT, OCTO_F32>), grid_of(s), dim3(NTHREADS), 0, st, A, B, s, e); break;
      default: return octo_fail(OCTO_EUNSUPPORTED, "gemm_store: output dtype %d", e.dtype);
    }
  }
  OCTO_CHECK_LAUNCH("gemm_store");
  return OCTO_OK;
}

template <int DT>
static int go_grads(const Operand &Ah, const Operand &Bh, const GemmShape &sh, const StoreArgs &eh, bool wh_kmajor,
                    const Operand &Aw, const Operand &Bw, const GemmShape &sw, const StoreArgs &ew, hipStream_t st) {
  const int64_t nh = tile_grid(sh.mtiles, sh.ntiles), nw = tile_grid(sw.mtiles, sw.ntiles);
  if (nh + nw > 0x7fffffffLL) return octo_fail(OCTO_EINVAL, "gemm_grads: %lld tiles", (long long)(nh + nw));
  const dim3 grid((unsigned)(nh + nw));
  if (wh_kmajor)
    hipLaunchKernelGGL((gemm_grads8_kernel<DT, KM_B>), grid, dim3(2 * NTHREADS), 0, st, Ah, Bh, sh, eh, Aw, Bw, sw, ew,
                       (unsigned)nh);
  else
    hipLaunchKernelGGL((gemm_grads8_kernel<DT, KM_NONE>), grid, dim3(2 * NTHREADS), 0, st, Ah, Bh, sh, eh, Aw, Bw, sw,
                       ew, (unsigned)nh);
  OCTO_CHECK_LAUNCH("gemm_grads");
  return OCTO_OK;
}

// The K-major loader (OpColsN) reads whole 512-byte rows of the tile's 256 columns of a plain (unmapped) matrix,
// up to the next multiple of 64 K-rows: the caller guarantees those rows exist.
static bool kmajor_layout_ok(const Operand &X) {
  return !X.map && !(X.ld & 15) && X.ld >= 512 && X.ld <= 0xffffffffLL / 64 && (uintptr_t)X.base % 16 == 0;
}

int launch_gemm_grads(int dt, const Operand &Ah, const Operand &Bh, const GemmShape &sh, const StoreArgs &eh,
                      bool wh_kmajor, const Operand &Aw, const Operand &Bw, const GemmShape &sw, const StoreArgs &ew,
                      hipStream_t st) {
  if (!eh.C || !ew.C || !Ah.base || !Bh.base || !Aw.base || !Bw.base)
    return octo_fail(OCTO_EINVAL, "gemm_grads: null operand or output");
  if (wh_kmajor && !kmajor_layout_ok(Bh)) return octo_fail(OCTO_EINVAL, "gemm_grads: K-major W layout");
  if (!kmajor_layout_ok(Aw)) return octo_fail(OCTO_EINVAL, "gemm_grads: K-major dz layout");
  for (int t : {eh.dtype, ew.dtype})
    if (t != OCTO_BF16 && t != OCTO_F16 && t != OCTO_F32) return octo_fail(OCTO_EUNSUPPORTED, "gemm_grads: output dtype %d", t);
  switch (dt) {
    case OCTO_BF16: return go_grads<OCTO_BF16>(Ah, Bh, sh, eh, wh_kmajor, Aw, Bw, sw, ew, st);
    case OCTO_F16: return go_grads<OCTO_F16>(Ah, Bh, sh, eh, wh_kmajor, Aw, Bw, sw, ew, st);
  }
  return octo_fail(OCTO_EUNSUPPORTED, "gemm_grads: dtype %d", dt);
}

int launch_gemm_store(int dt, const Operand &A, const Operand &B, const GemmShape &s, const StoreArgs &e,
                      hipStream_t st, int kmajor) {
  if (!e.C || !A.base || !B.base) return octo_fail(OCTO_EINVAL, "gemm_store: null operand or output");
  if (dt == OCTO_F32 && (e.part || e.part_blocked))
    return octo_fail(OCTO_EUNSUPPORTED, "gemm_store: fp32 operands store no partials");
  if (kmajor != KM_NONE) {
    if (!kmajor_layout_ok(kmajor == KM_A ? A : B)) return octo_fail(OCTO_EINVAL, "gemm_store: K-major operand layout");
    switch (dt) {
      case OCTO_BF16: return kmajor == KM_A ? go_store<OCTO_BF16, KM_A>(A, B, s, e, st) : go_store<OCTO_BF16, KM_B>(A, B, s, e, st);
      case OCTO_F16: return kmajor == KM_A ? go_store<OCTO_F16, KM_A>(A, B, s, e, st) : go_store<OCTO_F16, KM_B>(A, B, s, e, st);
    }
    return octo_fail(OCTO_EUNSUPPORTED, "gemm_store: K-major operand of dtype %d", dt);
  }
  switch (dt) {
    case OCTO_BF16: return go_store<OCTO_BF16, KM_NONE>(A, B, s, e, st);
    case OCTO_F16: return go_store<OCTO_F16, KM_NONE>(A, B, s, e, st);
    case OCTO_F32: return go_store<OCTO_F32, KM_NONE>(A, B, s, e, st);
  }
  return octo_fail(OCTO_EUNSUPPORTED, "gemm_store: dtype %d", dt);
}

}  // namespace octo
