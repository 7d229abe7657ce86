// Memory-bound kernels of the LM-head path and their C-ABI entry points:
//   merge          per-row merge of the vocab-tile softmax partials + target logit -> logp, entropy, lse
//   hit            per-row dz value at the label (the backward's dz epilogue writes it over the dense entry)
//   transpose      K-contiguous copies (W^T, gathered h^T) feeding the backward's gradient GEMMs
//   widen_fp8      e4m3 weights to bf16 (exact), the GEMMs' operand for fp8 weights
//   compact_rows   masked-row compaction, ascending (torch.nonzero order), count left on the device
//   columns fwd/bwd  _head_columns over materialised logits
//   pairs expand/grad, rows scatter, gather   the index plumbing of tree_head_output / _scored_rows
//   grpo           the per-token policy-gradient weight g = dL/dlogp of the GRPO objective
//   quantise_fp8   per-row e4m3 quantisation of a weight matrix (the fp8 weight format of the head)
#include "octo_internal.h"

namespace octo {

// 8 consecutive 16-bit values (one 16-byte chunk) as fp32, and back (round to nearest even).
__device__ __forceinline__ void unpack8(const i32x4 v, bool f16, float (&x)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t b = ((uint32_t)v[e >> 1] >> (16 * (e & 1))) & 0xffffu;
    x[e] = f16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)b) : __uint_as_float(b << 16);
  }
}
__device__ __forceinline__ i32x4 pack8(const float (&x)[8], bool f16) {
  i32x4 v;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    uint32_t lo, hi;
    if (f16) {
      lo = __builtin_bit_cast(uint16_t, (_Float16)x[2 * h]);
      hi = __builtin_bit_cast(uint16_t, (_Float16)x[2 * h + 1]);
    } else {
      lo = __builtin_bit_cast(uint16_t, (__bf16)x[2 * h]);
      hi = __builtin_bit_cast(uint16_t, (__bf16)x[2 * h + 1]);
    }
    v[h] = (int)(lo | (hi << 16));
  }
  return v;
}

// This lane's part of the fp32 dot product of hidden row hrow and weight row y (the target logit before any scale):
// 16-byte chunks when both are the same 16-bit type, element by element otherwise.
__device__ __forceinline__ float row_dot(const void *h, int h_dtype, int64_t hoff, const void *w, int w_dtype,
                                         int64_t woff, int d, int lane) {
  float dot = 0.f;
  if (h_dtype == w_dtype && (h_dtype == OCTO_BF16 || h_dtype == OCTO_F16) && d % 8 == 0) {
    const bool f16 = h_dtype == OCTO_F16;
    const char *hp = (const char *)h + hoff * 2, *wp = (const char *)w + woff * 2;
    for (int k = lane; k < d / 8; k += 64) {
      float a[8], b[8];
      unpack8(*(const i32x4 *)(hp + k * 16), f16, a);
      unpack8(*(const i32x4 *)(wp + k * 16), f16, b);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(a[e], b[e], dot);
    }
    return dot;
  }
  if (h_dtype == OCTO_BF16 && w_dtype == OCTO_FP8E4M3 && d % 16 == 0) {
    // 16 e4m3 weights per 16-byte load against 16 bf16 hidden values (rows are 16-byte aligned: the head's checks);
    // byte-wise loads made the merge 0.75 ms at 114,688 rows, d 2560
    const char *hp = (const char *)h + hoff * 2;
    const uint8_t *wp = (const uint8_t *)w + woff;
    for (int k = lane; k < d / 16; k += 64) {
      const i32x4 wv = *(const i32x4 *)(wp + k * 16);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float a[8];
        unpack8(*(const i32x4 *)(hp + k * 32 + half * 16), false, a);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t byte = ((uint32_t)wv[2 * half + (e >> 2)] >> (8 * (e & 3))) & 0xffu;
          dot = __builtin_fmaf(a[e], e4m3_to_f32(byte), dot);
        }
      }
    }
    return dot;
  }
  for (int k = lane; k < d; k += 64) {
    const float hv = load_as_f32(h, h_dtype, hoff + k);
    const float wv = w_dtype == OCTO_FP8E4M3 ? e4m3_to_f32(((const uint8_t *)w)[woff + k])
                                             : load_as_f32(w, w_dtype, woff + k);
    dot = __builtin_fmaf(hv, wv, dot);
  }
  return dot;
}

__device__ __forceinline__ void grpo_token(float lp, const float *prox, const float *old, float A, float eps_lo,
                                           float eps_hi, float reject_upper, float inv_z, float &gt, float &lt);

// ---- merge: vocab-tile partials -> per-row outputs ----------------------------------------------
// One wave per compact row, kMergeRows rows per workgroup: lanes merge the row's partials (m, S, U) strided by 64,
// then a wave butterfly; the target logit h_r . W_y is a wave dot product in fp32. With a GRPO tail the rows' loss
// terms are summed in LDS and added with one atomic per workgroup (one per row serialises on the scalar).
constexpr int kMergeRows = 16;

__global__ __launch_bounds__(64 * kMergeRows) void merge_kernel(MergeArgs a) {
  __shared__ float loss_part[kMergeRows];
  const int wave = threadIdx.x >> 6;
  const int64_t rl = (int64_t)blockIdx.x * kMergeRows + wave;  // row of this launch
  const int64_t r = a.row_off + rl;                              // compact row
  const int lane = threadIdx.x & 63;
  const int64_t cnt = a.count ? min((int64_t)(*a.count), a.n_max) : a.n_max;
  const int64_t rows = a.rows < 0 ? a.n_max : a.rows;
  float lt = 0.f;
  if (rl < rows && r < cnt) {
    const int64_t hrow = a.idx ? a.idx[r] : r;
    const int64_t y = a.labels[(a.flags & OCTO_ROWS_VIA_IDX) ? hrow : r];

    Stat3 st{-INFINITY, 0.f, 0.f};
    const f32x4 *pr = a.part + rl * a.mtiles;
    for (int64_t mt = lane; mt < a.mtiles; mt += 64) {
      const f32x4 p = pr[mt];
      st = stat_merge(st, Stat3{fmaxf(p[0], p[3]), p[1], p[2]});
    }
    st = wave_stat_merge(st);

    float dot = 0.f;
    const bool y_ok = y >= 0 && y < a.V;
    if (a.tdot) {
      dot = a.tdot[r];
    } else {
      if (y_ok) dot = row_dot(a.h, a.h_dtype, hrow * a.ldh, a.w, a.w_dtype, y * a.ldw, a.d, lane);
      dot = wave_sum(dot);
    }
    if (lane == 0) {
      const float raw = dot;  // h . W_y as stored (fp8: before the row scale)
      if (a.w_dtype == OCTO_FP8E4M3 && y_ok) dot *= a.wscale[y];
      const float zt = a.use_tanh ? a.post * tanhf(a.pre * dot) : a.post * a.pre * dot;
      const float sy = zt * a.inv_T;
      const float l2S = flog2(st.S);
      const float lse = (st.m + l2S) * OCTO_LN2;
      const float ent = (l2S - st.U / st.S) * OCTO_LN2;
      const float lp = y_ok ? sy - lse : __builtin_nanf("");
      if (a.logp) a.logp[r] = lp;
      if (a.ent) a.ent[r] = ent;
      if (a.lse) {
        if (a.lse_pair) {
          a.lse[2 * r] = st.m;
          a.lse[2 * r + 1] = l2S;
        } else {
          a.lse[r] = lse;
        }
      }
      if (a.out2) {
        const int64_t orow = (a.flags & OCTO_OUT_SCATTER) ? hrow : r;
        a.out2[orow * a.ld_out2] = lp;
        a.out2[orow * a.ld_out2 + 1] = ent;
      }
      if (a.g) {  // the GRPO weight of the row's token, in compact order
        float gt = 0.f;
        if (hrow < a.n_tokens && a.gmask[hrow] != 0.f)
          grpo_token(lp, a.gprox ? a.gprox + hrow : nullptr, a.gold ? a.gold + hrow : nullptr, a.gadv[hrow],
                     a.eps_lo, a.eps_hi, a.reject_upper, 1.f / a.z[0], gt, lt);
        a.g[r] = gt;
      }
      if (a.hit) {  // the label entry per unit of g gmul: launch_hit's formula from the same target logit and state
        float v = 0.f;
        if (y_ok) {
          const bool f8 = a.w_dtype == OCTO_FP8E4M3;
          const float x = f8 ? raw * a.wscale[y] : raw;
          if (a.use_tanh) {
            const float th = ftanh(a.pre * x);
            v = (1.f - fexp2(__builtin_fmaf(th, a.c, -st.m) - l2S)) * (1.f - th * th);
          } else {
            v = 1.f - fexp2(__builtin_fmaf(x, a.c, -st.m) - l2S);
          }
          if (f8) v *= a.wscale[y];
        }
        a.hit[rl] = v;
        if (a.exs) {  // row-offset exponentials: the label entry, or the row flagged for launch_ex_fix
          const float xo = a.xoff[r];
          if (st.m - xo <= kExClamp) {  // false for xo = -inf (a label outside [0, V)) and NaN
            a.xuse[rl] = xo;
            if (y_ok) ((__bf16 *)a.exs)[rl * a.ldx + y] = (__bf16)(-v * fexp2(st.m - xo + l2S));
          } else {
            a.xuse[rl] = st.m;
            a.flag_rows[atomicAdd(a.flag_cnt, 1)] = (int32_t)rl;
          }
        }
      }
      if (a.zero_g) a.g_zero[r] = 0.f;
    }
  } else if (lane == 0 && rl < rows) {
    if (a.hit) a.hit[rl] = 0.f;
    if (a.zero_g && a.row_off + rl < a.n_max) a.g_zero[a.row_off + rl] = 0.f;
  }
  if (!a.loss) return;  // uniform across the workgroup: no barrier below is skipped by part of it
  if (lane == 0) loss_part[wave] = lt;
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < kMergeRows; ++k) sum += loss_part[k];
    if (sum != 0.f) atomicAdd(a.loss, sum);
  }
}

int launch_merge(const MergeArgs &a, hipStream_t st) {
  const int64_t rows = a.rows < 0 ? a.n_max : a.rows;
  if (rows == 0) return OCTO_OK;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)cdiv(rows, kMergeRows)), dim3(64 * kMergeRows), 0, st, a);
  OCTO_CHECK_LAUNCH("merge");
  return OCTO_OK;
}

// ---- dz label entries ----------------------------------------------------------------------------------
// One wave per row: the target logit h . W_y in fp32 (as the forward's merge), then the dz value at the label with
// the dz kernel's own formula, so the GEMM epilogue writes it over the dense entry -g p / T instead of testing every
// element against the label.
__global__ __launch_bounds__(256) void hit_kernel(HitArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= a.rows) return;
  const int64_t r = a.r0 + i;
  const int64_t cnt = a.count ? min((int64_t)(*a.count), a.n_max) : a.n_max;
  float hv_out = 0.f;
  if (r < cnt) {
    const int64_t hrow = a.idx ? a.idx[r] : r;
    const int64_t y = a.labels[a.label_idx ? a.label_idx[r] : r];
    if (y >= 0 && y < a.V) {
      float dot = row_dot(a.h, a.h_dtype, hrow * a.ldh, a.w, a.w_dtype, y * a.ldw, a.d, lane);
      dot = wave_sum(dot);
      const bool f8 = a.w_dtype == OCTO_FP8E4M3;
      const float x = f8 ? dot * a.wscale[y] : dot;
      float m2, l2s;
      row_state(a.lse, a.lse_pair, r, m2, l2s);
      const float gs = a.g[r] * a.gmul;
      float v;
      if (a.use_tanh) {
        const float th = ftanh(a.pre * x);
        v = __builtin_fmaf(-gs, fexp2(__builtin_fmaf(th, a.c, -m2) - l2s), gs) * (1.f - th * th);
      } else {
        v = __builtin_fmaf(-gs, fexp2(__builtin_fmaf(x, a.c, -m2) - l2s), gs);
      }
      hv_out = f8 ? v * a.wscale[y] : v;
    }
  }
  if (lane == 0) a.hit[i] = hv_out;
}

int launch_hit(const HitArgs &a, hipStream_t st) {
  if (a.rows == 0) return OCTO_OK;
  hipLaunchKernelGGL(hit_kernel, dim3((unsigned)cdiv(a.rows, 4)), dim3(256), 0, st, a);
  OCTO_CHECK_LAUNCH("hit");
  return OCTO_OK;
}

// ---- dz from the stored exponentials (the fused step) ---------------------------------------------------
// One workgroup per (row, 4,096 columns): 2 x 16 bytes per thread, loaded together, scaled by the row's factor for
// their half tile (8 columns never straddle a 128-column half tile), the label entry replaced, stored back. The
// row's state is uniform over the workgroup (scalar loads). Non-temporal: the rows are read back only by the
// gradient GEMMs, after the rest of the pass's [rows, V] has streamed through. Same box, 24,576 rows at V 151,936 and
// 114,688 at fp8: 2 chunks per thread 2.50 and 12.2 ms per step, against 2.73 and 15.0 for 4, 2.60 and 13.5 for 1,
// 31.7 ms at fp8 for 8; temporal loads 2.52 and 13.0.
#ifndef OCTO_SCALE_CHUNKS
#define OCTO_SCALE_CHUNKS 2
#endif
#ifndef OCTO_SCALE_NT_LOAD
#define OCTO_SCALE_NT_LOAD 1
#endif
constexpr int kScaleChunks = OCTO_SCALE_CHUNKS;  // 16-byte chunks per thread

__global__ __launch_bounds__(256) void dz_scale_kernel(DzScaleArgs a) {
  const int64_t i = blockIdx.y;  // row of the pass
  const int64_t r = a.r0 + i;
  const int64_t cnt = a.count ? min((int64_t)(*a.count), a.n_max) : a.n_max;
  if (r >= cnt) return;
  float m2, l2s;
  row_state(a.lse, a.lse_pair, r, m2, l2s);
  const float ngs = -(a.g[r] * a.gmul);
  const int64_t y = a.labels[a.label_idx ? a.label_idx[r] : r];
  const bool f16 = a.dtype == OCTO_F16;
  const f32x4 *pr = a.part + i * a.mtiles;
  char *row = (char *)a.dz + i * a.ld * 2;
  const int64_t chunk0 = (int64_t)blockIdx.x * (256 * kScaleChunks) + threadIdx.x;
  i32x4 v[kScaleChunks];
#pragma unroll
  for (int k = 0; k < kScaleChunks; ++k) {
    const int64_t c0 = (chunk0 + 256 * k) * 8;
    if (c0 < a.V_pad)
      v[k] = OCTO_SCALE_NT_LOAD ? __builtin_nontemporal_load((const i32x4 *)(row + c0 * 2)) : *(const i32x4 *)(row + c0 * 2);
  }
#pragma unroll
  for (int k = 0; k < kScaleChunks; ++k) {
    const int64_t c0 = (chunk0 + 256 * k) * 8;
    if (c0 >= a.V_pad) continue;
    const f32x4 q = pr[c0 >> 8];  // the maximum the exponentials of this half of the tile are relative to
    const float s = ngs * fexp2(((c0 & 128) ? q[3] : q[0]) - m2 - l2s);
    float x[8];
    unpack8(v[k], true, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= s;
    if (a.wscale) {  // fp8 weights: each column's row scale (the chain rule through z = scale x raw product)
      if (c0 + 8 <= a.V) {  // two aligned 16-byte loads (c0 is a multiple of 8, the scales 16-byte aligned)
        const f32x4 s0 = *(const f32x4 *)(a.wscale + c0), s1 = *(const f32x4 *)(a.wscale + c0 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] *= s0[e];
          x[e + 4] *= s1[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= (c0 + e < a.V) ? a.wscale[c0 + e] : 0.f;
      }
    }
    if (y >= c0 && y < c0 + 8 && y < a.V) x[y - c0] = -ngs * a.hit[i];  // g gmul (1 - p_y) post'(z_y) (x scale)
    __builtin_nontemporal_store(pack8(x, f16), (i32x4 *)(row + c0 * 2));
  }
}

int launch_dz_scale(const DzScaleArgs &a, hipStream_t st) {
  if (a.rows == 0) return OCTO_OK;
  OCTO_CHECK_ARG(a.dtype == OCTO_BF16 || a.dtype == OCTO_F16, "dz_scale: dtype %d", a.dtype);
  OCTO_CHECK_ARG(a.V_pad % 8 == 0 && a.ld % 8 == 0 && a.ld >= a.V_pad && ((uintptr_t)a.dz) % 16 == 0,
                 "dz_scale: rows of 16-byte chunks");
  OCTO_CHECK_ARG(a.rows <= 65535, "dz_scale: %lld rows in one launch", (long long)a.rows);
  const unsigned bx = (unsigned)cdiv(a.V_pad / 8, 256 * kScaleChunks);
  hipLaunchKernelGGL(dz_scale_kernel, dim3(bx, (unsigned)a.rows), dim3(256), 0, st, a);
  OCTO_CHECK_LAUNCH("dz_scale");
  return OCTO_OK;
}

// ---- the row-offset exponentials of the fused step (StatsArgs::xoff) ------------------------------------------
// Before the passes, one wave per compact row (4 per workgroup): the target dot product exactly as the merge forms it
// (row_dot, wave_sum), kept for the merge, and the row's offset: the label's base-2 logit + kExAbove. The label's
// logit lies at or below the row's maximum m2, so every element within 2^-40 of the row's largest is stored at
// 2^-88 or more (a bf16 normal), and a row's exponentials need no rescaling unless m2 lies more than kExAbove +
// kExClamp = 112 (base 2; 77.6 nats) above its label's logit.
__global__ __launch_bounds__(256) void row_offsets_kernel(RowOffArgs a) {
  if (blockIdx.x == 0)
    for (int k = threadIdx.x; k < a.nflag; k += 256) a.flag_cnt[k] = 0;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t cnt = a.count ? min((int64_t)(*a.count), a.n_max) : a.n_max;
  if (r >= cnt) return;
  const int64_t hrow = a.idx ? a.idx[r] : r;
  const int64_t y = a.labels[a.label_via_idx ? hrow : r];
  const bool y_ok = y >= 0 && y < a.V;
  float dot = 0.f;
  if (y_ok) dot = row_dot(a.h, a.h_dtype, hrow * a.ldh, a.w, a.w_dtype, y * a.ldw, a.d, lane);
  dot = wave_sum(dot);
  if (lane == 0) {
    a.tdot[r] = dot;
    float x = (a.w_dtype == OCTO_FP8E4M3 && y_ok) ? dot * a.wscale[y] : dot;
    if (a.use_tanh) x = ftanh(a.pre * x);
    a.xoff[r] = y_ok ? __builtin_fmaf(x, a.c, kExAbove) : -INFINITY;
  }
}

int launch_row_offsets(const RowOffArgs &a, hipStream_t st) {
  const int64_t blocks = cdiv(a.n_max, 4) > 0 ? cdiv(a.n_max, 4) : 1;
  OCTO_CHECK_ARG(blocks <= 0x7fffffff, "row_offsets: %lld rows", (long long)a.n_max);
  hipLaunchKernelGGL(row_offsets_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
  OCTO_CHECK_LAUNCH("row_offsets");
  return OCTO_OK;
}

// After a pass's merge: the workgroups set the dz scales of a strided slice of the pass's rows, then share the
// rescale of the flagged rows (none in the usual case: each workgroup then reads the count and ends). The rescale is
// cut into work items of one flagged row x kExFixCols columns, dealt to the workgroups in turn, so that at a low
// temperature, where most rows are flagged, it streams at the HBM rate: each thread issues its four 16-byte loads
// before the first store. A flagged row is rescaled in place to its new offset (the merge set xuse = m2) by its half
// tiles' factors (8 columns never straddle a 128-column half tile): the stored value of half tile h is
// e exp2(min(m_h - xoff, kExClamp)) with e = exp2(c t - m_h), and exp2(c t - m2) = that x exp2(m_h - m2 - min(m_h -
// xoff, kExClamp)). Same box, 24,576 of 32,768 rows at d 2560, V 151,936, T 0.012 (almost every row flagged): the
// 64-workgroup form that took one whole row per workgroup at a time ran 17.5 ms per step.
constexpr int kExFixBlocks = 2048;        // 8 per CU
constexpr int kExFixLoads = 4;            // 16-byte chunks per thread and work item
constexpr int kExFixCols = 256 * 8 * kExFixLoads;
__global__ __launch_bounds__(256) void ex_fix_kernel(ExFixArgs a) {
  const int64_t cnt = a.count ? min((int64_t)(*a.count), a.n_max) : a.n_max;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.rows; i += (int64_t)gridDim.x * 256) {
    const int64_t r = a.r0 + i;
    float s = 0.f;
    if (r < cnt) {
      float m2, l2s;
      row_state(a.lse, a.lse_pair, r, m2, l2s);
      s = -(a.g[r] * a.gmul) * fexp2(a.xuse[i] - m2 - l2s);
    }
    a.scale[i] = s;
  }
  const int64_t nf = *a.flag_cnt;
  const int64_t chunks = (a.V_pad + kExFixCols - 1) / kExFixCols;
  for (int64_t k = blockIdx.x; k < nf * chunks; k += gridDim.x) {
    const int64_t f = k / chunks, cbase = (k - f * chunks) * kExFixCols;
    const int64_t i = a.flag_rows[f], r = a.r0 + i;
    const float xo = a.xoff[r], xn = a.xuse[i];
    float m2, l2s;
    row_state(a.lse, a.lse_pair, r, m2, l2s);
    const int64_t y = a.labels[a.label_idx ? a.label_idx[r] : r];
    const f32x4 *pr = a.part + i * a.mtiles;
    char *row = (char *)a.ex + i * a.ldx * 2;
    i32x4 v[kExFixLoads];
#pragma unroll
    for (int u = 0; u < kExFixLoads; ++u) {
      const int64_t c0 = cbase + (int64_t)(u * 256 + threadIdx.x) * 8;
      if (c0 < a.V_pad) v[u] = *(const i32x4 *)(row + c0 * 2);
    }
#pragma unroll
    for (int u = 0; u < kExFixLoads; ++u) {
      const int64_t c0 = cbase + (int64_t)(u * 256 + threadIdx.x) * 8;
      if (c0 >= a.V_pad) continue;
      const f32x4 q = pr[c0 >> 8];
      const float mh = (c0 & 128) ? q[3] : q[0];  // -inf: no column of the half lies below V (stored zeros)
      const float fac = mh == -INFINITY ? 0.f : fexp2(mh - xn - fminf(mh - xo, kExClamp));
      float x[8];
      unpack8(v[u], false, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= fac;
      if (y >= c0 && y < c0 + 8 && y < a.V) x[y - c0] = -a.hit[i] * fexp2(m2 - xn + l2s);
      *(i32x4 *)(row + c0 * 2) = pack8(x, false);
    }
  }
}

int launch_ex_fix(const ExFixArgs &a, hipStream_t st) {
  if (a.rows == 0) return OCTO_OK;
  OCTO_CHECK_ARG(a.V_pad % 256 == 0 && a.ldx >= a.V_pad && ((uintptr_t)a.ex) % 16 == 0 && a.ldx % 8 == 0,
                 "ex_fix: rows of whole 256-column tiles");
  hipLaunchKernelGGL(ex_fix_kernel, dim3(kExFixBlocks), dim3(256), 0, st, a);
  OCTO_CHECK_LAUNCH("ex_fix");
  return OCTO_OK;
}

// ---- y = c y + x over a vector (the bound GRPO step's backward) ------------------------------------------------------
// c is read from device memory, and so is `skip_x` (when given): while it is non-zero x counts as zero and is not read.
// x = NULL: y = c y. The product and the sum are formed in fp32 and rounded once to the vector's type. With c = 1 and
// no x to add, y is already the result and every workgroup ends at once. 16 bytes per thread and step.
__global__ __launch_bounds__(256) void scale_add_kernel(void *y, const void *x, int dtype, int64_t n, const float *c,
                                                        const int32_t *skip_x) {
  const float s = *c;
  const bool add = x && !(skip_x && *skip_x);
  if (s == 1.f && !add) return;
  const int per = dtype == OCTO_F32 ? 4 : 8;  // elements per 16-byte chunk
  const int64_t chunks = n / per;
  for (int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x; k < chunks; k += (int64_t)gridDim.x * 256) {
    i32x4 *yp = (i32x4 *)((char *)y + k * 16);
    const i32x4 xv = add ? *(const i32x4 *)((const char *)x + k * 16) : i32x4{0, 0, 0, 0};
    if (dtype == OCTO_F32) {
      f32x4 a = __builtin_bit_cast(f32x4, *yp);
      const f32x4 b = __builtin_bit_cast(f32x4, xv);
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = __builtin_fmaf(s, a[e], b[e]);
      *yp = __builtin_bit_cast(i32x4, a);
    } else {
      const bool f16 = dtype == OCTO_F16;
      float a[8], b[8];
      unpack8(*yp, f16, a);
      unpack8(xv, f16, b);
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = __builtin_fmaf(s, a[e], b[e]);
      *yp = pack8(a, f16);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n - chunks * per) {  // the last n % per elements
    const int64_t i = chunks * per + threadIdx.x;
    const float b = add ? load_as_f32(x, dtype, i) : 0.f;
    store_from_f32(y, dtype, i, __builtin_fmaf(s, load_as_f32(y, dtype, i), b));
  }
}

// ---- the fused step's GRPO tail over prefix-tree pair rows ----------------------------------------------
// One thread per flat token; the workgroup's loss terms are summed in LDS and added with one atomic (as the merge).
__global__ __launch_bounds__(256) void pairs_grpo_kernel(PairsGrpoArgs a) {
  __shared__ float part[256];
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t cnt = a.count ? min((int64_t)(*a.count), a.n_max) : a.n_max;
  float lt = 0.f;
  if (t < a.n_flat) {
    const int64_t p = a.flat_pair[t];
    const bool paired = p >= 0 && p < cnt;
    if (paired && p >= a.r0 && p < a.r0 + a.rows) {
      const float lp = a.rowout[2 * p], ent = a.rowout[2 * p + 1];
      a.out2[t * a.ld_out2] = lp;
      a.out2[t * a.ld_out2 + 1] = ent;
      if (t < a.n_tokens && a.mask[t] != 0.f) {
        float gt = 0.f;
        grpo_token(lp, a.prox ? a.prox + t : nullptr, a.old ? a.old + t : nullptr, a.adv[t], a.eps_lo, a.eps_hi,
                   a.reject_upper, 1.f / a.z[0], gt, lt);
        if (gt != 0.f) atomicAdd(a.g + p, gt);
      }
    } else if (!paired && a.first_pass) {  // columns 0; a masked token adds its loss term at logprob 0 (no row)
      a.out2[t * a.ld_out2] = 0.f;
      a.out2[t * a.ld_out2 + 1] = 0.f;
      if (t < a.n_tokens && a.mask[t] != 0.f) {
        float gt = 0.f;
        grpo_token(0.f, a.prox ? a.prox + t : nullptr, a.old ? a.old + t : nullptr, a.adv[t], a.eps_lo, a.eps_hi,
                   a.reject_upper, 1.f / a.z[0], gt, lt);
      }
    }
  }
  if (!a.loss) return;  // uniform across the workgroup
  part[threadIdx.x] = lt;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0 && part[0] != 0.f) atomicAdd(a.loss, part[0]);
}

int launch_pairs_grpo(const PairsGrpoArgs &a, hipStream_t st) {
  if (a.n_flat == 0) return OCTO_OK;
  hipLaunchKernelGGL(pairs_grpo_kernel, dim3((unsigned)cdiv(a.n_flat, 256)), dim3(256), 0, st, a);
  OCTO_CHECK_LAUNCH("pairs_grpo");
  return OCTO_OK;
}

// ---- transpose -----------------------------------------------------------------------------------
// Rows of dst written: all rows_pad without a device count (zeros past rows: a staged W^T is read to the next multiple
// of 256); with one, the count rounded up to 64, the K extent the gradient GEMMs read of a count-bounded h^T
// (GemmShape count_on 3), so that columns no GEMM reads are not zero-filled. A whole tile past it ends at once (the
// check is uniform across the block: r0 is the block's).
__device__ __forceinline__ int64_t written_rows(const int32_t *count, int64_t valid, int64_t rows_pad) {
  return count ? min(rows_pad, (valid + 63) / 64 * 64) : rows_pad;
}

// dst[c, r] = src[row(r), c]: 64 x 64 tiles through LDS (fp32 words, padded against bank conflicts).
__global__ __launch_bounds__(256) void transpose_kernel(const void *src, int64_t ld_src, int src_dtype,
                                                        const int64_t *map, const int32_t *count,
                                                        int64_t count_off, int64_t rows, int64_t rows_pad,
                                                        int64_t cols, void *dst, int64_t ld_dst, int dst_dtype) {
  __shared__ float tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int64_t valid = dev_count(count, count_off, rows);
  const int64_t lim = written_rows(count, valid, rows_pad);
  if (r0 >= lim) return;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    float x = 0.f;
    if (r < valid && c < cols) {
      const int64_t pr = map ? map[r] : r;
      if (src_dtype == OCTO_FP8E4M3) x = e4m3_to_f32(((const uint8_t *)src)[pr * ld_src + c]);
      else x = load_as_f32(src, src_dtype, pr * ld_src + c);
    }
    tile[i][tx] = x;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (c < cols && r < lim) store_from_f32(dst, dst_dtype, c * ld_dst + r, tile[tx][i]);
  }
}

// The 16-bit form: 16-byte loads and stores. In the LDS tile, element (column c, row r) sits at
// c * 128 + ((r >> 3) ^ ((c >> 3) & 7)) * 16 + (r & 7) * 2: a wave's 2-byte writes (8 rows x 8 column chunks, one
// element of each) and its 16-byte reads (whole 128-byte column rows) both hit distinct banks.
typedef __attribute__((address_space(3))) short lds_short16;
typedef __attribute__((address_space(3))) i32x4 lds_i32x4_t;
__global__ __launch_bounds__(256) void transpose16_kernel(const char *src, int64_t ld_src, const int64_t *map,
                                                          const int32_t *count, int64_t count_off, int64_t rows,
                                                          int64_t rows_pad, int64_t cols, char *dst, int64_t ld_dst,
                                                          const float *rscale, int is_f16) {
  __shared__ __attribute__((aligned(16))) char tile_[64 * 128];
  __attribute__((address_space(3))) char *tile = (__attribute__((address_space(3))) char *)tile_;
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int64_t valid = dev_count(count, count_off, rows);
  const int64_t lim = written_rows(count, valid, rows_pad);
  if (r0 >= lim) return;
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int c = t + 256 * k;  // 16-byte chunk of the source tile: row c >> 3, columns 8 (c & 7) ..
    const int row = c >> 3, cc = c & 7;
    const int64_t r = r0 + row, col = c0 + 8 * cc;
    i32x4 v = {0, 0, 0, 0};
    if (r < valid && col < cols) {
      v = *(const i32x4 *)(src + (map ? map[r] : r) * ld_src + col * 2);
      if (rscale) {  // row r times its scale, rounded once
        float x[8];
        unpack8(v, is_f16 != 0, x);
        const float sc = rscale[r];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= sc;
        v = pack8(x, is_f16 != 0);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const short x = (short)((uint32_t)v[e >> 1] >> (16 * (e & 1)));
      *(lds_short16 *)(tile + (8 * cc + e) * 128 + (((row >> 3) ^ cc) << 4) + (row & 7) * 2) = x;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int c = t + 256 * k;  // destination row c0 + (c >> 3), source rows r0 + 8 (c & 7) ..
    const int drow = c >> 3, rc = c & 7;
    const int64_t col = c0 + drow, r = r0 + 8 * rc;
    if (col < cols && r < lim) {
      const i32x4 v = *(const lds_i32x4_t *)(tile + drow * 128 + ((rc ^ ((drow >> 3) & 7)) << 4));
      *(i32x4 *)(dst + (col * ld_dst + r) * 2) = v;
    }
  }
}

int launch_transpose(const void *src, int64_t ld_src, int src_dtype, const float *row_scale,
                     const int64_t *map, const int32_t *count, int64_t count_off, int64_t rows,
                     int64_t rows_pad, int64_t cols, void *dst, int64_t ld_dst, int dst_dtype, hipStream_t st) {
  if (rows_pad == 0 || cols == 0) return OCTO_OK;
  dim3 grid((unsigned)cdiv(rows_pad, 64), (unsigned)cdiv(cols, 64));
  const bool b16 = (src_dtype == OCTO_BF16 || src_dtype == OCTO_F16) && dst_dtype == src_dtype;
  if (b16 && cols % 8 == 0 && rows_pad % 64 == 0 && ld_src % 8 == 0 && ld_dst % 8 == 0 &&
      ((uintptr_t)src) % 16 == 0 && ((uintptr_t)dst) % 16 == 0) {
    hipLaunchKernelGGL(transpose16_kernel, grid, dim3(256), 0, st, (const char *)src, ld_src * 2, map, count,
                       count_off, rows, rows_pad, cols, (char *)dst, ld_dst, row_scale, src_dtype == OCTO_F16 ? 1 : 0);
    OCTO_CHECK_LAUNCH("transpose");
    return OCTO_OK;
  }
  if (row_scale) return octo_fail(OCTO_EUNSUPPORTED, "transpose: row scales need 16-bit rows of 16-byte chunks");
  hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, st, src, ld_src, src_dtype, map, count, count_off, rows,
                     rows_pad, cols, dst, ld_dst, dst_dtype);
  OCTO_CHECK_LAUNCH("transpose");
  return OCTO_OK;
}

// ---- fp8 weight widening -----------------------------------------------------------------------------
// dst[V, d] bf16 = the e4m3 weight values, exactly (no row scale: the GEMM epilogues apply it in fp32). One thread per
// 16 weights.
__global__ __launch_bounds__(256) void widen_fp8_kernel(const uint8_t *w, int64_t ldw, int64_t V, int64_t chunks,
                                                        char *dst) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= V * chunks) return;
  const int64_t r = i / chunks, c = i - r * chunks;
  const i32x4 raw = *(const i32x4 *)(w + r * ldw + c * 16);
  i32x4 o[2];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    o[h >> 1][2 * (h & 1)] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[h], 1.0f, false));
    o[h >> 1][2 * (h & 1) + 1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[h], 1.0f, true));
  }
  i32x4 *d = (i32x4 *)(dst + (r * chunks + c) * 32);
  d[0] = o[0];
  d[1] = o[1];
}

int launch_widen_fp8(const void *w, int64_t ldw, int64_t V, int d, void *dst, hipStream_t st) {
  if (V == 0) return OCTO_OK;
  if (d % 16 || ldw % 16) return octo_fail(OCTO_EINVAL, "widen_fp8: rows must be whole 16-byte chunks");
  const int64_t chunks = d / 16;
  hipLaunchKernelGGL(widen_fp8_kernel, dim3((unsigned)cdiv(V * chunks, 256)), dim3(256), 0, st, (const uint8_t *)w,
                     ldw, V, chunks, (char *)dst);
  OCTO_CHECK_LAUNCH("widen_fp8");
  return OCTO_OK;
}

// ---- compaction ----------------------------------------------------------------------------------
// One workgroup of 16 waves sweeps the mask 1024 entries at a time: a ballot per wave, the lane's
// rank from the bits below it, the waves' totals scanned through LDS.
__global__ __launch_bounds__(1024) void compact_kernel(const uint8_t *mask, int64_t n, int64_t *idx, int32_t *count) {
  __shared__ int wsum[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int64_t base = 0;
  for (int64_t s0 = 0; s0 < n; s0 += 1024) {
    const int64_t i = s0 + threadIdx.x;
    const bool f = i < n && mask[i] != 0;
    const uint64_t bal = __ballot(f);
    const int rank = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wsum[w] = __popcll(bal);
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int c = wsum[k];
      off += (k < w) ? c : 0;
      tot += c;
    }
    if (f) idx[base + off + rank] = i;
    base += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) *count = (int32_t)base;
}

// ---- _head_columns over materialised logits ------------------------------------------------------
__global__ __launch_bounds__(256) void columns_fwd_kernel(const void *logits, int64_t ld, int dtype,
                                                          const int64_t *labels, int V, float inv_T,
                                                          float *out2, float *lse_out) {
  const int64_t r = blockIdx.x;
  __shared__ float red[3][4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const float c = inv_T * OCTO_LOG2E;
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < V; j += 256) mx = fmaxf(mx, load_as_f32(logits, dtype, r * ld + j));
  mx = wave_max(mx);
  if (lane == 0) red[0][w] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float m2 = mx * c;
  float S = 0.f, U = 0.f;
  for (int j = threadIdx.x; j < V; j += 256) {
    const float t = __builtin_fmaf(load_as_f32(logits, dtype, r * ld + j), c, -m2);
    const float e = fexp2(t);
    S += e;
    U = __builtin_fmaf(e, t, U);
  }
  S = wave_sum(S);
  U = wave_sum(U);
  if (lane == 0) {
    red[1][w] = S;
    red[2][w] = U;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    S = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    U = red[2][0] + red[2][1] + red[2][2] + red[2][3];
    const float l2S = flog2(S);
    const float lse = (m2 + l2S) * OCTO_LN2;
    const int64_t y = labels[r];
    const float sy = (y >= 0 && y < V) ? load_as_f32(logits, dtype, r * ld + y) * inv_T : __builtin_nanf("");
    out2[2 * r] = sy - lse;
    out2[2 * r + 1] = (l2S - U / S) * OCTO_LN2;
    if (lse_out) {  // the row state (m2, l2S) for columns_bwd, as row_state's paired form
      lse_out[2 * r] = m2;
      lse_out[2 * r + 1] = l2S;
    }
  }
}

__global__ __launch_bounds__(256) void columns_bwd_kernel(const void *logits, int64_t ld, int dtype,
                                                          const int64_t *labels, int V, float inv_T,
                                                          const float *lse, const float *g, void *dl,
                                                          int64_t ld_d) {
  const int64_t r = blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= V) return;
  // the forward's own t = fma(x, c, -m2), so the row's p keep the forward's rounding (row_state)
  const float p = fexp2(__builtin_fmaf(load_as_f32(logits, dtype, r * ld + j), inv_T * OCTO_LOG2E, -lse[2 * r]) -
                        lse[2 * r + 1]);
  const float onehot = (labels[r] == j) ? 1.f : 0.f;
  store_from_f32(dl, dtype, r * ld_d + j, g[r] * inv_T * (onehot - p));
}

// ---- pairs / rows plumbing -----------------------------------------------------------------------
__global__ void pairs_expand_kernel(const float *pairs, int64_t P, int C, const int64_t *fp, int64_t T, float *out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * C) return;
  const int64_t t = i / C, c = i - t * C;
  const int64_t p = fp[t];
  out[i] = (p >= 0 && p < P) ? pairs[p * C + c] : 0.f;
}

__global__ void fill_zero_kernel(float *x, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = 0.f;
}

__global__ void pairs_grad_kernel(const float *gf, int64_t T, int C, const int64_t *fp, int64_t P, float *gp) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * C) return;
  const int64_t t = i / C, c = i - t * C;
  const int64_t p = fp[t];
  if (p >= 0 && p < P) atomicAdd(gp + p * C + c, gf[i]);
}

// One workgroup per compact row r that starts a run of equal idx; it sums the run in fp32.
// dst row r = src row idx[r] for r < *count (rows at and after it untouched), 16-byte chunks; one workgroup per row.
// The GEMMs address rows read through a row map with 32-bit offsets from the matrix base, so a hidden matrix of
// 2 GiB or more is gathered into a contiguous copy first.
__global__ __launch_bounds__(256) void rows_gather_kernel(const char *src, int64_t ld_src, const int64_t *idx,
                                                          const int32_t *count, int64_t n_max, int64_t row_bytes,
                                                          char *dst) {
  const int64_t r = blockIdx.x;
  const int64_t cnt = count ? min((int64_t)(*count), n_max) : n_max;
  if (r >= cnt) return;
  const char *s = src + idx[r] * ld_src;
  char *o = dst + r * row_bytes;
  for (int64_t c = threadIdx.x; c < row_bytes / 16; c += 256) *(i32x4 *)(o + 16 * c) = *(const i32x4 *)(s + 16 * c);
}

int launch_rows_gather(const void *src, int64_t ld_src_bytes, const int64_t *idx, const int32_t *count,
                       int64_t n_max, int64_t row_bytes, void *dst, hipStream_t st) {
  if (n_max == 0) return OCTO_OK;
  if (row_bytes % 16 || ld_src_bytes % 16 || (uintptr_t)src % 16 || (uintptr_t)dst % 16)
    return octo_fail(OCTO_EINVAL, "rows_gather: rows must be 16-byte aligned");
  hipLaunchKernelGGL(rows_gather_kernel, dim3((unsigned)n_max), dim3(256), 0, st, (const char *)src, ld_src_bytes,
                     idx, count, n_max, row_bytes, (char *)dst);
  OCTO_CHECK_LAUNCH("rows_gather");
  return OCTO_OK;
}

__global__ __launch_bounds__(256) void rows_scatter_kernel(const void *src, int64_t ld_src, int src_dtype,
                                                           const int64_t *idx, const int32_t *count, int64_t n_max,
                                                           int d, void *dst, int64_t ld_dst, int dst_dtype,
                                                           int accumulate) {
  const int64_t r = blockIdx.x;
  const int64_t cnt = count ? min((int64_t)(*count), n_max) : n_max;
  if (r >= cnt) return;
  const int64_t row = idx[r];
  if (r > 0 && idx[r - 1] == row) return;
  int64_t e = r + 1;
  while (e < cnt && idx[e] == row) ++e;
  if (src_dtype == dst_dtype && (src_dtype == OCTO_BF16 || src_dtype == OCTO_F16) && d % 8 == 0 && ld_src % 8 == 0 &&
      ld_dst % 8 == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0) {  // 16-byte chunks
    const bool f16 = src_dtype == OCTO_F16;
    for (int k = threadIdx.x; k < d / 8; k += 256) {
      float s[8], x[8];
      if (accumulate) unpack8(*(const i32x4 *)((const char *)dst + (row * ld_dst + 8 * k) * 2), f16, s);
      else
#pragma unroll
        for (int u = 0; u < 8; ++u) s[u] = 0.f;
      for (int64_t q = r; q < e; ++q) {
        unpack8(*(const i32x4 *)((const char *)src + (q * ld_src + 8 * k) * 2), f16, x);
#pragma unroll
        for (int u = 0; u < 8; ++u) s[u] += x[u];
      }
      *(i32x4 *)((char *)dst + (row * ld_dst + 8 * k) * 2) = pack8(s, f16);
    }
    return;
  }
  for (int k = threadIdx.x; k < d; k += 256) {
    float s = accumulate ? load_as_f32(dst, dst_dtype, row * ld_dst + k) : 0.f;
    for (int64_t q = r; q < e; ++q) s += load_as_f32(src, src_dtype, q * ld_src + k);
    store_from_f32(dst, dst_dtype, row * ld_dst + k, s);
  }
}

__global__ void gather_f32_kernel(const float *src, int64_t ld, const int64_t *idx, const int32_t *count,
                                  int64_t n_max, float *out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_max) return;
  const int64_t cnt = count ? min((int64_t)(*count), n_max) : n_max;
  out[r] = (r < cnt) ? src[idx[r] * ld] : 0.f;
}

// ---- the bound GRPO step's fit of the incoming dL/dlogprob -------------------------------------------------------
// a[r], the incoming dL/dlogprob of compact row r: src[idx[r] ld] (src[r ld] without idx) for r below the count, 0
// past it; h[r], the step's own GRPO weight of row r. c = <a, h> / <h, h> (0 when h is 0) and rest = a - c h. The rest
// is negligible when ||rest|| <= tol ||a||: then *count_rest = 0 and *skip = 1, so the rest's backward ends at once,
// else *count_rest = the row count and *skip = 0. One workgroup; every sum in a fixed order, so equal inputs give
// equal bits.
__global__ __launch_bounds__(1024) void grpo_fit_kernel(const float *src, int64_t ld, const int64_t *idx,
                                                        const float *h, int64_t n, const int32_t *count, float tol,
                                                        float *c_out, float *rest, int32_t *count_rest,
                                                        int32_t *skip) {
  __shared__ float part[3][16];
  __shared__ float cs;
  const int64_t cnt = count ? min((int64_t)(*count), n) : n;
  const int w = threadIdx.x >> 6;
  float ah = 0.f, hh = 0.f, aa = 0.f;
  for (int64_t r = threadIdx.x; r < n; r += 1024) {
    const float a = r < cnt ? src[(idx ? idx[r] : r) * ld] : 0.f, g = h[r];
    ah = __builtin_fmaf(a, g, ah);
    hh = __builtin_fmaf(g, g, hh);
    aa = __builtin_fmaf(a, a, aa);
  }
  ah = wave_sum(ah);
  hh = wave_sum(hh);
  aa = wave_sum(aa);
  if ((threadIdx.x & 63) == 0) {
    part[0][w] = ah;
    part[1][w] = hh;
    part[2][w] = aa;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float s0 = 0.f, s1 = 0.f;
    for (int k = 0; k < 16; ++k) {
      s0 += part[0][k];
      s1 += part[1][k];
    }
    cs = s1 > 0.f ? s0 / s1 : 0.f;
  }
  __syncthreads();
  const float c = cs;
  float rr = 0.f;
  for (int64_t r = threadIdx.x; r < n; r += 1024) {
    const float a = r < cnt ? src[(idx ? idx[r] : r) * ld] : 0.f;
    const float x = a - c * h[r];
    rest[r] = x;
    rr = __builtin_fmaf(x, x, rr);
  }
  rr = wave_sum(rr);
  if ((threadIdx.x & 63) == 0) part[0][w] = rr;  // part[0] was last read by thread 0 before the barrier above
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f, a2 = 0.f;
    for (int k = 0; k < 16; ++k) {
      s += part[0][k];
      a2 += part[2][k];
    }
    const bool small = sqrtf(s) <= tol * sqrtf(a2);
    *c_out = c;
    *count_rest = small ? 0 : (int32_t)cnt;
    *skip = small ? 1 : 0;
  }
}

// ---- GRPO ----------------------------------------------------------------------------------------
// ws[0] = Z (masked-token count, at least 1); *loss zeroed. One workgroup.
__global__ __launch_bounds__(1024) void grpo_count_kernel(const float *mask, int64_t n, float *ws, float *loss) {
  __shared__ float part[16];
  float c = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) c += (mask[i] != 0.f) ? 1.f : 0.f;
  c = wave_sum(c);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    float z = 0.f;
    for (int k = 0; k < 16; ++k) z += part[k];
    ws[0] = fmaxf(z, 1.f);
    if (loss) *loss = 0.f;
  }
}

int launch_grpo_count(const float *mask, int64_t n, float *z, float *loss, hipStream_t st) {
  hipLaunchKernelGGL(grpo_count_kernel, dim3(1), dim3(1024), 0, st, mask, n, z, loss);
  OCTO_CHECK_LAUNCH("grpo_count");
  return OCTO_OK;
}

// The objective's term and dL/dlogp of one token with mask != 0 (logp lp; prox, old as pointers to its entries
// or NULL), both already divided by Z.
__device__ __forceinline__ void grpo_token(float lp, const float *prox, const float *old, float A, float eps_lo,
                                           float eps_hi, float reject_upper, float inv_z, float &gt, float &lt) {
  const float px = prox ? *prox : lp;
  const float r = expf(lp - px);
  float w = 1.f;
  if (old) {
    w = expf(px - *old);
    if (reject_upper > 0.f && w > reject_upper) w = 0.f;
  }
  const float lo = 1.f - eps_lo, hi = 1.f + eps_hi;
  const float cl = fminf(fmaxf(r, lo), hi);
  const float a = -A * r, b = -A * cl;
  const bool inside = (r >= lo) && (r <= hi);
  float ga, gb;
  if (a > b) { ga = 1.f; gb = 0.f; }
  else if (a < b) { ga = 0.f; gb = 1.f; }
  else { ga = 0.5f; gb = 0.5f; }
  const float dmax_dr = ga * (-A) + gb * (-A) * (inside ? 1.f : 0.f);
  gt = w * dmax_dr * r * inv_z;
  lt = w * fmaxf(a, b) * inv_z;
}

__global__ __launch_bounds__(256) void grpo_grad_kernel(const float *logp, const float *prox, const float *old,
                                                        const float *adv, const float *mask, int64_t n,
                                                        float eps_lo, float eps_hi, float reject_upper,
                                                        const float *ws, float *g, float *loss) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  float lt = 0.f;
  if (t < n) {
    float gt = 0.f;
    if (mask[t] != 0.f)
      grpo_token(logp[t], prox ? prox + t : nullptr, old ? old + t : nullptr, adv[t], eps_lo, eps_hi, reject_upper,
                 1.f / ws[0], gt, lt);
    g[t] = gt;
  }
  if (loss) {
    lt = wave_sum(lt);
    if ((threadIdx.x & 63) == 0 && lt != 0.f) atomicAdd(loss, lt);
  }
}

// ---- fp8 weight quantiser ---------------------------------------------------------------------------
// Per row: the absmax in fp32, scale = max(absmax / 448, 1e-12), then every element divided by the scale (IEEE
// fp32 division), clamped to +-448 and rounded to OCP e4m3, nearest even (v_cvt_pk_fp8_f32).
// General form (any d % 4 == 0): one workgroup per row, four elements per thread and step (8 or 16 bytes loaded,
// 4 bytes stored); the second sweep re-reads the row from cache.
template <int DT>
__device__ __forceinline__ f32x4 load4(const char *row, int k) {
  f32x4 x;
  if constexpr (DT == OCTO_F32) {
    x = *(const f32x4 *)(row + 4 * k);
  } else {
    typedef typename Elem<DT>::T T;
    typedef T T4 __attribute__((ext_vector_type(4)));
    const T4 v = *(const T4 *)(row + 2 * k);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (float)v[i];
  }
  return x;
}

template <int DT>
__global__ __launch_bounds__(256) void quantise_fp8_kernel(const char *w, int64_t ld_bytes, int d, uint8_t *q,
                                                           int64_t ldq, float *scale) {
  __shared__ float red[4];
  const int64_t v = blockIdx.x;
  const char *row = w + v * ld_bytes;
  float m = 0.f;
  for (int k = 4 * threadIdx.x; k < d; k += 1024) {
    const f32x4 x = load4<DT>(row, k);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3]))));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(m / 448.f, 1e-12f);
  uint8_t *qrow = q + v * ldq;
  for (int k = 4 * threadIdx.x; k < d; k += 1024) {
    const f32x4 x = load4<DT>(row, k);
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = fminf(fmaxf(x[i] / s, -448.f), 448.f);
    int packed = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    packed = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], packed, true);
    *(int *)(qrow + k) = packed;
  }
  if (threadIdx.x == 0) scale[v] = s;
}

// One wave per row, the row held in registers (d <= 4096, d % 8 == 0): lane l takes elements 512 c + 8 l .. + 8 of
// chunk c (16-byte loads of bf16 / f16, 2 x 16 for fp32), the absmax is a wave reduction, and the codes go out as
// 8 bytes per lane and chunk. Four rows per workgroup.
constexpr int QF8_MAXC = 8;
template <int DT>
__global__ __launch_bounds__(256) void quantise_fp8_rows_kernel(const char *w, int64_t ld_bytes, int64_t V, int d,
                                                                uint8_t *q, int64_t ldq, float *scale) {
  const int lane = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= V) return;
  const char *row = w + v * ld_bytes;
  float x[QF8_MAXC][8];
  float m = 0.f;
#pragma unroll
  for (int c = 0; c < QF8_MAXC; ++c) {
    const int k = c * 512 + lane * 8;
    if (k < d) {
      const f32x4 a = load4<DT>(row, k), b = load4<DT>(row, k + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[c][i] = a[i];
        x[c][4 + i] = b[i];
        m = fmaxf(m, fmaxf(fabsf(a[i]), fabsf(b[i])));
      }
    }
  }
  m = wave_max(m);
  const float s = fmaxf(m / 448.f, 1e-12f);
  uint8_t *qrow = q + v * ldq;
#pragma unroll
  for (int c = 0; c < QF8_MAXC; ++c) {
    const int k = c * 512 + lane * 8;
    if (k < d) {
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = fminf(fmaxf(x[c][i] / s, -448.f), 448.f);
      i32x2 o;
      o[0] = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
      o[0] = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], o[0], true);
      o[1] = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
      o[1] = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], o[1], true);
      *(i32x2 *)(qrow + k) = o;
    }
  }
  if (lane == 0) scale[v] = s;
}

}  // namespace octo

using namespace octo;

// ---- C ABI: small entry points -------------------------------------------------------------------
extern "C" {

int octo_compact_rows(const uint8_t *mask, int64_t n, int64_t *idx, int32_t *count, void *stream) {
  OCTO_CHECK_ARG(n >= 0, "compact_rows: n < 0");
  OCTO_CHECK_ARG(count != nullptr && (n == 0 || (mask && idx)), "compact_rows: null pointer");
  hipLaunchKernelGGL(compact_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, mask, n, idx, count);
  OCTO_CHECK_LAUNCH("compact_rows");
  return OCTO_OK;
}

int octo_columns_fwd(const void *logits, int64_t ld, int dtype, const int64_t *labels, int64_t n, int V,
                     float inv_T, float *out2, float *lse, void *stream) {
  OCTO_CHECK_ARG(n >= 0 && V > 0 && ld >= V, "columns_fwd: bad shape n=%lld V=%d ld=%lld", (long long)n, V, (long long)ld);
  OCTO_CHECK_ARG(dtype == OCTO_BF16 || dtype == OCTO_F16 || dtype == OCTO_F32, "columns_fwd: dtype %d", dtype);
  OCTO_CHECK_ARG(inv_T > 0.f, "columns_fwd: temperature must be positive");
  if (n == 0) return OCTO_OK;
  OCTO_CHECK_ARG(logits && labels && out2, "columns_fwd: null pointer");
  hipLaunchKernelGGL(columns_fwd_kernel, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream, logits, ld, dtype,
                     labels, V, inv_T, out2, lse);
  OCTO_CHECK_LAUNCH("columns_fwd");
  return OCTO_OK;
}

int octo_columns_bwd(const void *logits, int64_t ld, int dtype, const int64_t *labels, int64_t n, int V,
                     float inv_T, const float *lse, const float *g, void *dlogits, int64_t ld_d, void *stream) {
  OCTO_CHECK_ARG(n >= 0 && V > 0 && ld >= V && ld_d >= V, "columns_bwd: bad shape");
  OCTO_CHECK_ARG(dtype == OCTO_BF16 || dtype == OCTO_F16 || dtype == OCTO_F32, "columns_bwd: dtype %d", dtype);
  if (n == 0) return OCTO_OK;
  OCTO_CHECK_ARG(logits && labels && lse && g && dlogits, "columns_bwd: null pointer");
  OCTO_CHECK_ARG(n <= 65535, "columns_bwd: more than 65535 rows per call");
  dim3 grid((unsigned)cdiv(V, 256), (unsigned)n);
  hipLaunchKernelGGL(columns_bwd_kernel, grid, dim3(256), 0, (hipStream_t)stream, logits, ld, dtype, labels, V, inv_T,
                     lse, g, dlogits, ld_d);
  OCTO_CHECK_LAUNCH("columns_bwd");
  return OCTO_OK;
}

int octo_pairs_expand(const float *pairs, int64_t P, int C, const int64_t *flat_pair, int64_t T, float *out,
                      void *stream) {
  OCTO_CHECK_ARG(P >= 0 && C > 0 && T >= 0, "pairs_expand: bad shape");
  if (T == 0) return OCTO_OK;
  OCTO_CHECK_ARG(flat_pair && out && (P == 0 || pairs), "pairs_expand: null pointer");
  hipLaunchKernelGGL(pairs_expand_kernel, dim3((unsigned)cdiv(T * C, 256)), dim3(256), 0, (hipStream_t)stream, pairs, P,
                     C, flat_pair, T, out);
  OCTO_CHECK_LAUNCH("pairs_expand");
  return OCTO_OK;
}

int octo_pairs_grad(const float *grad_flat, int64_t T, int C, const int64_t *flat_pair, int64_t P,
                    float *grad_pairs, void *stream) {
  OCTO_CHECK_ARG(P >= 0 && C > 0 && T >= 0, "pairs_grad: bad shape");
  if (P > 0) {
    OCTO_CHECK_ARG(grad_pairs != nullptr, "pairs_grad: null pointer");
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)cdiv(P * C, 256)), dim3(256), 0, (hipStream_t)stream,
                       grad_pairs, P * C);
  }
  if (T > 0 && P > 0) {
    OCTO_CHECK_ARG(grad_flat && flat_pair, "pairs_grad: null pointer");
    hipLaunchKernelGGL(pairs_grad_kernel, dim3((unsigned)cdiv(T * C, 256)), dim3(256), 0, (hipStream_t)stream,
                       grad_flat, T, C, flat_pair, P, grad_pairs);
  }
  OCTO_CHECK_LAUNCH("pairs_grad");
  return OCTO_OK;
}

int octo_rows_scatter(const void *src, int64_t ld_src, int src_dtype, const int64_t *idx, const int32_t *count,
                      int64_t n_max, int d, void *dst, int64_t ld_dst, int dst_dtype, int accumulate, void *stream) {
  OCTO_CHECK_ARG(n_max >= 0 && d >= 0, "rows_scatter: bad shape");
  OCTO_CHECK_ARG(src_dtype == OCTO_BF16 || src_dtype == OCTO_F16 || src_dtype == OCTO_F32, "rows_scatter: src dtype");
  OCTO_CHECK_ARG(dst_dtype == OCTO_BF16 || dst_dtype == OCTO_F16 || dst_dtype == OCTO_F32, "rows_scatter: dst dtype");
  if (n_max == 0 || d == 0) return OCTO_OK;
  OCTO_CHECK_ARG(src && idx && dst, "rows_scatter: null pointer");
  OCTO_CHECK_ARG(n_max <= 0x7fffffff, "rows_scatter: too many rows");
  hipLaunchKernelGGL(rows_scatter_kernel, dim3((unsigned)n_max), dim3(256), 0, (hipStream_t)stream, src, ld_src,
                     src_dtype, idx, count, n_max, d, dst, ld_dst, dst_dtype, accumulate);
  OCTO_CHECK_LAUNCH("rows_scatter");
  return OCTO_OK;
}

int octo_scale_add(void *y, const void *x, int dtype, int64_t n, const float *c, const int32_t *skip_x,
                   void *stream) {
  OCTO_CHECK_ARG(n >= 0, "scale_add: n < 0");
  OCTO_CHECK_ARG(dtype == OCTO_BF16 || dtype == OCTO_F16 || dtype == OCTO_F32, "scale_add: dtype %d", dtype);
  if (n == 0) return OCTO_OK;
  OCTO_CHECK_ARG(y && c, "scale_add: null pointer");
  OCTO_CHECK_ARG(((uintptr_t)y) % 16 == 0 && ((uintptr_t)x) % 16 == 0, "scale_add: vectors must be 16-byte aligned");
  const int64_t chunks = n / (dtype == OCTO_F32 ? 4 : 8);
  const int64_t blocks = cdiv(chunks, 256);
  hipLaunchKernelGGL(scale_add_kernel, dim3((unsigned)(blocks < 1 ? 1 : (blocks > 2048 ? 2048 : blocks))), dim3(256),
                     0, (hipStream_t)stream, y, x, dtype, n, c, skip_x);
  OCTO_CHECK_LAUNCH("scale_add");
  return OCTO_OK;
}

int octo_grpo_fit(const float *src, int64_t ld_src, const int64_t *idx, const float *g_head, int64_t n,
                  const int32_t *count, float tol, float *c, float *rest, int32_t *count_rest, int32_t *skip,
                  void *stream) {
  OCTO_CHECK_ARG(n >= 0 && ld_src >= 1, "grpo_fit: bad shape");
  OCTO_CHECK_ARG(c && count_rest && skip && (n == 0 || (src && g_head && rest)), "grpo_fit: null pointer");
  hipLaunchKernelGGL(grpo_fit_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, src, ld_src, idx, g_head, n, count,
                     tol, c, rest, count_rest, skip);
  OCTO_CHECK_LAUNCH("grpo_fit");
  return OCTO_OK;
}

int octo_gather_f32(const float *src, int64_t ld_src, const int64_t *idx, const int32_t *count, int64_t n_max,
                    float *out, void *stream) {
  OCTO_CHECK_ARG(n_max >= 0, "gather_f32: bad shape");
  if (n_max == 0) return OCTO_OK;
  OCTO_CHECK_ARG(src && idx && out, "gather_f32: null pointer");
  hipLaunchKernelGGL(gather_f32_kernel, dim3((unsigned)cdiv(n_max, 256)), dim3(256), 0, (hipStream_t)stream, src,
                     ld_src, idx, count, n_max, out);
  OCTO_CHECK_LAUNCH("gather_f32");
  return OCTO_OK;
}

int octo_quantise_fp8_rows(const void *w, int64_t ldw, int w_dtype, int64_t V, int d, uint8_t *q, int64_t ldq,
                           float *scale, void *stream) {
  OCTO_CHECK_ARG(w_dtype == OCTO_BF16 || w_dtype == OCTO_F16 || w_dtype == OCTO_F32, "quantise_fp8: dtype %d",
                 w_dtype);
  OCTO_CHECK_ARG(V >= 0 && V <= 0x7fffffff && d >= 0 && d % 4 == 0 && ldw >= d && ldq >= d,
                 "quantise_fp8: bad shape V=%lld d=%d (d must be a multiple of 4)", (long long)V, d);
  if (V == 0) return OCTO_OK;
  OCTO_CHECK_ARG(w && q && scale, "quantise_fp8: null pointer");
  const int esz = w_dtype == OCTO_F32 ? 4 : 2;
  OCTO_CHECK_ARG((ldw * esz) % (4 * esz) == 0 && ((uintptr_t)w) % (4 * esz) == 0 && ldq % 4 == 0 &&
                     ((uintptr_t)q) % 4 == 0, "quantise_fp8: rows must be aligned to 4 elements");
  hipStream_t st = (hipStream_t)stream;
  const char *wc = (const char *)w;
  if (d % 8 == 0 && d <= QF8_MAXC * 512 && ldq % 8 == 0 && ((uintptr_t)q) % 8 == 0 && ldw % 8 == 0 &&
      ((uintptr_t)w) % 16 == 0) {  // one wave per row, the row in registers
    const dim3 g4((unsigned)cdiv(V, 4));
    switch (w_dtype) {
      case OCTO_BF16: hipLaunchKernelGGL(quantise_fp8_rows_kernel<OCTO_BF16>, g4, dim3(256), 0, st, wc, ldw * 2, V, d, q, ldq, scale); break;
      case OCTO_F16: hipLaunchKernelGGL(quantise_fp8_rows_kernel<OCTO_F16>, g4, dim3(256), 0, st, wc, ldw * 2, V, d, q, ldq, scale); break;
      default: hipLaunchKernelGGL(quantise_fp8_rows_kernel<OCTO_F32>, g4, dim3(256), 0, st, wc, ldw * 4, V, d, q, ldq, scale); break;
    }
    OCTO_CHECK_LAUNCH("quantise_fp8");
    return OCTO_OK;
  }
  const dim3 grid((unsigned)V);
  switch (w_dtype) {
    case OCTO_BF16: hipLaunchKernelGGL(quantise_fp8_kernel<OCTO_BF16>, grid, dim3(256), 0, st, wc, ldw * 2, d, q, ldq, scale); break;
    case OCTO_F16: hipLaunchKernelGGL(quantise_fp8_kernel<OCTO_F16>, grid, dim3(256), 0, st, wc, ldw * 2, d, q, ldq, scale); break;
    default: hipLaunchKernelGGL(quantise_fp8_kernel<OCTO_F32>, grid, dim3(256), 0, st, wc, ldw * 4, d, q, ldq, scale); break;
  }
  OCTO_CHECK_LAUNCH("quantise_fp8");
  return OCTO_OK;
}

int octo_grpo_workspace_bytes(size_t *bytes) {
  OCTO_CHECK_ARG(bytes != nullptr, "grpo_workspace_bytes: null pointer");
  *bytes = 256;
  return OCTO_OK;
}

int octo_grpo_grad(const float *logp, const float *prox, const float *old, const float *adv, const float *mask,
                   int64_t n, float eps_lo, float eps_hi, float reject_upper, float *g, float *loss, void *ws,
                   size_t ws_bytes, void *stream) {
  OCTO_CHECK_ARG(n >= 0, "grpo_grad: n < 0");
  if (ws_bytes < 256 || ws == nullptr) return octo_fail(OCTO_EWORKSPACE, "grpo_grad: workspace needs 256 bytes");
  OCTO_CHECK_ARG(n == 0 || (logp && adv && mask && g), "grpo_grad: null pointer");
  hipLaunchKernelGGL(grpo_count_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, mask, n, (float *)ws, loss);
  if (n > 0)
    hipLaunchKernelGGL(grpo_grad_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, logp, prox,
                       old, adv, mask, n, eps_lo, eps_hi, reject_upper, (const float *)ws, g, loss);
  OCTO_CHECK_LAUNCH("grpo_grad");
  return OCTO_OK;
}

}  // extern "C"
