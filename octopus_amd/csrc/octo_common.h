// Shared device helpers for the gfx950 LM-head kernels: vector types, buffer-resource loads,
// bf16/fp8 conversions, wave reductions and the host-side status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/octo_head.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

#define OCTO_LOG2E 1.4426950408889634f
#define OCTO_LN2 0.6931471805599453f

// Buffer resource word 3 for raw (untyped, stride 0) buffers on gfx9-family parts.
#define OCTO_RSRC_WORD3 0x00020000

// A voffset at or above num_records makes a raw buffer load return zeros.
#define OCTO_OOB 0x7fffffff

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, OCTO_RSRC_WORD3);
}

__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
}
__device__ __forceinline__ i32x2 buf_load8(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
}

// ---- element conversions ----------------------------------------------------------------------
template <int DT> struct Elem;
template <> struct Elem<OCTO_BF16> { typedef __bf16 T; static constexpr int bytes = 2; };
template <> struct Elem<OCTO_F16> { typedef _Float16 T; static constexpr int bytes = 2; };
template <> struct Elem<OCTO_F32> { typedef float T; static constexpr int bytes = 4; };

template <int DT> __device__ __forceinline__ float to_f32(typename Elem<DT>::T x) { return (float)x; }

template <int DT> __device__ __forceinline__ typename Elem<DT>::T from_f32(float x) {
  return (typename Elem<DT>::T)x;  // round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
}

__device__ __forceinline__ float load_as_f32(const void *p, int dt, int64_t i) {
  if (dt == OCTO_BF16) return (float)((const __bf16 *)p)[i];
  if (dt == OCTO_F16) return (float)((const _Float16 *)p)[i];
  return ((const float *)p)[i];
}
__device__ __forceinline__ void store_from_f32(void *p, int dt, int64_t i, float x) {
  if (dt == OCTO_BF16) ((__bf16 *)p)[i] = (__bf16)x;
  else if (dt == OCTO_F16) ((_Float16 *)p)[i] = (_Float16)x;
  else ((float *)p)[i] = x;
}

// OCP e4m3 (bias 7, no infinities, S.1111.111 = NaN) to fp32, from the bit pattern. Every e4m3
// value is exactly representable in bf16 and fp32.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  uint32_t s = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xfu;
  uint32_t m = b & 0x7u;
  float mag;
  if (e == 0) mag = (float)m * 0.001953125f;  // m * 2^-9 (subnormal)
  else if (e == 15 && m == 7) mag = __builtin_nanf("");
  else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(mag) | s);
}

// ---- fast math (hardware v_exp_f32 / v_log_f32, base 2) ---------------------------------------
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }

// ---- wave64 reductions ------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Online softmax statistics in base-2 units: for values t_j (already * log2 e),
//   m = max t_j, S = sum 2^(t_j - m), U = sum 2^(t_j - m) (t_j - m).
// Merging two partials keeps the same meaning over the union.
struct Stat3 {
  float m, S, U;
};
__device__ __forceinline__ Stat3 stat_merge(Stat3 a, Stat3 b) {
  if (a.S == 0.f) return b;
  if (b.S == 0.f) return a;
  float m = fmaxf(a.m, b.m);
  float da = a.m - m, db = b.m - m;
  float ea = fexp2(da), eb = fexp2(db);
  Stat3 r;
  r.m = m;
  r.S = a.S * ea + b.S * eb;
  r.U = ea * (a.U + da * a.S) + eb * (b.U + db * b.S);
  return r;
}
__device__ __forceinline__ Stat3 wave_stat_merge(Stat3 s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    Stat3 t;
    t.m = __shfl_xor(s.m, o, 64);
    t.S = __shfl_xor(s.S, o, 64);
    t.U = __shfl_xor(s.U, o, 64);
    s = stat_merge(s, t);
  }
  return s;
}

// Post-head transform of a raw logit z, in base-2 softmax units: t = z' * inv_T * log2 e, with
// z' = post * tanh(pre * z) (softcap) or post * pre * z.
struct PostXf {
  float c;      // linear: pre * post * inv_T * log2e ; tanh: post * inv_T * log2e
  float pre;    // tanh argument scale
  int use_tanh;
};
__device__ __forceinline__ float ftanh(float x) {
  // tanh(x) = 1 - 2 / (exp(2x) + 1), saturating cleanly for large |x|
  float e = fexp2(2.f * OCTO_LOG2E * x);
  return 1.f - 2.f / (e + 1.f);
}

// Rows of a logical range [off, off + cap) that lie below a device-held count (all cap when none).
__device__ __forceinline__ int64_t dev_count(const int32_t *count, int64_t off, int64_t cap) {
  if (!count) return cap;
  int64_t c = (int64_t)(*count) - off;
  return c < 0 ? 0 : (c > cap ? cap : c);
}

// ---- host-side status plumbing ----------------------------------------------------------------
void octo_set_error(const char *fmt, ...);
int octo_fail(int code, const char *fmt, ...);

#define OCTO_CHECK_ARG(cond, ...)                                  \
  do {                                                             \
    if (!(cond)) return octo_fail(OCTO_EINVAL, __VA_ARGS__);       \
  } while (0)

#define OCTO_CHECK_LAUNCH(what)                                                        \
  do {                                                                                 \
    hipError_t e_ = hipGetLastError();                                                 \
    if (e_ != hipSuccess) return octo_fail(OCTO_EHIP, "%s: %s", what, hipGetErrorString(e_)); \
  } while (0)

__host__ __device__ static inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
__host__ __device__ static inline int64_t cdiv(int64_t x, int64_t m) { return (x + m - 1) / m; }
