// The MFMA GEMM core shared by every contraction of the LM-head path.
//
//   C[m, n] = sum_k A[m, k] * B[n, k]        (both operands K-contiguous, "NT")
//
// One workgroup = 256 threads = 4 wave64s computes a 256 x 256 tile of C; the waves sit 2 x 2 and
// each owns a 128 x 128 sub-tile as 4 x 4 accumulators of v_mfma_f32_32x32x16_{bf16,f16}
// (v_mfma_f32_32x32x2_f32 for fp32), i.e. all 256 accumulation registers of a wave.
//
// Two mainloops feed the MFMAs from LDS:
//   mainloop_dma  (every bf16 / f16 / f32 contraction): the A and B K-slices go straight from global memory
//                 into a ring of LDS stages by buffer_load_dwordx4 ... lds (no register hop), with the
//                 instruction order fixed in the source: fragment reads a sub-step ahead of their MFMAs and
//                 the DMA issues spread one per two MFMAs;
//   mainloop      (fp8 weights): register-staged, so that e4m3 bytes can be widened to bf16 on the way
//                 into LDS; K advances 128 bytes per step, double buffered (2 x 64 KB).
//
// Global loads are raw buffer loads: rows past the operand's end and K chunks past K read as zero
// (voffset >= 2^31 is out of range), so partial tiles need no branches in the loop. Operand rows can
// be gathered through a row map (compacted hidden rows), which fuses the reference's `index_select`
// into the GEMM.
//
// Workgroup -> tile: blocks are dealt to the 8 XCDs round-robin, so block b runs on XCD b % 8; each
// XCD walks its own M-tiles in groups of `group_m` across all N-tiles, so the ~32 workgroups resident
// on one XCD share a few A and B K-slices in that XCD's L2.
#pragma once

#include "octo_common.h"

namespace octo {

constexpr int TM = 256;          // tile rows (M)
constexpr int TN = 256;          // tile cols (N)
constexpr int KB = 128;          // K bytes per step
constexpr int NTHREADS = 256;
constexpr int TILE_BYTES = 256 * KB;  // one operand K-slice in LDS: 32 KB

typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) i32x4 lds_i32x4;

// One GEMM operand: logical row i of the operand is physical row map[i] (or i) of base.
struct Operand {
  const char *base;      // matrix base
  int64_t ld;            // row stride, bytes
  const int64_t *map;    // optional row map (logical -> physical row)
  int64_t rows;          // logical rows that exist (rows >= this read as zero)
  const int32_t *count;  // optional device bound on logical rows (min with rows)
  int64_t count_off;     // logical row 0 corresponds to count index count_off
  uint32_t extent;       // bytes addressable from base when map != NULL
};

struct GemmShape {
  int64_t M, N;         // logical sizes (tile grid)
  int64_t K;            // contraction length in elements of the staged (MFMA) type
  int mtiles, ntiles, group_m;
  int count_on;         // 0: none; 1: count bounds M; 2: count bounds N; 3: count bounds K
  const int32_t *count; // device row count (with count_off)
  int64_t count_off;
};

// Block -> (mt, nt). Blocks run on XCD b % 8. M-tiles are dealt to the XCDs round-robin (XCD x owns
// mt = x, x + 8, ...), so a device-side count that idles a suffix of M-tiles idles them evenly on every
// XCD; each XCD walks its own M-tiles in groups of group_m across all N-tiles, so the ~32 workgroups
// resident on an XCD share a few A and B K-slices in its L2. The grid is 8 * (tiles of the largest
// XCD); blocks past their XCD's tiles return false.
__host__ __device__ inline int64_t tile_grid(int mtiles, int ntiles) {
  return 8 * ((int64_t)((mtiles + 7) / 8) * ntiles);
}
__device__ __forceinline__ bool tile_of(const GemmShape &s, int &mt, int &nt) {
  const int64_t b = blockIdx.x;
  const int x = (int)(b & 7);
  const int64_t k = b >> 3;
  const int64_t mx = (s.mtiles - x + 7) / 8;  // M-tiles owned by XCD x
  if (k >= mx * s.ntiles) return false;
  const int64_t span = (int64_t)s.group_m * s.ntiles;
  const int64_t gid = k / span;
  const int64_t first = gid * s.group_m;
  const int64_t gsize = (mx - first) < s.group_m ? (mx - first) : s.group_m;
  const int64_t local = k - gid * span;
  mt = (int)(x + 8 * (first + local % gsize));
  nt = (int)(local / gsize);
  return true;
}

template <int DT> struct Mfma;
template <> struct Mfma<OCTO_BF16> {
  static __device__ __forceinline__ void run(const i32x4 a, const i32x4 b, f32x16 &c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<OCTO_F16> {
  static __device__ __forceinline__ void run(const i32x4 a, const i32x4 b, f32x16 &c) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<OCTO_F32> {
  // a 16-byte fragment holds 4 fp32 K values: four 32x32x2 steps, lane half h supplies k = 4h + e
  static __device__ __forceinline__ void run(const i32x4 a, const i32x4 b, f32x16 &c) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(__int_as_float(a[e]), __int_as_float(b[e]), c, 0, 0, 0);
  }
};

// 8 OCP e4m3 bytes -> 8 bf16 (exact), as one 16-byte chunk.
__device__ __forceinline__ i32x4 fp8x8_to_bf16x8(i32x2 q) {
  i32x4 o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t w = (uint32_t)q[h];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      float lo = e4m3_to_f32((w >> (16 * p)) & 0xffu);
      float hi = e4m3_to_f32((w >> (16 * p + 8)) & 0xffu);
      // fp32 -> bf16 is exact here (3 mantissa bits): keep the top 16 bits
      o[2 * h + p] = (int)((__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u));
    }
  }
  return o;
}

__device__ __forceinline__ const char *uniform_ptr(const char *p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const char *)(((uint64_t)hi << 32) | lo);
}

// Buffer resource and per-thread row offsets of one operand tile (rows row0 .. row0 + 255); the
// thread loads rows (t >> 3) + 32 q, q = 0..7, at 16-byte chunk t & 7 of each K step.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t operand_rows(const Operand &op, int64_t row0, uint32_t (&off)[8]) {
  const int t = threadIdx.x;
  const int64_t valid = dev_count(op.count, op.count_off + row0, op.rows - row0);
  if (op.map) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int r = (t >> 3) + 32 * q;
      off[q] = (r < valid) ? (uint32_t)(op.map[row0 + r] * op.ld) : 0x80000000u;
    }
    return make_rsrc(uniform_ptr(op.base), op.extent);
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int r = (t >> 3) + 32 * q;
    off[q] = (r < valid) ? (uint32_t)(r * op.ld) : 0x80000000u;
  }
  return make_rsrc(uniform_ptr(op.base + row0 * op.ld), (uint32_t)(256 * op.ld));
}

// Stage one K step (kb = its first byte in a source row) into regs. A chunk past the row's K bytes
// (kbytes) reads zero. FP8: the source holds 1 byte per element, widened to bf16.
template <bool FP8>
__device__ __forceinline__ void load_step(__amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[8], uint32_t kb,
                                          uint32_t kbytes, i32x4 (&reg)[8]) {
  const int c = threadIdx.x & 7;
  constexpr uint32_t CH = FP8 ? 8 : 16;
  const uint32_t kc = kb + c * CH;
  const uint32_t dead = (kc < kbytes) ? 0u : 0x80000000u;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint32_t o = (off[q] | dead) + kc;
    if constexpr (FP8) reg[q] = fp8x8_to_bf16x8(buf_load8(rs, (int)o));
    else reg[q] = buf_load16(rs, (int)o);
  }
}

__device__ __forceinline__ void lds_store_slice(lds_char *buf, const i32x4 (&reg)[8]) {
  const int t = threadIdx.x;
  const int r = t >> 3, c = t & 7;
  lds_char *p = buf + r * KB + ((c ^ (r & 7)) << 4);
#pragma unroll
  for (int q = 0; q < 8; ++q) *(lds_i32x4 *)(p + q * 32 * KB) = reg[q];
}

// The mainloop. acc[i][j] is the 32x32 block (wm*128 + 32 i, wn*128 + 32 j) of the tile.
// smem: SMEM_BYTES of LDS: [A0 | B0 | A1 | B1].
template <int DT, bool A_FP8>
__device__ __forceinline__ void mainloop(const Operand &A, const Operand &B, int64_t m0, int64_t n0, int64_t K_eff,
                                         lds_char *smem, f32x16 (&acc)[4][4]) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  constexpr int ebytes = (DT == OCTO_F32) ? 4 : 2;
  const uint32_t kbytes = (uint32_t)(K_eff * ebytes);               // staged bytes per row
  const uint32_t kbytes_a = A_FP8 ? (uint32_t)K_eff : kbytes;        // source bytes per A row
  const int nkt = (int)((kbytes + KB - 1) / KB);
  if (nkt == 0) return;
  constexpr uint32_t KBA = A_FP8 ? KB / 2 : KB;                      // source bytes per A step

  uint32_t offa[8], offb[8];
  const __amdgpu_buffer_rsrc_t rsa = operand_rows(A, m0, offa);
  const __amdgpu_buffer_rsrc_t rsb = operand_rows(B, n0, offb);

  // fragment byte offsets within a K-slice: row = base + (lane & 31), chunk = 2 ks + (lane >> 5)
  int aoff[4], boff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int pc = ((2 * ks + (lane >> 5)) ^ (lane & 7)) << 4;
    aoff[ks] = (wm * 128 + (lane & 31)) * KB + pc;
    boff[ks] = TILE_BYTES + (wn * 128 + (lane & 31)) * KB + pc;
  }

  i32x4 ra[8], rb[8];
  load_step<A_FP8>(rsa, offa, 0, kbytes_a, ra);
  load_step<false>(rsb, offb, 0, kbytes, rb);
  lds_store_slice(smem, ra);
  lds_store_slice(smem + TILE_BYTES, rb);
  __syncthreads();

  for (int kt = 0; kt < nkt; ++kt) {
    const int cur = (kt & 1) * (2 * TILE_BYTES);
    const bool more = kt + 1 < nkt;
    if (more) {
      load_step<A_FP8>(rsa, offa, (uint32_t)(kt + 1) * KBA, kbytes_a, ra);
      load_step<false>(rsb, offb, (uint32_t)(kt + 1) * KB, kbytes, rb);
    }
    const lds_char *s = smem + cur;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      i32x4 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = *(const lds_i32x4 *)(s + aoff[ks] + i * 32 * KB);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = *(const lds_i32x4 *)(s + boff[ks] + j * 32 * KB);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) Mfma<DT>::run(af[i], bfr[j], acc[i][j]);
    }
    if (more) {
      lds_char *nxt = smem + (2 * TILE_BYTES - cur);
      lds_store_slice(nxt, ra);
      lds_store_slice(nxt + TILE_BYTES, rb);
    }
    __syncthreads();
  }
}

// ---- direct-to-LDS mainloop -----------------------------------------------------------------------
//
// K advances DKB bytes per stage (64: 32 bf16 / 16 fp32; 128: 64 bf16 / 32 fp32). The A and B slices of a
// stage (256 rows x DKB bytes each) are written straight into LDS by buffer_load_dwordx4 ... lds: each
// wave instruction moves 1 KB, lane i's 16 bytes landing at the instruction's LDS base + 16 i, so the LDS
// layout is chosen by which global chunk each lane fetches (64 / (DKB / 16) whole rows per instruction).
// DNSTAGE stages form a ring; the DMA for stage k + DNSTAGE is issued in iteration k, DNSTAGE - 1 stages
// ahead of its use. One bare s_barrier per stage (no memory fence: the waits are explicit) separates
// "stage k + 1 landed in every wave" and "every wave has read stage k" from the DMA that overwrites stage
// k's buffer.
//
// LDS rows are DKB bytes of 16-byte chunks; chunk c of row r sits at physical chunk c ^ swz(r), which keeps
// the fragment reads of consecutive lanes (consecutive rows, same logical chunk) on distinct bank groups.
#ifndef OCTO_DKB
#define OCTO_DKB 64
#endif
constexpr int DKB = OCTO_DKB;              // K bytes per stage
constexpr int DSTAGE = 2 * 256 * DKB;      // A + B bytes per stage
#ifndef OCTO_NSTAGE
#define OCTO_NSTAGE (DKB == 64 ? 4 : 2)
#endif
constexpr int DNSTAGE = OCTO_NSTAGE;       // ring depth
constexpr int DLPR = DKB / 16;             // lanes per row in one DMA instruction
constexpr int DRPI = 64 / DLPR;            // rows per DMA instruction
constexpr int DIPW = 256 / DRPI / 4;       // DMA instructions per wave per operand and stage
constexpr int DNSUB = DKB / 32;            // 16-byte-fragment sub-steps per stage
// LDS of one GEMM workgroup: the register-staged mainloop's 2 x (A + B) 32 KB slices or the DMA ring.
constexpr int SMEM_BYTES = (4 * TILE_BYTES > DNSTAGE * DSTAGE) ? 4 * TILE_BYTES : DNSTAGE * DSTAGE;
static_assert(DKB == 64 || DKB == 128, "stage width");
static_assert(SMEM_BYTES <= 160 * 1024, "LDS budget");

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] + vmcnt[5:4] at bits 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int WAIT_LGKM0 = 15 | (3 << 14) | (7 << 4);
static_assert(2 * DIPW * DNSTAGE <= 63, "vmcnt range");

// 64-byte rows: chunk c of row r at c ^ ((r >> 2) & 3), so the 8 lanes of a 128-byte LDS access (rows r0..r0+7
// of one logical chunk: two rows per physical chunk index) cover all four chunk positions twice in two
// different 64-byte halves of the bank space; 128-byte rows: c ^ (r & 7).
__device__ __forceinline__ int swz_row(int r) {
  if (DKB == 128) return r & 7;
  return (r >> 2) & 3;
}

// Per-thread DMA sources of one operand: instruction q (0..DIPW-1) of wave w fills LDS rows
// (4 q + w) * DRPI .. + DRPI; lane i takes row + i / DLPR and physical chunk i % DLPR.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_rows(const Operand &op, int64_t row0, uint32_t (&off)[DIPW],
                                                           uint32_t (&coff)[DIPW]) {
  const int w = threadIdx.x >> 6, i = threadIdx.x & 63;
  const int64_t valid = dev_count(op.count, op.count_off + row0, op.rows - row0);
#pragma unroll
  for (int q = 0; q < DIPW; ++q) {
    const int r = (4 * q + w) * DRPI + i / DLPR;
    coff[q] = (uint32_t)(((i % DLPR) ^ swz_row(r)) << 4);
    uint32_t rowoff;
    if (r < valid) rowoff = op.map ? (uint32_t)(op.map[row0 + r] * op.ld) : (uint32_t)(r * op.ld);
    else rowoff = 0x80000000u;
    off[q] = rowoff + coff[q];
  }
  if (op.map) return make_rsrc(uniform_ptr(op.base), op.extent);
  return make_rsrc(uniform_ptr(op.base + row0 * op.ld), (uint32_t)(256 * op.ld));
}

__device__ __forceinline__ void dma_stage(__amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[DIPW],
                                          const uint32_t (&coff)[DIPW], uint32_t kb, uint32_t kbytes,
                                          lds_char *dst) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int q = 0; q < DIPW; ++q) {
    const uint32_t o = (kb + coff[q] < kbytes) ? off[q] + kb : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(dst + (4 * q + w) * 1024),
                                             16, o, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ void mfma_block(const i32x4 (&af)[4], const i32x4 (&bf)[4], f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) Mfma<DT>::run(af[i], bf[j], acc[i][j]);
}

__device__ __forceinline__ void read_frags(const lds_char *s, int aoff, int boff, i32x4 (&af)[4], i32x4 (&bf)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) af[i] = *(const lds_i32x4 *)(s + aoff + i * 32 * DKB);
#pragma unroll
  for (int j = 0; j < 4; ++j) bf[j] = *(const lds_i32x4 *)(s + boff + j * 32 * DKB);
}

// Fragment q (0..7) of a sub-step: A block q (q < 4) or B block q - 4.
__device__ __forceinline__ void read_frag(const lds_char *s, int aoff, int boff, int q, i32x4 (&af)[4],
                                          i32x4 (&bf)[4]) {
  if (q < 4) af[q] = *(const lds_i32x4 *)(s + aoff + q * 32 * DKB);
  else bf[q - 4] = *(const lds_i32x4 *)(s + boff + (q - 4) * 32 * DKB);
}

// One DMA instruction q (0..DIPW-1) of an operand slice (see dma_stage).
__device__ __forceinline__ void dma_one(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t coff, uint32_t kb,
                                        uint32_t kbytes, lds_char *dst, int q) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t o = (kb + coff < kbytes) ? off + kb : 0x80000000u;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(dst + (4 * q + w) * 1024),
                                           16, o, 0, 0, 0);
}

// Instruction order is fixed in the source: a scheduling fence after every MFMA / load keeps the fragment
// reads of the next sub-step early (so register allocation cannot fold them onto fragments still in use)
// and spreads the DMA issues evenly between MFMAs.
#define OCTO_FENCE() __builtin_amdgcn_sched_barrier(0)

// smem: DNSTAGE * DSTAGE bytes; stage s at s * DSTAGE, A rows first then B rows.
//
// Stage j's A slice is issued right after the barrier that frees its slot (in iteration j - DNSTAGE), its
// B slice under the first sub-step of the next iteration (into the slot stage j - DNSTAGE left), so the
// 2 * DIPW DMA instructions of a stage are spread over two sub-steps. With a ring of 2 both slices go
// after the barrier.
template <int DT>
__device__ __forceinline__ void mainloop_dma(const Operand &A, const Operand &B, int64_t m0, int64_t n0, int64_t K_eff,
                                             lds_char *smem, f32x16 (&acc)[4][4]) {
  constexpr bool SPLIT = DNSTAGE >= 3;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  constexpr int ebytes = (DT == OCTO_F32) ? 4 : 2;
  const uint32_t kbytes = (uint32_t)(K_eff * ebytes);
  const int nk = (int)((kbytes + DKB - 1) / DKB);
  if (nk == 0) return;

  uint32_t offa[DIPW], offb[DIPW], ca[DIPW], cb[DIPW];
  const __amdgpu_buffer_rsrc_t rsa = dma_rows(A, m0, offa, ca);
  const __amdgpu_buffer_rsrc_t rsb = dma_rows(B, n0, offb, cb);

  const int f = swz_row(lane);
  int aoff[DNSUB], boff[DNSUB];
#pragma unroll
  for (int ks = 0; ks < DNSUB; ++ks) {
    const int pc = ((2 * ks + (lane >> 5)) ^ f) << 4;
    aoff[ks] = (wm * 128 + (lane & 31)) * DKB + pc;
    boff[ks] = 256 * DKB + (wn * 128 + (lane & 31)) * DKB + pc;
  }

  if constexpr (SPLIT) {
#pragma unroll
    for (int s = 0; s < DNSTAGE - 1; ++s) {
      dma_stage(rsa, offa, ca, (uint32_t)s * DKB, kbytes, smem + s * DSTAGE);
      dma_stage(rsb, offb, cb, (uint32_t)s * DKB, kbytes, smem + s * DSTAGE + 256 * DKB);
    }
    dma_stage(rsa, offa, ca, (uint32_t)(DNSTAGE - 1) * DKB, kbytes, smem + (DNSTAGE - 1) * DSTAGE);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * DIPW * (DNSTAGE - 2) + DIPW));
  } else {
#pragma unroll
    for (int s = 0; s < DNSTAGE; ++s) {
      dma_stage(rsa, offa, ca, (uint32_t)s * DKB, kbytes, smem + s * DSTAGE);
      dma_stage(rsb, offb, cb, (uint32_t)s * DKB, kbytes, smem + s * DSTAGE + 256 * DKB);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * DIPW * (DNSTAGE - 1)));
  }
  __builtin_amdgcn_s_barrier();

  i32x4 fa[2][4], fb[2][4];
  read_frags(smem, aoff[0], boff[0], fa[0], fb[0]);
  int slot = 0;                 // k % DNSTAGE
  int prev_slot = DNSTAGE - 1;  // (k - 1) % DNSTAGE
  for (int k = 0; k < nk; ++k) {
    const int next_slot = (slot + 1 == DNSTAGE) ? 0 : slot + 1;
    const lds_char *cur = smem + slot * DSTAGE;
    OCTO_FENCE();
    // sub-steps 0 .. DNSUB - 2: read the next sub-step's fragments under the first 8 MFMAs
#pragma unroll
    for (int sub = 0; sub + 1 < DNSUB; ++sub) {
      const uint32_t kbB = (uint32_t)(k + DNSTAGE - 1) * DKB;
      lds_char *dstB = smem + prev_slot * DSTAGE + 256 * DKB;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        Mfma<DT>::run(fa[sub & 1][q >> 2], fb[sub & 1][q & 3], acc[q >> 2][q & 3]);
        OCTO_FENCE();
        if (q < 8) {
          read_frag(cur, aoff[sub + 1], boff[sub + 1], q, fa[(sub + 1) & 1], fb[(sub + 1) & 1]);
          OCTO_FENCE();
        } else if (SPLIT && sub == 0) {
          // B slice of stage k + DNSTAGE - 1, DIPW instructions over MFMAs 8..15
          constexpr int every = 8 / DIPW;
          if ((q - 8) % every == every - 1) {
            const int d = (q - 8) / every;
            dma_one(rsb, offb[d], cb[d], kbB, kbytes, dstB, d);
            OCTO_FENCE();
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);                                // this wave's reads of stage k are done
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * DIPW * (DNSTAGE - 2)));     // stage k + 1 landed (this wave's part)
    __builtin_amdgcn_s_barrier();                                          // ... in every wave; stage k is free
    OCTO_FENCE();
    // last sub-step: read the next stage's first fragments under the first 8 MFMAs, refill stage k's
    // buffer (stage k + DNSTAGE) under the last 8
    lds_char *refill = smem + slot * DSTAGE;
    const uint32_t kb = (uint32_t)(k + DNSTAGE) * DKB;
    const lds_char *nxt = smem + next_slot * DSTAGE;
    constexpr int LASTF = (DNSUB - 1) & 1;
    constexpr int NV = SPLIT ? DIPW : 2 * DIPW;  // DMA instructions under the last sub-step
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      Mfma<DT>::run(fa[LASTF][q >> 2], fb[LASTF][q & 3], acc[q >> 2][q & 3]);
      OCTO_FENCE();
      if (q < 8) {
        read_frag(nxt, aoff[0], boff[0], q, fa[0], fb[0]);
        OCTO_FENCE();
      } else {
        // NV DMA instructions over MFMAs 8..15: A slice first, then (ring of 2) the B slice
#pragma unroll
        for (int d = (q - 8) * NV / 8; d < (q - 7) * NV / 8; ++d) {
          if (d < DIPW) dma_one(rsa, offa[d], ca[d], kb, kbytes, refill, d);
          else dma_one(rsb, offb[d - DIPW], cb[d - DIPW], kb, kbytes, refill + 256 * DKB, d - DIPW);
          OCTO_FENCE();
        }
      }
    }
    prev_slot = slot;
    slot = next_slot;
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0) & WAIT_LGKM0);
  __builtin_amdgcn_s_barrier();
}

// Row (M) and column (N) of accumulator element v of block (i, j), relative to the tile origin.
__device__ __forceinline__ int acc_row(int wm, int i, int v, int lane) {
  return wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}
__device__ __forceinline__ int acc_col(int wn, int j, int lane) { return wn * 128 + j * 32 + (lane & 31); }

}  // namespace octo
