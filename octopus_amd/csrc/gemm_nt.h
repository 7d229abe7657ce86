// The MFMA GEMM core shared by every contraction of the LM-head path.
//
//   C[m, n] = sum_k A[m, k] * B[n, k]        (both operands K-contiguous, "NT")
//
// One workgroup = 256 threads = 4 wave64s computes a 256 x 256 tile of C; the waves sit 2 x 2 and
// each owns a 128 x 128 sub-tile as 4 x 4 accumulators of v_mfma_f32_32x32x16_{bf16,f16}
// (v_mfma_f32_32x32x2_f32 for fp32). K advances 128 bytes per step (64 bf16 / 32 fp32); the
// A and B K-slices are staged through LDS, double buffered (2 x 64 KB), with the 16-byte chunks of
// each 128-byte LDS row XOR-swizzled by (row & 7) so that the fragment reads of 8 consecutive lanes
// (8 consecutive rows, same logical chunk) land on 8 distinct bank groups.
//
// Global loads are raw buffer loads: rows past the operand's end and K chunks past K read as zero
// (voffset >= 2^31 is out of range), so partial tiles need no branches in the loop. Operand rows can
// be gathered through a row map (compacted hidden rows), which fuses the reference's `index_select`
// into the GEMM.
//
// Workgroup -> tile: blocks are dealt to the 8 XCDs round-robin, so block b runs on XCD b % 8; each
// XCD gets a contiguous range of the tile order, and the tile order walks groups of `group_m`
// M-tiles across all N-tiles, so the ~32 workgroups resident on one XCD share a few A and B
// K-slices in that XCD's L2.
#pragma once

#include "octo_common.h"

namespace octo {

constexpr int TM = 256;          // tile rows (M)
constexpr int TN = 256;          // tile cols (N)
constexpr int KB = 128;          // K bytes per step
constexpr int NTHREADS = 256;
constexpr int TILE_BYTES = 256 * KB;  // one operand K-slice in LDS: 32 KB
constexpr int SMEM_BYTES = 4 * TILE_BYTES;

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
// K advances 64 bytes per stage (32 bf16 / 16 fp32). The A and B slices of a stage (256 rows x 64 B each,
// 32 KB together) are written straight into LDS by buffer_load_dwordx4 ... lds: each wave instruction
// moves 1 KB, lane i's 16 bytes landing at the instruction's LDS base + 16 i, so the LDS layout is chosen
// by which global chunk each lane fetches. Four stages form a ring (128 KB); the DMA for stage k + 4 is
// issued in iteration k, three stages ahead of its use, so global latency is covered by ~3 stages of MFMA
// work. One bare s_barrier per stage (no memory fence: the waits are explicit) separates "stage k + 1
// landed in every wave" and "every wave has read stage k" from the DMA that overwrites stage k's buffer.
//
// LDS row layout (64-byte rows, 4 chunks of 16 bytes): chunk c of row r sits at physical chunk
// c ^ f(r), f(r) = ((r >> 1) ^ (r >> 3)) & 3, which keeps the fragment reads of 8 consecutive lanes
// (rows r..r+7, same c) on distinct 16-byte bank groups of a 128-byte bank window and those of 16
// consecutive lanes distinct within a 256-byte window.
constexpr int DKB = 64;                    // K bytes per stage
constexpr int DSTAGE = 2 * 256 * DKB;      // A + B bytes per stage (32 KB)
constexpr int DNSTAGE = 4;

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] + vmcnt[5:4] at bits 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int WAIT_LGKM0 = 15 | (3 << 14) | (7 << 4);

#ifndef OCTO_SWZ
#define OCTO_SWZ 2
#endif
__device__ __forceinline__ int swz64(int r) {
  if (OCTO_SWZ == 1) return (r >> 1) & 3;
  if (OCTO_SWZ == 2) return (r >> 2) & 3;
  if (OCTO_SWZ == 3) return 0;
  return ((r >> 1) ^ (r >> 3)) & 3;
}

// Per-thread DMA sources of one operand: instruction q (0..3) of wave w fills LDS rows
// (4 q + w) * 16 .. +16; lane i takes row + (i >> 2) and physical chunk i & 3.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_rows(const Operand &op, int64_t row0, uint32_t (&off)[4],
                                                           uint32_t (&coff)[4]) {
  const int w = threadIdx.x >> 6, i = threadIdx.x & 63;
  const int64_t valid = dev_count(op.count, op.count_off + row0, op.rows - row0);
  uint32_t rowoff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = (4 * q + w) * 16 + (i >> 2);
    coff[q] = (uint32_t)(((i & 3) ^ swz64(r)) << 4);
    if (r < valid) rowoff[q] = op.map ? (uint32_t)(op.map[row0 + r] * op.ld) : (uint32_t)(r * op.ld);
    else rowoff[q] = 0x80000000u;
    off[q] = rowoff[q] + coff[q];
  }
  if (op.map) return make_rsrc(uniform_ptr(op.base), op.extent);
  return make_rsrc(uniform_ptr(op.base + row0 * op.ld), (uint32_t)(256 * op.ld));
}

__device__ __forceinline__ void dma_stage(__amdgpu_buffer_rsrc_t rs, const uint32_t (&off)[4],
                                          const uint32_t (&coff)[4], uint32_t kb, uint32_t kbytes,
                                          lds_char *dst) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
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

// smem: DNSTAGE * DSTAGE bytes; stage s at s * DSTAGE, A rows first then B rows.
template <int DT>
__device__ __forceinline__ void mainloop_dma(const Operand &A, const Operand &B, int64_t m0, int64_t n0, int64_t K_eff,
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
  const uint32_t kbytes = (uint32_t)(K_eff * ebytes);
  const int nk = (int)((kbytes + DKB - 1) / DKB);
  if (nk == 0) return;

  uint32_t offa[4], offb[4], ca[4], cb[4];
  const __amdgpu_buffer_rsrc_t rsa = dma_rows(A, m0, offa, ca);
  const __amdgpu_buffer_rsrc_t rsb = dma_rows(B, n0, offb, cb);

  const int f = swz64(lane);
  int aoff[2], boff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int pc = ((2 * ks + (lane >> 5)) ^ f) << 4;
    aoff[ks] = (wm * 128 + (lane & 31)) * DKB + pc;
    boff[ks] = 256 * DKB + (wn * 128 + (lane & 31)) * DKB + pc;
  }

#pragma unroll
  for (int s = 0; s < DNSTAGE; ++s) {
    dma_stage(rsa, offa, ca, (uint32_t)s * DKB, kbytes, smem + s * DSTAGE);
    dma_stage(rsb, offb, cb, (uint32_t)s * DKB, kbytes, smem + s * DSTAGE + 256 * DKB);
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(8 * (DNSTAGE - 1)));
  __builtin_amdgcn_s_barrier();

  // scheduling groups (__builtin_amdgcn_sched_group_barrier masks): MFMA 0x8, VMEM read 0x20, DS read 0x100
  constexpr int NMF = (DT == OCTO_F32) ? 64 : 16;  // MFMA instructions per 16-byte-fragment block
  i32x4 a0[4], b0[4], a1[4], b1[4];
  read_frags(smem, aoff[0], boff[0], a0, b0);
  for (int k = 0; k < nk; ++k) {
    const lds_char *cur = smem + (k & (DNSTAGE - 1)) * DSTAGE;
    // half 1: fragments of sub-step 1 read under the MFMAs of sub-step 0
    read_frags(cur, aoff[1], boff[1], a1, b1);
    mfma_block<DT>(a0, b0, acc);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, NMF / 16, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NMF / 2, 0);
    __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);                       // this wave's reads of stage k are done
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(8 * (DNSTAGE - 2)));    // stage k + 1 landed (this wave's part)
    __builtin_amdgcn_s_barrier();                                 // ... in every wave; stage k is free
    // half 2: refill stage k's buffer four stages ahead and read sub-step 0 of stage k + 1 under the
    // MFMAs of sub-step 1
    lds_char *refill = smem + (k & (DNSTAGE - 1)) * DSTAGE;
    const uint32_t kb = (uint32_t)(k + DNSTAGE) * DKB;
    dma_stage(rsa, offa, ca, kb, kbytes, refill);
    dma_stage(rsb, offb, cb, kb, kbytes, refill + 256 * DKB);
    const lds_char *nxt = smem + ((k + 1) & (DNSTAGE - 1)) * DSTAGE;
    read_frags(nxt, aoff[0], boff[0], a0, b0);
    mfma_block<DT>(a1, b1, acc);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, NMF / 16, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, NMF / 16, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
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
