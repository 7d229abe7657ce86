// The MFMA GEMM core shared by every contraction of the LM-head path.
//
//   C[m, n] = sum_k A[m, k] * B[n, k]        (operands K-contiguous, "NT", or one of them K-major: OpColsN)
//
// One workgroup computes a 256 x 256 tile of C. The 16-bit loop runs 512 threads = 8 wave64s, two per SIMD, sat
// 2 x 4, each owning a 128 x 64 sub-tile as 8 x 4 blocks of v_mfma_f32_16x16x32_{bf16,f16} (Acc16N<4>, 128
// accumulation registers): while one wave of a SIMD waits on a stage the other issues MFMAs. The fp32 loop runs 4
// waves, 2 x 2, each 128 x 128 as 4 x 4 blocks of v_mfma_f32_32x32x2_f32 (Acc32). Under the part's power limit the
// 16x16x32 form sustains 12% more bf16 FLOP/s than the 32x32x16 one on random operands (2.10 against 1.88 PFLOP/s,
// a register-only loop on every SIMD), and each MFMA streams fewer accumulator bytes per FLOP.
//
// The mainloop feeds the MFMAs from LDS: the A and B K-slices go straight from global memory into a ring of
// LDS stages by buffer_load_dwordx4 ... lds (no register hop), with the instruction order fixed in the source:
// fragment reads a step ahead of their MFMAs and the DMA issues spread between MFMAs. fp8 (e4m3) weights are
// widened to bf16 once per call (exactly: e4m3 has 3 mantissa bits) and run the 16-bit loop, their per-row scale
// applied in the epilogue.
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
#include "tile_order.h"

namespace octo {

constexpr int TM = 256;          // tile rows (M)
constexpr int TN = 256;          // tile cols (N)
constexpr int NTHREADS = 256;

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

// Block -> (mt, nt): the order of tile_order.h, block b being XCD b % 8's (b / 8)-th tile. A device-side row count
// that bounds M or N shrinks the tile grid (read once per block), so the idle blocks all come after the working ones.
__host__ __device__ inline int64_t tile_grid(int mtiles, int ntiles) { return octo_tiles::tile_grid(mtiles, ntiles); }
// The tile grid after a device-side row count's bound (read from memory).
__device__ __forceinline__ void bounded_tiles(const GemmShape &s, int64_t &mtiles, int64_t &ntiles) {
  mtiles = s.mtiles;
  ntiles = s.ntiles;
  if (s.count_on == 1) mtiles = min(mtiles, cdiv(dev_count(s.count, s.count_off, s.M), (int64_t)TM));
  if (s.count_on == 2) ntiles = min(ntiles, cdiv(dev_count(s.count, s.count_off, s.N), (int64_t)TN));
}
// XCD x's k-th tile; false past its tiles.
__device__ __forceinline__ bool tile_at(const GemmShape &s, int x, int64_t k, int64_t mtiles, int64_t ntiles, int &mt,
                                        int &nt) {
  return octo_tiles::tile_at(s.group_m, x, k, mtiles, ntiles, mt, nt);
}
// The one-shot grid's block -> (mt, nt): block b is XCD b % 8's (b / 8)-th tile.
__device__ __forceinline__ bool tile_of(const GemmShape &s, int &mt, int &nt) {
  int64_t mtiles, ntiles;
  bounded_tiles(s, mtiles, ntiles);
  return tile_at(s, (int)(blockIdx.x & 7), (int64_t)(blockIdx.x >> 3), mtiles, ntiles, mt, nt);
}

template <int DT> struct Mfma;
template <> struct Mfma<OCTO_F32> {
  // a 16-byte fragment holds 4 fp32 K values: four 32x32x2 steps, lane half h supplies k = 4h + e
  static __device__ __forceinline__ void run(const i32x4 a, const i32x4 b, f32x16 &c) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      c = __builtin_amdgcn_mfma_f32_32x32x2f32(__int_as_float(a[e]), __int_as_float(b[e]), c, 0, 0, 0);
  }
};

__device__ __forceinline__ const char *uniform_ptr(const char *p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const char *)(((uint64_t)hi << 32) | lo);
}

// ---- 4-stage mainloop (fp32 operands) ----------------------------------------------------------------
//
// K advances 64 bytes per stage (16 fp32). Each operand's stage slice (16 KB)
// is written straight into LDS by buffer_load_dwordx4 ... lds: a wave instruction moves 1 KB, lane i's 16 bytes
// landing at the instruction's LDS base + 16 i, so the LDS layout is chosen by which global chunk each lane
// fetches. DNSTAGE stages form a ring (A slice, then B slice, per stage). One bare s_barrier per stage (no
// memory fence: the waits are explicit) separates "stage k + 1 landed in every wave" and "every wave has read
// stage k" from the DMA that overwrites stage k's slot.
//
// The operand (OpRows, K-contiguous rows): a slice is 256 rows x 64 bytes. Chunk c of row r sits at
//     physical chunk c ^ ((r >> 2) & 3), so a 16-lane pass of fragment reads (rows r0..r0+15 of one logical
//     chunk) covers all 64 banks once. A fragment is one ds_read_b128: lane l holds row l & 31 of a 32-row
//     block, K chunk 2 sub + (l >> 5).
constexpr int DKB = 64;                    // K bytes per stage
constexpr int DSLICE = 256 * DKB;          // one operand's stage slice (16 KB)
constexpr int DSTAGE = 2 * DSLICE;         // A + B bytes per stage
#ifndef OCTO_NSTAGE
#define OCTO_NSTAGE 4
#endif
constexpr int DNSTAGE = OCTO_NSTAGE;       // ring depth
constexpr int DIPW = 4;                    // DMA instructions per wave per operand and stage
constexpr int DNSUB = 2;                   // 16-byte-fragment sub-steps per stage
// LDS of one GEMM workgroup: the DMA ring.
constexpr int SMEM_BYTES = DNSTAGE * DSTAGE;
static_assert(SMEM_BYTES <= 160 * 1024, "LDS budget");

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] + vmcnt[5:4] at bits 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int WAIT_LGKM0 = 15 | (3 << 14) | (7 << 4);

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, lds_char *dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, 0, 0, 0);
}

// K-contiguous operand: instruction q of wave w fills slice rows (4 q + w) * 16 .. + 16; lane i takes row
// + (i >> 2) and physical chunk i & 3.
struct OpRows {
  static constexpr int NI = DIPW;     // DMA instructions per wave and stage
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[DIPW], coff[DIPW];
  int fo[DNSUB];  // fragment byte offsets in the slice (block 0)

  __device__ __forceinline__ void init(const Operand &op, int64_t row0, int wsub, uint32_t /*krows*/) {
    const int w = threadIdx.x >> 6, i = threadIdx.x & 63, lane = i;
    const int64_t valid = dev_count(op.count, op.count_off + row0, op.rows - row0);
#pragma unroll
    for (int q = 0; q < DIPW; ++q) {
      const int r = (4 * q + w) * 16 + (i >> 2);
      coff[q] = (uint32_t)(((i & 3) ^ ((r >> 2) & 3)) << 4);
      uint32_t rowoff;
      if (r < valid) rowoff = op.map ? (uint32_t)(op.map[row0 + r] * op.ld) : (uint32_t)(r * op.ld);
      else rowoff = 0x80000000u;
      off[q] = rowoff + coff[q];
    }
    if (op.map) rs = make_rsrc(uniform_ptr(op.base), op.extent);
    else rs = make_rsrc(uniform_ptr(op.base + row0 * op.ld), (uint32_t)(256 * op.ld));
#pragma unroll
    for (int ks = 0; ks < DNSUB; ++ks) {
      const int c = 2 * ks + (lane >> 5);
      fo[ks] = (wsub * 128 + (lane & 31)) * DKB + ((c ^ ((lane >> 2) & 3)) << 4);
    }
  }
  // K chunks at or past kbytes (bytes per row) read zero
  __device__ __forceinline__ void dma(int k, int q, uint32_t kbytes, lds_char *slice) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t kb = (uint32_t)k * DKB;
    lds_dma16(rs, (kb + coff[q] < kbytes) ? off[q] + kb : 0x80000000u, slice + (4 * q + w) * 1024);
  }
  __device__ __forceinline__ i32x4 frag(const lds_char *slice, int sub, int blk) const {
    return *(const lds_i32x4 *)(slice + fo[sub] + blk * 32 * DKB);
  }
};

// Instruction order is fixed in the source: a scheduling fence after every MFMA / load keeps the fragment
// reads of the next sub-step early (so register allocation cannot fold them onto fragments still in use)
// and spreads the DMA issues evenly between MFMAs.
#define OCTO_FENCE() __builtin_amdgcn_sched_barrier(0)

// smem: DNSTAGE * DSTAGE bytes; stage s at s * DSTAGE, A slice first then B slice. `krows` bounds the K-rows
// of MN-contiguous operands.
//
// Stage j's A slice is issued right after the barrier that frees its slot (in iteration j - DNSTAGE), its B slice
// under the first sub-step of the next iteration (into the slot stage j - DNSTAGE left), so the DMA instructions
// of a stage are spread over two sub-steps.
template <int DT, typename OA, typename OB>
__device__ __forceinline__ void mainloop_dma(const Operand &A, const Operand &B, int64_t m0, int64_t n0, int64_t K_eff,
                                             lds_char *smem, f32x16 (&acc)[4][4]) {
  static_assert(DNSTAGE >= 3, "ring depth");
  constexpr int NA = OA::NI, NB = OB::NI, NPS = NA + NB;  // DMA instructions per wave and stage
  constexpr int SPA = 8 / NA, SPB = 8 / NB;                // MFMAs between two DMA issues
  static_assert(NPS * DNSTAGE <= 63, "vmcnt range");
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

  OA opa;
  OB opb;
  opa.init(A, m0, wm, (uint32_t)K_eff);
  opb.init(B, n0, wn, (uint32_t)K_eff);

#pragma unroll
  for (int st = 0; st < DNSTAGE; ++st) {
#pragma unroll
    for (int q = 0; q < NA; ++q) opa.dma(st, q, kbytes, smem + st * DSTAGE);
    if (st < DNSTAGE - 1) {
#pragma unroll
      for (int q = 0; q < NB; ++q) opb.dma(st, q, kbytes, smem + st * DSTAGE + DSLICE);
    }
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(NPS * (DNSTAGE - 2) + NA));  // stage 0 landed
  __builtin_amdgcn_s_barrier();

  i32x4 fa[2][4], fb[2][4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    fa[0][b] = opa.frag(smem, 0, b);
    fb[0][b] = opb.frag(smem + DSLICE, 0, b);
  }
  int slot = 0;                 // k % DNSTAGE
  int prev_slot = DNSTAGE - 1;  // (k - 1) % DNSTAGE
  for (int k = 0; k < nk; ++k) {
    const int next_slot = (slot + 1 == DNSTAGE) ? 0 : slot + 1;
    const lds_char *cur = smem + slot * DSTAGE;
    __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);  // this sub-step's fragments (read under the previous one) are in
    OCTO_FENCE();
    // sub-step 0: read sub-step 1's fragments under the first 8 MFMAs; the B slice of stage k + DNSTAGE - 1 (into
    // the slot stage k - 1 left) under the last 8
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      Mfma<DT>::run(fa[0][q >> 2], fb[0][q & 3], acc[q >> 2][q & 3]);
      OCTO_FENCE();
      if (q < 8) {
        if (q < 4) fa[1][q] = opa.frag(cur, 1, q);
        else fb[1][q - 4] = opb.frag(cur + DSLICE, 1, q - 4);
        OCTO_FENCE();
      }
      if (q >= 8 && (q - 8) % SPB == SPB - 1) {
        opb.dma(k + DNSTAGE - 1, (q - 8) / SPB, kbytes, smem + prev_slot * DSTAGE + DSLICE);
        OCTO_FENCE();
      }
    }
    __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);                           // this wave's reads of stage k are done
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(NPS * (DNSTAGE - 2)));     // stage k + 1 landed (this wave's part)
    __builtin_amdgcn_s_barrier();                                     // ... in every wave; stage k is free
    OCTO_FENCE();
    // sub-step 1: read the next stage's first fragments under the first 8 MFMAs, refill stage k's slot with
    // stage k + DNSTAGE's A slice under the last 8
    const lds_char *nxt = smem + next_slot * DSTAGE;
    lds_char *refill = smem + slot * DSTAGE;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      Mfma<DT>::run(fa[1][q >> 2], fb[1][q & 3], acc[q >> 2][q & 3]);
      OCTO_FENCE();
      if (q < 8) {
        if (q < 4) fa[0][q] = opa.frag(nxt, 0, q);
        else fb[0][q - 4] = opb.frag(nxt + DSLICE, 0, q - 4);
        OCTO_FENCE();
      }
      if (q >= 8 && (q - 8) % SPA == SPA - 1) {
        opa.dma(k + DNSTAGE, (q - 8) / SPA, kbytes, refill);
        OCTO_FENCE();
      }
    }
    prev_slot = slot;
    slot = next_slot;
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0) & WAIT_LGKM0);
  __builtin_amdgcn_s_barrier();
}

// ---- full-line mainloop: K = 64 per stage, a 5-slot ring ------------------------------------------
//
// For 16-bit types. A stage holds K = 64 (128 bytes of every operand row), so each row fetch of a K-contiguous
// operand is one whole 128-byte cache line; with 64-byte rows (the 4-stage ring above) every line is requested
// twice, once per half, which doubles the L1 -> L2 requests and stalls the address unit on the L1.
//
// A stage is two 32 KB slices (A, B). The LDS holds five slices, 2.5 stages: stage j's A slice sits in slot
// 2 j mod 5, its B slice in slot 2 j + 1 mod 5. One s_barrier per stage, B_k, placed between stage k's two K-steps,
// means "every wave has read stage k" (its last fragments are read under its first K-step) and "stage k + 1 has
// landed in every wave". It frees stage k's two slots: slot 2 k (mod 5) takes stage k + 2's B slice, slot 2 k + 1
// stage k + 3's A slice. So iteration k issues stage k + 2 whole: its A slice under K-step 0 (into the slot freed at
// B_(k-1)), its B slice under K-step 1 (the slot freed at B_k). At B_k only stage k + 2's A slice may still be in
// flight: vmcnt(32 / NW).
//
//   OpRowsN (K-contiguous rows): a slice is 256 rows x 128 bytes. Chunk c (0..7) of row r sits at physical
//     chunk c ^ ((r >> 1) & 7), so a 16-lane pass of fragment reads (rows r0..r0+15, r0 a multiple of 16, of
//     one logical chunk) covers all 64 banks once. DMA instruction q of wave w fills slice rows (NW q + w) * 8 ..
//     + 8; lane i takes row + (i >> 3) and physical chunk i & 7, so the 8 lanes of a row fetch its 128 bytes.
//     A fragment is one ds_read_b128: lane l holds row l & 15 of a 16-row block, K chunk 4 ks + (l >> 4) of the
//     stage's K-step ks (the v_mfma_f32_16x16x32 operand layout).
constexpr int EKB = 128;              // K bytes per stage and row
constexpr int ESLICE = 256 * EKB;     // one operand's stage slice (32 KB)
constexpr int ENSLOT = 5;             // ring slots
constexpr int SMEM_RING5 = ENSLOT * ESLICE;
static_assert(SMEM_RING5 <= 160 * 1024, "LDS budget");

// The loop runs with NW = 4 waves (2 x 2, each 128 x 128 of the tile) or NW = 8 (2 x 4, each 128 x 64: two waves
// per SIMD, so one issues MFMAs while the other waits on a stage or runs its epilogue). An operand's SUB is the
// wave's rows of it (128; 64 for the B operand of the 8-wave loop). A slice takes 32 DMA instructions, 32 / NW per
// wave.
template <int NW, int SUB>
struct OpRowsN {
  static constexpr int NI = 32 / NW;   // DMA instructions per wave and stage
  static constexpr int NB = SUB / 16;  // the wave's 16-row fragment blocks
  typedef i32x4 F;  // fragment as held between its read and its MFMAs
  static __device__ __forceinline__ i32x4 op(const F &f) { return f; }
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[NI];
  uint32_t coff;
  int fo;  // fragment byte offset of K-step 0, block 0 (K-step 1: fo ^ 64)
  __device__ __forceinline__ void init(const Operand &op, int64_t row0, int wsub, uint32_t /*krows*/) {
    const int w = threadIdx.x >> 6, i = threadIdx.x & 63, lane = i;
    const int64_t valid = dev_count(op.count, op.count_off + row0, op.rows - row0);
    // row (NW q + w) * 8 + (i >> 3): its swizzle ((row >> 1) & 7) = (4 (w & 1) + (i >> 4)) & 7 for every q
    coff = (uint32_t)(((i & 7) ^ ((4 * (w & 1) + (i >> 4)) & 7)) << 4);
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int r = (NW * q + w) * 8 + (i >> 3);
      uint32_t rowoff;
      if (r < valid) rowoff = op.map ? (uint32_t)(op.map[row0 + r] * op.ld) : (uint32_t)(r * op.ld);
      else rowoff = 0x80000000u;
      off[q] = rowoff + coff;
    }
    if (op.map) rs = make_rsrc(uniform_ptr(op.base), op.extent);
    else rs = make_rsrc(uniform_ptr(op.base + row0 * op.ld), (uint32_t)(256 * op.ld));
    // lane l holds row l & 15 of a 16-row block and chunk 4 ks + (l >> 4) of K-step ks; (row >> 1) & 7 depends on
    // l & 15 alone, and 4 ks + g = (4 ks) ^ g for g < 4, so K-step 1's offset is K-step 0's with chunk bit 2 flipped
    const int row = wsub * SUB + (lane & 15);
    fo = row * EKB + ((((lane >> 4) ^ ((lane >> 1) & 7))) << 4);
  }
  // K chunks at or past kbytes (bytes per row) read zero
  __device__ __forceinline__ void dma(int k, int q, uint32_t kbytes, lds_char *slice) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t kb = (uint32_t)k * EKB;
    lds_dma16(rs, (kb + coff < kbytes) ? off[q] + kb : 0x80000000u, slice + (NW * q + w) * 1024);
  }
  // the 16 K values (chunk 4 ks + (l >> 4)) of row l & 15 of 16-row block blk, K-step ks (0, 1) of the stage
  __device__ __forceinline__ i32x4 frag(const lds_char *slice, int ks, int blk) const {
    return *(const lds_i32x4 *)(slice + (fo ^ (ks << 6)) + blk * 16 * EKB);
  }
};


typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16 through a restrict pointer: inlining gives the read alias-scope information, without which
// the compiler waits for every LDS DMA in flight (vmcnt(0)) before it, as for a read it cannot tell apart from them.
__device__ __forceinline__ s16x4 lds_read_tr16(lds_s16x4 *__restrict__ p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(p);
}

// K-major operand: the GEMM's K runs down the matrix rows and M along them, element (k, m) at base + k ld + 2 m
// (grad_W = dz^T h reads dz token-major this way, so dz needs no vocab-major copy). A stage slice is 64 K-rows of
// the tile's 256 M values (512 bytes). The 32-byte segment s (M values 16 s .. 16 s + 15) of slice row r sits at
// physical segment s ^ f(r), f(r) = (r & 3) | ((r >> 3) & 3) << 2.
// A fragment is two ds_read_b64_tr_b16. In a 16-lane group the instruction returns to lane i, element e, element
// i & 3 of what lane 4 e + (i >> 2) addressed; so lane s of group G addresses K-row 8 G + (s >> 2) (+ 4 for the
// second read) and M values 4 (s & 3) .. + 3 of the block, and lane l receives M value l & 15 at K values
// 8 (l >> 4) + 0..7: the K-contiguous fragment layout of OpRowsN. The 16 rows one read touches have distinct
// f(r), so its 64 lanes cover 512 consecutive bank bytes.
// DMA instruction q of wave w fills rows r0 = 2 (q & 1) + 4 ((q >> 1) & 1) + 8 w + 8 NW (q >> 2) and r0 + 1, lane i
// row r0 + (i >> 5) and physical 16-byte chunk i & 31: f(r) then depends on the lane and q & 1 only, so two
// lane offsets serve all of a wave's instructions, the row offset riding in the instruction's scalar offset.
// Nothing is bounds-checked: the caller guarantees K-rows up to the next multiple of 64 exist and read zero past K.
template <int NW, int SUB>
struct OpColsN {
  static constexpr int NI = 32 / NW;
  static constexpr int NB = SUB / 16;
  // A fragment is carried as its two 8-byte halves and joined at each MFMA: a joined 16-byte value carried across
  // the loop makes the register allocator keep the halves and the join apart (64 more VGPRs, spilled accumulators).
  struct F {
    i32x2 lo, hi;
  };
  static __device__ __forceinline__ i32x4 op(const F &f) { return __builtin_shufflevector(f.lo, f.hi, 0, 1, 2, 3); }
  const char *base;  // K-row 0, M value col0
  uint32_t ld;       // K-row stride, bytes
  uint32_t lo[2];    // lane offset (row 8 w + (i >> 5)) of the DMA instructions with q & 1 = 0, 1
  int fo, fx;        // fragment byte offset of K-step 0, read 0; segment XOR of block 0

  __device__ __forceinline__ void init(const Operand &op, int64_t col0, int wsub, uint32_t /*krows*/) {
    const int w = threadIdx.x >> 6, i = threadIdx.x & 63, c = i & 31;
    base = uniform_ptr(op.base + col0 * 2);
    ld = (uint32_t)op.ld;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int f = (i >> 5) | (b << 1) | ((w & 3) << 2);
      lo[b] = (uint32_t)((i >> 5) + 8 * w) * ld + (uint32_t)((((c >> 1) ^ f) << 5) | ((c & 1) << 4));
    }
    const int g = (i >> 4) & 3, s = i & 15;
    fo = (8 * g + (s >> 2)) * 512 + 8 * (s & 3);
    fx = (NB * wsub) ^ ((s >> 2) | (g << 2));
  }
  __device__ __forceinline__ void dma(int k, int q, uint32_t /*kbytes*/, lds_char *slice) const {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = 2 * (q & 1) + 4 * ((q >> 1) & 1) + 8 * NW * (q >> 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(base + (int64_t)k * 64 * ld, 64u * ld),
                                             (__attribute__((address_space(3))) void *)(slice + (r0 + 8 * w) * 512),
                                             16, lo[q & 1], (uint32_t)r0 * ld, 0, 0);
  }
  __device__ __forceinline__ F frag(const lds_char *slice, int ks, int blk) const {
    const lds_char *p = slice + fo + ks * 32 * 512 + ((fx ^ blk) << 5);
    F f;
    f.lo = __builtin_bit_cast(i32x2, lds_read_tr16((lds_s16x4 *)p));
    f.hi = __builtin_bit_cast(i32x2, lds_read_tr16((lds_s16x4 *)(p + 4 * 512)));
    return f;
  }
};

// The 16-bit GEMMs (bf16 / f16 operands; fp8 weights are widened to bf16 before the GEMM) run the ring loop, fp32
// the 4-stage one.
__host__ __device__ constexpr bool ring5_ok(int dt) { return dt == OCTO_BF16 || dt == OCTO_F16; }

// MFMA order within a K-step: A block i fixed for NBB consecutive MFMAs, B blocks walked forward for even i and
// backward for odd i, so the B operand is also unchanged across each change of A (25 B changes per K-step of 8 x 4
// blocks, against 32 walking forward each time). Under the part's power limit fewer operand changes per MFMA leave
// a little more clock: same box, d 2560, V 151,936, the 24,576-row forward + backward 56.1-56.2 against 56.2-56.4 ms,
// the 32,768-row forward 18.33-18.40 against 18.45-18.47 ms (bitwise the same results: each accumulator sees the
// same K order).
#ifndef OCTO_MFMA_SNAKE
#define OCTO_MFMA_SNAKE 1
#endif

template <int DT> struct Mfma16;
template <> struct Mfma16<OCTO_BF16> {
  static __device__ __forceinline__ void run(const i32x4 a, const i32x4 b, f32x4 &c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<OCTO_F16> {
  static __device__ __forceinline__ void run(const i32x4 a, const i32x4 b, f32x4 &c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// One stage of the ring loop on the stage in slots (sa, sa + 1): two K-steps of K = 32, each 64 v_mfma_f32_16x16x32
// over the wave's 8 x 8 blocks (A fragment i reused by 8 consecutive MFMAs). The 16 fragment reads of the next K-step
// go under the first 16 MFMAs (double-buffered: K-step ks uses fa[ks], fb[ks]); the barrier B_k sits between the two
// K-steps, after the last reads of stage k. DMA: issue stage kd of the operands' current tile (stage k + 2 of the
// stream: A under K-step 0, B under K-step 1, one instruction per 6 MFMAs). NEXT: a stage k + 1 exists (barrier B_k);
// XFRAG: its first fragments are read under K-step 1 (else the caller reads them).
// SPLIT: B_k only frees stage k's slots; the wait for stage k + 1 (vmcnt, then a second barrier L_k) moves to the
// middle of K-step 1, and stage k + 1's first fragments are read after L_k. The wait then covers DMA issued half a
// K-step longer ago, for a second barrier per stage.
template <int DT, typename OA, typename OB, bool DMA, bool NEXT, bool XFRAG, bool SPLIT>
__device__ __forceinline__ void ring5_stage(const OA &opa, const OB &opb, int kd, int sa, uint32_t kbytes,
                                            lds_char *smem, typename OA::F (&fa)[2][OA::NB],
                                            typename OB::F (&fb)[2][OB::NB], f32x4 (&acc)[OA::NB][OB::NB]) {
  constexpr int NA = OA::NB, NBB = OB::NB, NQ = NA * NBB, NR = NA + NBB, NI = OA::NI;
  constexpr int D0 = NR + 1, DS = (NQ - D0 + NI - 1) / NI;  // DMA issues: MFMA D0, D0 + DS, ... (4 waves: 17 + 6 j)
  // SPLIT: L_k at MFMA QX; DQX DMA instructions of this K-step are issued before it
  constexpr int QX = NQ / 2, DQX = QX <= D0 ? 0 : ((QX - 1 - D0) / DS + 1 < NI ? (QX - 1 - D0) / DS + 1 : NI);
  static_assert(!SPLIT || QX + NR <= NQ, "next-stage fragment reads fit the K-step");
  constexpr int XQ = SPLIT ? QX : 0;  // first MFMA under which stage k + 1's fragments are read
  // slots: stage k at (sa, sa + 1), stage k + 1 at (sa + 2, sa + 3), stage k + 2's A at sa + 4, its B at sa
  auto slot = [&](int d) -> lds_char * { const int x = sa + d; return smem + (x >= ENSLOT ? x - ENSLOT : x) * ESLICE; };
  const lds_char *cA = slot(0), *cB = slot(1);
  const lds_char *nA = slot(2), *nB = slot(3);
  lds_char *dA = slot(4), *dB = slot(0);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    if (ks == 1 && NEXT) {
      __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);  // this wave's reads of stage k are done
      if (!SPLIT) {
        if (DMA) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NI));  // stage k + 1 landed (k + 2's A may be in flight)
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      }
      __builtin_amdgcn_s_barrier();  // ... in every wave; stage k's slots are free
    } else {
      __builtin_amdgcn_s_waitcnt(WAIT_LGKM0);  // this K-step's fragments are in
    }
    OCTO_FENCE();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (SPLIT && ks == 1 && NEXT && q == QX) {
        // L_k: stage k + 1 landed (stage k + 2's A and this K-step's first B issues may be in flight) ... everywhere
        if (DMA) __builtin_amdgcn_s_waitcnt(waitcnt_vm(NI + DQX));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __builtin_amdgcn_s_barrier();
        OCTO_FENCE();
      }
      const int qi = q / NBB;
      const int qj = (OCTO_MFMA_SNAKE && (qi & 1)) ? NBB - 1 - q % NBB : q % NBB;
      Mfma16<DT>::run(OA::op(fa[ks][qi]), OB::op(fb[ks][qj]), acc[qi][qj]);
      OCTO_FENCE();
      if (ks == 0 && q < NR) {
        if (q < NA) fa[1][q] = opa.frag(cA, 1, q);
        else fb[1][q - NA] = opb.frag(cB, 1, q - NA);
        OCTO_FENCE();
      } else if (ks == 1 && NEXT && XFRAG && q >= XQ && q < XQ + NR) {
        if (q - XQ < NA) fa[0][q - XQ] = opa.frag(nA, 0, q - XQ);
        else fb[0][q - XQ - NA] = opb.frag(nB, 0, q - XQ - NA);
        OCTO_FENCE();
      }
      if (DMA && q >= D0 && (q - D0) % DS == 0 && (q - D0) / DS < NI) {
        if (ks == 0) opa.dma(kd, (q - D0) / DS, kbytes, dA);
        else opb.dma(kd, (q - D0) / DS, kbytes, dB);
        OCTO_FENCE();
      }
    }
  }
}

__device__ __forceinline__ int ring_slot(int s) { return s >= ENSLOT ? s - ENSLOT : s; }

// The ring loop's prologue: stage 0 into slots (sa0, sa0 + 1), stage 1 (when nk > 1) into (sa0 + 2, sa0 + 3), mod 5.
template <typename OA, typename OB>
__device__ __forceinline__ void ring5_prologue(const OA &opa, const OB &opb, int sa0, uint32_t kbytes, int nk,
                                               lds_char *smem) {
  constexpr int NI = OA::NI;
#pragma unroll
  for (int q = 0; q < NI; ++q) opa.dma(0, q, kbytes, smem + ring_slot(sa0) * ESLICE);
#pragma unroll
  for (int q = 0; q < NI; ++q) opb.dma(0, q, kbytes, smem + ring_slot(sa0 + 1) * ESLICE);
  if (nk > 1) {
#pragma unroll
    for (int q = 0; q < NI; ++q) opa.dma(1, q, kbytes, smem + ring_slot(sa0 + 2) * ESLICE);
#pragma unroll
    for (int q = 0; q < NI; ++q) opb.dma(1, q, kbytes, smem + ring_slot(sa0 + 3) * ESLICE);
  }
}

// The ring loop after its prologue, stage j of the tile in slots (sa0 + 2 j, sa0 + 2 j + 1) mod 5; acc is zeroed
// here. Ends with every DMA landed and every wave past its last LDS read (the slots are free), and returns the slot
// that continues the ring, (sa0 + 2 nk) mod 5. VMEM instructions issued after the prologue's (a previous tile's
// epilogue stores) are fine: loads complete in order among themselves, so at most 2 NI outstanding means stage 0 in.
template <int DT, typename OA, typename OB, bool SPLIT>
__device__ __forceinline__ int ring5_run(const OA &opa, const OB &opb, int sa0, uint32_t kbytes, int nk,
                                         lds_char *smem, f32x4 (&acc)[OA::NB][OB::NB]) {
  constexpr int NI = OA::NI;
#pragma unroll
  for (int i = 0; i < OA::NB; ++i)
#pragma unroll
    for (int j = 0; j < OB::NB; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;
  if (nk == 0) return sa0;
  if (nk > 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * NI));  // stage 0 landed
  else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  __builtin_amdgcn_s_barrier();

  typename OA::F fa[2][OA::NB];
  typename OB::F fb[2][OB::NB];
#pragma unroll
  for (int b = 0; b < OA::NB; ++b) fa[0][b] = opa.frag(smem + ring_slot(sa0) * ESLICE, 0, b);
#pragma unroll
  for (int b = 0; b < OB::NB; ++b) fb[0][b] = opb.frag(smem + ring_slot(sa0 + 1) * ESLICE, 0, b);
  int sa = sa0;  // slot of stage k's A slice: sa0 + 2 k mod 5
  int k = 0;
  for (; k + 2 < nk; ++k) {
    ring5_stage<DT, OA, OB, true, true, true, SPLIT>(opa, opb, k + 2, sa, kbytes, smem, fa, fb, acc);
    sa = ring_slot(sa + 2);
  }
  if (k + 1 < nk) {
    ring5_stage<DT, OA, OB, false, true, true, SPLIT>(opa, opb, k, sa, kbytes, smem, fa, fb, acc);
    sa = ring_slot(sa + 2);
    ++k;
  }
  ring5_stage<DT, OA, OB, false, false, false, SPLIT>(opa, opb, k, sa, kbytes, smem, fa, fb, acc);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0) & WAIT_LGKM0);
  __builtin_amdgcn_s_barrier();
  return ring_slot(sa + 2);
}

// smem: SMEM_RING5 bytes. 16-bit types only.
template <int DT, typename OA, typename OB, bool SPLIT = false>
__device__ __forceinline__ void mainloop_ring5(const Operand &A, const Operand &B, int64_t m0, int64_t n0,
                                               int64_t K_eff, lds_char *smem, f32x4 (&acc)[OA::NB][OB::NB]) {
  static_assert(DT == OCTO_BF16 || DT == OCTO_F16, "16-bit operands");
  static_assert(OA::NI == OB::NI, "one workgroup shape");
  constexpr int NWN = TN / (16 * OB::NB);  // waves along N
  const int w = threadIdx.x >> 6;
  const int wm = w / NWN, wn = w % NWN;
  const uint32_t kbytes = (uint32_t)(K_eff * 2);
  const int nk = (int)((kbytes + EKB - 1) / EKB);
  OA opa;
  OB opb;
  if (nk > 0) {
    opa.init(A, m0, wm, (uint32_t)K_eff);
    opb.init(B, n0, wn, (uint32_t)K_eff);
    ring5_prologue(opa, opb, 0, kbytes, nk, smem);
  }
  ring5_run<DT, OA, OB, SPLIT>(opa, opb, 0, kbytes, nk, smem, acc);
}

// ---- accumulator layouts of a wave's 128 x 128 sub-tile --------------------------------------------
//
// Row (M) and column (N), relative to the tile origin, of element v of block (i, j) of wave (wm, wn). In both
// layouts elements 4 g .. 4 g + 3 of a block are 4 consecutive rows of one column, and the lanes holding one column
// (the rows of a column reduction) differ in the lane bits above the column bits.
struct Acc32 {  // 4 x 4 blocks of v_mfma_f32_32x32x*: column l & 31, rows 8 (v >> 2) + 4 (l >> 5) + (v & 3)
  static constexpr int NI = 4, NJ = 4, NV = 16;
  typedef f32x16 V;
  static __device__ __forceinline__ int wm(int w) { return w >> 1; }  // 2 x 2 waves
  static __device__ __forceinline__ int wn(int w) { return w & 1; }
  static __device__ __forceinline__ int row(int wm, int i, int v, int lane) {
    return wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
  }
  static __device__ __forceinline__ int col(int wn, int j, int lane) { return wn * 128 + j * 32 + (lane & 31); }
  static __device__ __forceinline__ float col_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
  static __device__ __forceinline__ float col_sum(float x) { return x + __shfl_xor(x, 32, 64); }
  static __device__ __forceinline__ bool col_lane(int lane) { return lane < 32; }  // one lane per column
};
// 8 x NJ blocks of v_mfma_f32_16x16x*: column l & 15, rows 4 (l >> 4) + v; NJ = 8 for 2 x 2 waves of 128 x 128,
// NJ = 4 for the 8-wave loop's 2 x 4 waves of 128 x 64.
template <int NJ_>
struct Acc16N {
  static constexpr int NI = 8, NJ = NJ_, NV = 4;
  typedef f32x4 V;
  static constexpr int NWN = 256 / (16 * NJ);  // waves along N
  static __device__ __forceinline__ int wm(int w) { return w / NWN; }
  static __device__ __forceinline__ int wn(int w) { return w % NWN; }
  static __device__ __forceinline__ int row(int wm, int i, int v, int lane) {
    return wm * 128 + i * 16 + 4 * (lane >> 4) + v;
  }
  static __device__ __forceinline__ int col(int wn, int j, int lane) { return wn * 16 * NJ + j * 16 + (lane & 15); }
  static __device__ __forceinline__ float col_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    return fmaxf(x, __shfl_xor(x, 32, 64));
  }
  static __device__ __forceinline__ float col_sum(float x) {
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
  }
  static __device__ __forceinline__ bool col_lane(int lane) { return lane < 16; }
};
// The fp32 path's layout.
__device__ __forceinline__ int acc_row(int wm, int i, int v, int lane) { return Acc32::row(wm, i, v, lane); }
__device__ __forceinline__ int acc_col(int wn, int j, int lane) { return Acc32::col(wn, j, lane); }

}  // namespace octo
