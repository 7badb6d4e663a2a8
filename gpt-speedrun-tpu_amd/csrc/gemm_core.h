// bf16 MFMA GEMM core for gfx950: C[m][n] = sum_k A(m,k) B(k,n), fp32 accumulate.
//
// Workgroup tile 256 x 256, 512 threads = 8 waves laid out 2 (M) x 4 (N),
// each wave owning a 128 x 64 sub-tile as 4 x 2 blocks of
// v_mfma_f32_32x32x16_bf16.  K advances in stages of 32.
//
// Operand staging: buffer_load_dwordx4 ... lds copies each 16-byte chunk
// straight from global memory into LDS (no registers, no LDS store
// instructions),
// through a 4-stage ring of separate LDS arrays (4 x 32 KB).  Stage kt is
// waited for with an exact vmcnt (the loads of the two younger stages stay in
// flight) followed by a bare s_barrier -- __syncthreads() would drain every
// outstanding load.  Keeping the stages in separate arrays lets the compiler
// see that LDS reads of one stage never alias the copies into another, so it
// inserts no vmcnt(0) before them.
//
// Each operand is K-major (A[m*ld + k], B[n*ld + k]) or MN-major
// (A[k*ld + m], B[k*ld + n]) and is copied in its natural layout:
//   K-major slab:  256 rows x 32 k = 64 B rows of 4 chunks; chunk c of row r
//                  sits at position c ^ ((r >> 2) & 3), so the 16 rows a
//                  quarter-wave reads at one chunk hit 16 distinct 16-byte
//                  bank groups;
//   MN-major slab: 32 k-rows x 256 = 512 B rows of 32 chunks; chunk c of row
//                  k sits at position c ^ (4 (k & 3)), so the 4 rows x 4
//                  chunks a half-wave of ds_read_b64_tr_b16 touches hit
//                  distinct bank groups.
// The swizzle is applied on the global side: lane L of a load writes LDS bytes
// [16L, 16L+16) of its 1 KB block and fetches whichever chunk belongs there.
// K-major fragments are one 16-byte LDS read per lane; MN-major fragments use
// ds_read_b64_tr_b16, which hands lane i of a 16-lane group the column of a
// 4 x 16 block: lane c supplies the address of row k0 + c/4, columns
// m0 + 4(c%4) .. +3, and lane i receives rows k0..k0+3 of column m0 + i.
//
// Per-lane global addresses are computed once per tile; a stage only adds a
// stride.  Fragment reads of the next half-stage are issued before the MFMAs
// of the current one, so LDS latency hides behind the matrix core.
#pragma once

#include <mutex>

#include "common.h"

namespace gemm {

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int THREADS = 512;
constexpr int OPE = 256 * BK;  // elements per operand slab of one stage (16 KB)
constexpr int STE = 2 * OPE;   // A slab then B slab
constexpr int kGroupM = 8;

__shared__ __attribute__((aligned(1024))) bf16 g_stage0[STE];
__shared__ __attribute__((aligned(1024))) bf16 g_stage1[STE];
__shared__ __attribute__((aligned(1024))) bf16 g_stage2[STE];
__shared__ __attribute__((aligned(1024))) bf16 g_stage3[STE];

typedef short v4i16 __attribute__((ext_vector_type(4)));
// Address-space-qualified views: LDS (3) so fragment traffic is ds_read/ds_write,
// global (1) so operand loads are global_load rather than flat.
typedef __attribute__((address_space(3))) bf16 lds_t;
typedef __attribute__((address_space(3))) bf16x8 lds_x8;
typedef __attribute__((address_space(3))) bf16x4 lds_x4;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(1))) void gbl_void;
typedef const __attribute__((address_space(1))) bf16x8 gbl_x8;

// A matrix operand: row-major with leading dimension ld, or (blk > 0)
// "32-blocked": element (r, c) at ((c / 32) * blk + r) * 32 + c % 32, i.e.
// column blocks of 32 stored one after another, each as blk rows of 64 bytes
// (so a 32-deep K-major stage, or the rows of an MN-major stage, read whole
// contiguous runs instead of 64-byte pieces of longer rows).
struct Operand {
  const bf16* p;
  int64_t ld;
  int64_t blk = 0;
};

__device__ __forceinline__ lds_t* lds_cast(bf16* p) { return (lds_t*)p; }

__device__ __forceinline__ bf16x4 read_tr(const lds_t* lds) {
  v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds));
  return __builtin_bit_cast(bf16x4, r);
}

template <int S>
__device__ __forceinline__ lds_t* stage_ptr() {
  if constexpr (S == 0) return (lds_t*)g_stage0;
  else if constexpr (S == 1) return (lds_t*)g_stage1;
  else if constexpr (S == 2) return (lds_t*)g_stage2;
  else return (lds_t*)g_stage3;
}

// Per-lane copy sources of one operand: the wave fills 1 KB blocks 2w and
// 2w+1 of each 16 KB slab with buffer_load_dwordx4 ... lds.  base is the
// operand's address at the tile origin and k_begin, step the bytes per stage
// (both uniform, so a stage's buffer resource is built in scalar registers);
// off[j] is the lane's byte offset from base, nvalid[j] the number of stages
// whose 16 bytes lie in [k_begin, k_end) and inside the M/N extent.  Later
// stages use an offset past the resource's range, which reads zeros.
// (The buffer form, unlike global_load_lds, is not taken by the compiler as
// a possible LDS access in flight, so its fragment reads keep exact lgkmcnt
// waits instead of lgkmcnt(0) while copies are outstanding.)
struct Src {
  const char* base;
  int64_t step;
  uint32_t off[2];
  int nvalid[2];
};

constexpr uint32_t kRsrcRange = 0x7FFFFFFFu;  // bytes a stage's resource covers
constexpr uint32_t kOffZero = 0xFFFFFFF0u;    // past the range: the copy reads zeros

template <bool KMAJOR>
__device__ __forceinline__ Src make_src(Operand op, int mn0, int k_begin, int MN, int k_end, int wave, int lane) {
  Src s;
  // (k_begin is a multiple of BK = 32 and mn0 of 256, so blocked stages and
  // tiles start on a 32-block.)
  const bf16* base;
  if (KMAJOR)
    base = op.blk ? op.p + ((int64_t)(k_begin >> 5) * op.blk + mn0) * 32 : op.p + (int64_t)mn0 * op.ld + k_begin;
  else
    base = op.blk ? op.p + ((int64_t)(mn0 >> 5) * op.blk + k_begin) * 32 : op.p + (int64_t)k_begin * op.ld + mn0;
  s.base = (const char*)base;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int blk = 2 * wave + j;
    if (KMAJOR) {
      const int row = blk * 16 + (lane >> 2);
      const int c = (lane & 3) ^ ((row >> 2) & 3);
      const int m = mn0 + row;
      s.off[j] = 2u * (uint32_t)(op.blk ? row * 32 + 8 * c : (int64_t)row * op.ld + 8 * c);
      const int rem = k_end - k_begin - 8 * c;
      s.nvalid[j] = (m < MN && rem > 0) ? (rem + BK - 1) / BK : 0;
    } else {
      const int row = blk * 2 + (lane >> 5);
      const int c = (lane & 31) ^ (4 * (row & 3));
      const int m = mn0 + 8 * c;
      s.off[j] = 2u * (uint32_t)(op.blk ? ((int64_t)(c >> 2) * op.blk + row) * 32 + 8 * (c & 3)
                                        : (int64_t)row * op.ld + 8 * c);
      const int rem = k_end - k_begin - row;
      s.nvalid[j] = (m < MN && rem > 0) ? (rem + BK - 1) / BK : 0;
    }
  }
  s.step = 2 * (op.blk ? (KMAJOR ? op.blk * 32 : (int64_t)BK * 32) : (KMAJOR ? (int64_t)BK : (int64_t)BK * op.ld));
  return s;
}

__device__ __forceinline__ void issue(lds_t* slab, const Src& s, int kt, int wave) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(s.base + kt * s.step, kRsrcRange);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int blk = 2 * wave + j;
    const uint32_t off = kt < s.nvalid[j] ? s.off[j] : kOffZero;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(slab + blk * 512), 16, off, 0, 0, 0);
  }
}

// MFMA operand (8 k-values) for rows r0 .. r0+31 at k-chunk kc (0 or 1) of a slab.
// K-major slabs: the lane reads row r0 + lrow (lrow = lane & 31 unless the
// caller permutes the rows of the block; accumulator row m then belongs to the
// slab row that lane m read).
template <bool KMAJOR>
__device__ __forceinline__ bf16x8 frag(const lds_t* slab, int r0, int kc, int lane, int lrow) {
  const int hl = lane >> 5;
  if (KMAJOR) {
    const int row = r0 + lrow;
    const int c = 2 * kc + hl;
    return *(const lds_x8*)(slab + row * BK + 8 * (c ^ ((row >> 2) & 3)));
  } else {
    const int cq = lane & 15;
    const int m = r0 + 16 * ((lane >> 4) & 1) + 4 * (cq & 3);
    const int k = 16 * kc + 8 * hl + (cq >> 2);
    const int off = 8 * ((m >> 3) ^ (4 * (k & 3))) + 4 * ((m >> 2) & 1);
    bf16x4 lo = read_tr(slab + k * 256 + off), hi = read_tr(slab + (k + 4) * 256 + off);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

// Column sums of B from the B operand fragments of one stage, already in
// registers: lane (l32, hl) of fragment nb holds B(k, wn0 + 32nb + l32) for
// the 8 k of its half of the 16-k chunk, so two v_dot2 against (1, 1) per
// 4 values add them to sum[nb].  Only waves of the first M half call this (the
// second half holds the same fragments); the two lane halves are combined by
// the caller.
__device__ __forceinline__ void colsum_frags(float* sum, const bf16x8 (&b0)[2], const bf16x8 (&b1)[2]) {
  const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sum[nb] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{b0[nb][2 * j], b0[nb][2 * j + 1]}, one, sum[nb], false);
      sum[nb] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{b1[nb][2 * j], b1[nb][2 * j + 1]}, one, sum[nb], false);
    }
}

// s_waitcnt immediates (gfx9 layout: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8]).
#define GEMM_WAIT_VM8_LGKM0() __builtin_amdgcn_s_waitcnt(0x0078)
#define GEMM_WAIT_VM12_LGKM0() __builtin_amdgcn_s_waitcnt(0x007C)
#define GEMM_WAIT_VM0_LGKM0() __builtin_amdgcn_s_waitcnt(0x0070)
// Keeps the compiler's scheduler from moving instructions across this point:
// the fragment reads of one half-stage stay ahead of the other half's MFMAs
// (left to itself it sinks each read next to its first use and then waits
// for it with lgkmcnt(0)).
#define GEMM_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

struct Ctx {
  Src sa, sb;
  int wm0, wn0, wave, lane, tid;
  int arow;  // row of each 32-row A block this lane reads (K-major A only; else lane & 31)
};

// The A-row order that gives lane (l32, hl) of a 32x32 accumulator the 16
// consecutive rows 16 hl .. 16 hl + 15 as elements 0 .. 15: element i sits in
// accumulator row 8 (i / 4) + 4 hl + i % 4, so lane l32 = 8a + 4h + b reads
// slab row 16h + 4a + b.
__device__ __forceinline__ int contiguous_row(int l32) { return 16 * ((l32 >> 2) & 1) + 4 * (l32 >> 3) + (l32 & 3); }

template <bool AK, bool BKM>
__device__ __forceinline__ void read_half(bf16x8 (&a)[4], bf16x8 (&b)[2], const lds_t* st, int kc, const Ctx& c) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) a[mb] = frag<AK>(st, c.wm0 + 32 * mb, kc, c.lane, c.arow);
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) b[nb] = frag<BKM>(st + OPE, c.wn0 + 32 * nb, kc, c.lane, c.lane & 31);
}

__device__ __forceinline__ void mma_half(f32x16 (&acc)[4][2], const bf16x8 (&a)[4], const bf16x8 (&b)[2]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(a[mb], b[nb], acc[mb][nb]);
}

__device__ __forceinline__ void fill(lds_t* st, const Ctx& c, int kt) {
  issue(st, c.sa, kt, c.wave);
  issue(st + OPE, c.sb, kt, c.wave);
}

// One stage of the persistent form: on entry a0/b0 hold k-chunk 0 of stage kt
// (buffer S).  Reads chunk 1, runs chunk 0's MFMAs, waits for stage kt+1 and
// the barrier (every wave is done with buffer S), refills S from `fc` at
// stage fkt (the current tile's stage kt+4, or one of the next tile's first
// stages), reads chunk 0 of stage kt+1, runs chunk 1's MFMAs.
template <bool AK, bool BKM, int S, bool kReadNext = true>
__device__ __forceinline__ void step_fill(f32x16 (&acc)[4][2], const Ctx& c, const Ctx& fc, int fkt, bf16x8 (&a0)[4],
                                          bf16x8 (&b0)[2]) {
  bf16x8 a1[4], b1[2];
  read_half<AK, BKM>(a1, b1, stage_ptr<S>(), 1, c);
  GEMM_SCHED_FENCE();
  mma_half(acc, a0, b0);
  GEMM_SCHED_FENCE();
  GEMM_WAIT_VM8_LGKM0();
  wg_barrier();
  fill(stage_ptr<S>(), fc, fkt);
  if (kReadNext) read_half<AK, BKM>(a0, b0, stage_ptr<(S + 1) % 4>(), 0, c);
  GEMM_SCHED_FENCE();
  mma_half(acc, a1, b1);
  GEMM_SCHED_FENCE();
}

// Persistent main loop for K a multiple of 4*BK (every tile then
// starts at stage buffer 0): the workgroup runs tiles blockIdx.x,
// blockIdx.x + gridDim.x, ... over the full K range, and the first four
// stages of its next tile are copied during the last four stages of the
// current one, so the epilogue runs while the next operands are in flight.
// coords(t, tm, tn) maps a tile index to tile coordinates; pre(tm, tn) runs
// before each tile's stages (after the previous tile's epilogue), e.g. to
// prefetch per-tile epilogue inputs far ahead of their use; epi(acc, tm, tn)
// must not touch the stage arrays (its own LDS and barriers are fine).
// kContiguousRows (K-major A only): A rows are read in the contiguous_row
// order, so each lane's accumulator elements 0 .. 15 are 16 consecutive rows.
template <bool AK, bool BKM, bool kContiguousRows = false, class Coords, class Pre, class Epi>
__device__ __forceinline__ void persistent(Operand A, Operand B, int M, int N, int K, int ntiles, Coords coords,
                                           Pre pre, Epi epi) {
  static_assert(AK || !kContiguousRows, "row permutation needs a K-major A operand");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int arow = kContiguousRows ? contiguous_row(lane & 31) : (lane & 31);
  int t = blockIdx.x;
  if (t >= ntiles) return;  // uniform
  const int nk = K / BK;
  int tm, tn;
  coords(t, tm, tn);
  Ctx c{make_src<AK>(A, tm * BM, 0, M, K, wave, lane), make_src<BKM>(B, tn * BN, 0, N, K, wave, lane),
        128 * (wave & 1), 64 * (wave >> 1), wave, lane, tid, arow};
  fill(stage_ptr<0>(), c, 0);
  fill(stage_ptr<1>(), c, 1);
  fill(stage_ptr<2>(), c, 2);
  fill(stage_ptr<3>(), c, 3);
  pre(tm, tn);
  GEMM_WAIT_VM12_LGKM0();
  wg_barrier();
  bf16x8 a0[4], b0[2];
  read_half<AK, BKM>(a0, b0, stage_ptr<0>(), 0, c);
  f32x16 acc[4][2];
  while (true) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};
    for (int kt = 0; kt < nk - 4; kt += 4) {
      step_fill<AK, BKM, 0>(acc, c, c, kt + 4, a0, b0);
      step_fill<AK, BKM, 1>(acc, c, c, kt + 5, a0, b0);
      step_fill<AK, BKM, 2>(acc, c, c, kt + 6, a0, b0);
      step_fill<AK, BKM, 3>(acc, c, c, kt + 7, a0, b0);
    }
    const int t_next = t + (int)gridDim.x;
    const bool has_next = t_next < ntiles;
    int tm_n = 0, tn_n = 0;
    if (has_next) coords(t_next, tm_n, tn_n);
    // Sources of the next tile; with none, extents of 0 make every copy read zeros.
    const Ctx cn{make_src<AK>(A, tm_n * BM, 0, has_next ? M : 0, K, wave, lane),
                 make_src<BKM>(B, tn_n * BN, 0, has_next ? N : 0, K, wave, lane), c.wm0, c.wn0, wave, lane, tid,
                 arow};
    step_fill<AK, BKM, 0>(acc, c, cn, 0, a0, b0);
    step_fill<AK, BKM, 1>(acc, c, cn, 1, a0, b0);
    step_fill<AK, BKM, 2>(acc, c, cn, 2, a0, b0);
    // (The next tile's first fragments are read after the epilogue, so they
    // are not live across it.)
    step_fill<AK, BKM, 3, false>(acc, c, cn, 3, a0, b0);
    epi(acc, tm, tn);
    if (!has_next) break;
    pre(tm_n, tn_n);
    t = t_next;
    tm = tm_n;
    tn = tn_n;
    c = cn;
    read_half<AK, BKM>(a0, b0, stage_ptr<0>(), 0, c);
  }
  GEMM_WAIT_VM0_LGKM0();  // no copy may land in LDS after the workgroup ends
}

// ---- ping-pong main loop ----
//
// The eight waves form two groups, g = wave / 4, with one wave of each group
// on every SIMD.  The groups take turns: while one issues the 16 MFMAs of a
// stage, the other reads the next stage's fragments from LDS and issues its
// share of the copies, and a barrier between the phases hands the matrix
// core to the other group.  The fragment reads and copies of one wave thus
// overlap the other wave's MFMAs instead of both waves reading, then both
// multiplying.  Group 0 copies the A slabs and group 1 the B slabs (each wave
// 4 KB of one operand per stage).  With phase p = 2t + h, stage t is read by
// group 0 in phase 2t - 1 and by group 1 in phase 2t, and multiplied in phases
// 2t and 2t + 1.  Group 0 refills the A half of stage t's buffer with stage
// t + 4 in phase 2t + 1 and group 1 the B half of stage t - 1's buffer with
// stage t + 3 in phase 2t; each memory phase ends waiting for the group's
// copies of the stage read next (vmcnt(8): the two younger stages stay in
// flight) and for its fragment reads, so the following barrier publishes
// both.

struct Src4 {
  const char* base;  // uniform: the operand at the tile origin and k_begin
  int64_t step;      // uniform: bytes per stage
  uint32_t jstep2;   // uniform: bytes from the wave's block j to block j + 2
  uint32_t off[2];   // lane: byte offsets of its chunks in blocks 0 and 1
  int krem[2];       // lane: block j is inside the K range at stage kt iff 32 kt + kj j < krem[j % 2]
  int rowlim;        // lane (K-major): block j is inside the M/N extent iff 16 j < rowlim
};

// As make_src, for the four 1 KB blocks 4 wq .. 4 wq + 3 of a 16 KB slab, in
// a compact form: blocks j and j + 2 of a wave differ by a fixed stride
// (32 rows of a K-major slab, 4 k-rows of an MN-major one) and the same chunk
// swizzle.  (In an MN-major slab the swizzle alternates between even and odd
// blocks, whose k-rows 2j + lane/32 differ in bit 1.)
template <bool KMAJOR>
__device__ __forceinline__ Src4 make_src4(Operand op, int mn0, int k_begin, int MN, int k_end, int wq, int lane) {
  Src4 s;
  const bf16* base;
  if (KMAJOR)
    base = op.blk ? op.p + ((int64_t)(k_begin >> 5) * op.blk + mn0) * 32 : op.p + (int64_t)mn0 * op.ld + k_begin;
  else
    base = op.blk ? op.p + ((int64_t)(mn0 >> 5) * op.blk + k_begin) * 32 : op.p + (int64_t)k_begin * op.ld + mn0;
  s.base = (const char*)base;
  if (KMAJOR) {
    const int row = 64 * wq + (lane >> 2);        // block 0; block j adds 16 j rows
    const int c = (lane & 3) ^ ((row >> 2) & 3);  // the same for the four blocks
    const int64_t rs = op.blk ? 32 : op.ld;       // elements per row
    s.off[0] = 2u * (uint32_t)(row * rs + 8 * c);
    s.off[1] = s.off[0] + 2u * (uint32_t)(16 * rs);
    s.jstep2 = 2u * (uint32_t)(32 * rs);
    s.krem[0] = s.krem[1] = k_end - k_begin - 8 * c;
    s.rowlim = MN - mn0 - row;
  } else {
    const int row0 = 8 * wq + (lane >> 5);  // block j holds k-row row0 + 2j
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = row0 + 2 * p;
      const int c = (lane & 31) ^ (4 * (row & 3));
      const int m = mn0 + 8 * c;
      s.off[p] = 2u * (uint32_t)(op.blk ? ((int64_t)(c >> 2) * op.blk + row) * 32 + 8 * (c & 3)
                                        : (int64_t)row * op.ld + 8 * c);
      s.krem[p] = m < MN ? k_end - k_begin - row0 : 0;
    }
    s.jstep2 = 2u * (uint32_t)(4 * (op.blk ? 32 : op.ld));
    s.rowlim = 64;
  }
  s.step = 2 * (op.blk ? (KMAJOR ? op.blk * 32 : (int64_t)BK * 32) : (KMAJOR ? (int64_t)BK : (int64_t)BK * op.ld));
  return s;
}

template <bool KMAJOR>
__device__ __forceinline__ void issue4(lds_t* slab, const Src4& s, int kt, int wq) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(s.base + kt * s.step, kRsrcRange);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool ok = BK * kt + (KMAJOR ? 0 : 2 * j) < s.krem[j & 1] && (!KMAJOR || 16 * j < s.rowlim);
    const uint32_t off = ok ? s.off[j & 1] + (j >> 1) * s.jstep2 : kOffZero;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(slab + (4 * wq + j) * 512), 16, off, 0, 0, 0);
  }
}

struct Frags {
  bf16x8 a0[4], b0[2], a1[4], b1[2];
};

template <bool AK, bool BKM>
__device__ __forceinline__ void read_stage(Frags& f, const lds_t* st, const Ctx& c) {
  read_half<AK, BKM>(f.a0, f.b0, st, 0, c);
  read_half<AK, BKM>(f.a1, f.b1, st, 1, c);
}

__device__ __forceinline__ void mma_stage(f32x16 (&acc)[4][2], const Frags& f) {
  mma_half(acc, f.a0, f.b0);
  mma_half(acc, f.a1, f.b1);
}

// A phase boundary: the barrier, with the scheduler kept from moving MFMAs or
// fragment reads across it.
__device__ __forceinline__ void pp_barrier() {
  GEMM_SCHED_FENCE();
  wg_barrier();
  GEMM_SCHED_FENCE();
}

// Group 0, stage t in buffer S: multiply stage t, then (memory phase) copy the
// A half of stage dkt of `ds` into buffer S -- stage t + 4 of the stream --,
// run mid(), and read stage t + 1 from buffer S + 1.
template <bool AK, bool BKM, bool kColSum, int S, class Mid>
__device__ __forceinline__ void pp_unit0(f32x16 (&acc)[4][2], Frags& f, const Ctx& c, const Src4& ds, int dkt,
                                         float* colsum, int colsum_period, int colsum_phase, int& colsum_r, Mid mid) {
  mma_stage(acc, f);
  if (kColSum && colsum_period) {
    if (colsum_r == colsum_phase && (c.wave & 1) == 0) colsum_frags(colsum, f.b0, f.b1);
    colsum_r = colsum_r + 1 == colsum_period ? 0 : colsum_r + 1;
  }
  pp_barrier();
  // Unconditional: past the K range the copies read zeros and the reads are
  // unused, and straight-line code keeps the compiler's wait counts exact.
  issue4<AK>(stage_ptr<S>(), ds, dkt, c.wave & 3);
  mid();
  read_stage<AK, BKM>(f, stage_ptr<(S + 1) % 4>(), c);
  GEMM_WAIT_VM8_LGKM0();
  pp_barrier();
}

// Group 1, stage t in buffer S: (memory phase) run mid(), copy the B half of
// stage dkt of `ds` -- stage t + 3 of the stream -- into buffer S - 1, read
// stage t; then multiply it.
template <bool AK, bool BKM, bool kColSum, int S, class Mid>
__device__ __forceinline__ void pp_unit1(f32x16 (&acc)[4][2], Frags& f, const Ctx& c, const Src4& ds, int dkt,
                                         float* colsum, int colsum_period, int colsum_phase, int& colsum_r, Mid mid) {
  mid();
  issue4<BKM>(stage_ptr<(S + 3) % 4>() + OPE, ds, dkt, c.wave & 3);
  read_stage<AK, BKM>(f, stage_ptr<S>(), c);
  GEMM_WAIT_VM8_LGKM0();
  pp_barrier();
  mma_stage(acc, f);
  if (kColSum && colsum_period) {
    if (colsum_r == colsum_phase && (c.wave & 1) == 0) colsum_frags(colsum, f.b0, f.b1);
    colsum_r = colsum_r + 1 == colsum_period ? 0 : colsum_r + 1;
  }
  pp_barrier();
}

struct NoMid {
  __device__ __forceinline__ void operator()() const {}
};

// acc[mb][nb][i] = C[tm0 + wm0 + 32mb + 8(i/4) + 4(lane/32) + i%4][tn0 + wn0 + 32nb + lane%32]
// with wm0 = 128*(wave&1), wn0 = 64*(wave>>1); K range [k_begin, k_end).
// With kColSum and colsum_period > 0, colsum[nb] (two floats per lane) also
// accumulates, in the waves with wave % 2 == 0, the sums of B(k, tn0 + wn0 +
// 32nb + lane%32) over this lane half's k of the stages kt of the K range
// with kt % colsum_period == colsum_phase (see colsum_frags): the workgroups
// that share a B slab split the sums between them.
// kContiguousRows (K-major A only): A rows are read in the contiguous_row
// order, so each lane's accumulator elements 0 .. 15 of a 32-row block are 16
// consecutive rows (16 hl .. 16 hl + 15).
// kLocalAddr: the lane's addresses are derived afresh on each call (the thread
// index passes through an empty asm, the wave index is re-read as a scalar),
// so a kernel that runs several main loops in one outer loop does not keep
// every loop's hoisted addresses live at once.
// On return no copy into the stage arrays is in flight, but other waves may
// still read the last stage: barrier before reusing them.
template <bool AK, bool BKM, bool kColSum = false, bool kContiguousRows = false, bool kLocalAddr = false>
__device__ __forceinline__ void mainloop_pp(f32x16 (&acc)[4][2], Operand A, Operand B, int M, int N, int k_begin,
                                            int k_end, int tm0, int tn0, float* colsum = nullptr,
                                            int colsum_period = 0, int colsum_phase = 0) {
  static_assert(AK || !kContiguousRows, "row permutation needs a K-major A operand");
  int tid = threadIdx.x;
  if (kLocalAddr) asm volatile("" : "+v"(tid));
  // The wave index is kept scalar either way: the group branches below hold
  // barriers and must stay uniform (scalar) branches.
  const int lane = tid & 63, wave = kLocalAddr ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
  const int g = wave >> 2, wq = wave & 3;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};
  const int nk_real = (k_end - k_begin + BK - 1) / BK;
  if (nk_real <= 0) return;
  // Whole groups of four stages: the stages past the K range read zeros and
  // add nothing, and the loop body stays free of conditions.
  const int nk = (nk_real + 3) & ~3;
  const Ctx c{Src{}, Src{}, 128 * (wave & 1), 64 * (wave >> 1), wave, lane, tid,
              kContiguousRows ? contiguous_row(lane & 31) : (lane & 31)};
  int colsum_r = 0;
  Frags f;
  if (g == 0) {
    const Src4 s = make_src4<AK>(A, tm0, k_begin, M, k_end, wq, lane);
    issue4<AK>(stage_ptr<0>(), s, 0, wq);
    issue4<AK>(stage_ptr<1>(), s, 1, wq);
    issue4<AK>(stage_ptr<2>(), s, 2, wq);
    issue4<AK>(stage_ptr<3>(), s, 3, wq);
    GEMM_WAIT_VM8_LGKM0();  // A halves of stages 0 and 1
    pp_barrier();
    read_stage<AK, BKM>(f, stage_ptr<0>(), c);
    GEMM_WAIT_VM8_LGKM0();
    for (int t = 0; t < nk; t += 4) {
      pp_unit0<AK, BKM, kColSum, 0>(acc, f, c, s, t + 4, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
      pp_unit0<AK, BKM, kColSum, 1>(acc, f, c, s, t + 5, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
      pp_unit0<AK, BKM, kColSum, 2>(acc, f, c, s, t + 6, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
      pp_unit0<AK, BKM, kColSum, 3>(acc, f, c, s, t + 7, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
    }
  } else {
    const Src4 s = make_src4<BKM>(B, tn0, k_begin, N, k_end, wq, lane);
    issue4<BKM>(stage_ptr<0>() + OPE, s, 0, wq);
    issue4<BKM>(stage_ptr<1>() + OPE, s, 1, wq);
    issue4<BKM>(stage_ptr<2>() + OPE, s, 2, wq);
    GEMM_WAIT_VM8_LGKM0();  // B half of stage 0
    pp_barrier();
    for (int t = 0; t < nk; t += 4) {
      pp_unit1<AK, BKM, kColSum, 0>(acc, f, c, s, t + 3, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
      pp_unit1<AK, BKM, kColSum, 1>(acc, f, c, s, t + 4, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
      pp_unit1<AK, BKM, kColSum, 2>(acc, f, c, s, t + 5, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
      pp_unit1<AK, BKM, kColSum, 3>(acc, f, c, s, t + 6, colsum, colsum_period, colsum_phase, colsum_r,
                                        NoMid{});
    }
  }
  GEMM_WAIT_VM0_LGKM0();  // no copy may land in LDS after the workgroup ends
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Give XCD x a contiguous range of logical tile ids so that the tiles sharing
// A/B slabs run on the same L2.
__device__ __forceinline__ int xcd_swizzle(int pid, int total) {
  const int q = total >> 3, r = total & 7, x = pid & 7;
  return x * q + min(x, r) + (pid >> 3);
}

// Grouped tile order: `group_m` M-tiles share each N sweep so their B slabs stay in L2.
__device__ __forceinline__ void tile_coords(int pid, int M, int N, int& tm, int& tn, int group_m = kGroupM) {
  const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
  pid = xcd_swizzle(pid, mt * nt);
  const int in_group = group_m * nt;
  const int group = pid / in_group;
  const int first_m = group * group_m;
  const int gsize = min(mt - first_m, group_m);
  tm = first_m + (pid % in_group) % gsize;
  tn = (pid % in_group) / gsize;
}

// (tile, K-split) of a split-K launch of tiles x splits workgroups.  The
// XCD-contiguous logical id runs fastest over the shorter tile dimension, then
// the longer one, then the split: workgroups that run together on one XCD
// share the same K range and the same slab of the long operand, so each slab
// leaves HBM about once instead of once per tile of the short dimension.
__device__ __forceinline__ void split_tile_coords(int pid, int total, int M, int N, int& tm, int& tn, int& split) {
  const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
  const int gid = xcd_swizzle(pid, total);
  if (mt <= nt) {
    tm = gid % mt;
    tn = (gid / mt) % nt;
  } else {
    tn = gid % nt;
    tm = (gid / nt) % mt;
  }
  split = gid / (mt * nt);
}

// ---- host side: launch shaping ----

// Compute units of the current device, looked up once per device (thread-safe:
// concurrent first calls on one device wait for the one lookup).
inline int device_cus() {
  static std::once_flag once[64];
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::call_once(once[dev], [dev] {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cached[dev] = c;
  });
  return cached[dev];
}

// K-split count for a GEMM of `tiles` output tiles over k_iters BK-steps.
// One 256x256 workgroup fills a CU (its LDS use allows no second), so the grid
// runs in ceil(tiles*split/CUs) rounds of k_iters/split steps each, plus one
// fp32 atomic epilogue per round (about 3% of a full-K mainloop).  The split
// minimising that estimate keeps the last round from running a CU-sized
// grid a quarter full, which a fixed split does for skinny outputs.
inline int choose_split(unsigned tiles, int k_iters) {
  const int cus = device_cus();
  const int max_split = k_iters / 8 > 1 ? k_iters / 8 : 1;
  double best = 1e30;
  int best_split = 1;
  for (int s = 1; s <= max_split && s <= 256; ++s) {
    const double rounds = (double)ceil_div((int64_t)tiles * s, (int64_t)cus);
    const double cost = rounds * (1.0 / s + 0.03);
    if (cost < best * 0.999) {
      best = cost;
      best_split = s;
    }
  }
  return best_split;
}

}  // namespace gemm
