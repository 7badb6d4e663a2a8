// Fused linear cross-entropy for gfx950 (rig/kernels/linear_cross_entropy.py).
//
// Every contraction is the bf16 MFMA GEMM core of gemm_core.h with a fused
// epilogue:
//
//   forward  (:115-179)  C = logits^T tile = W_tile h^T (m = vocabulary row,
//            n = token) -> per-token partial (max, sum exp) over the tile's
//            256 vocabulary rows (persistent launch when d % 128 == 0); the
//            target logit h . W[t] in its own pass; a combine pass gives
//            lse and loss = lse - target_logit.  The [n, vocab] logits never
//            exist.
//   backward (:220-302)  per vocabulary chunk (bounded workspace, like the
//            reference's [n, tile] live logits):
//            K1  recompute the logits, write G^T = bf16((exp(logit-lse) - onehot)*ct)
//                as [chunk, n] in 32-token column blocks (gemm::Operand blk),
//                zero for rows >= semantic vocab;
//            K2  dW[chunk] += G^T h;
//            K3  dh       += G W[chunk], rounded to bf16 after the last chunk.
//            One chunk (the whole vocabulary): three launches, K2 and K3 split
//            over their reduction with fp32 atomics.  Several chunks:
//            nchunks + 1 pipelined launches of flce_bwd_pipe_kernel over two
//            halves of the G^T buffer -- launch c runs K2 / K3 of chunk c - 1
//            from one half and K1 of chunk c into the other, its workgroups
//            taking items from per-XCD token-block counters and never
//            waiting for one another (the stream orders the launches).
//   kept-softmax forward / backward (a token chunk at a time, its kept
//            buffer bounded by the caller): the forward also stores fp16
//            exp(logit - max) in 4-row x 32-token groups; the backward
//            rescales them in place to the blocked G^T (no logits recompute)
//            and runs dW (+)= G^T h and dh = G W in one launch
//            (flce_keep_gemms_kernel), split as a host simulation of the
//            dispatch estimates fastest.
#include "gemm_core.h"

#include <math.h>

#include <algorithm>
#include <functional>
#include <mutex>
#include <vector>

namespace {

using gemm::BM;
using gemm::BN;
using gemm::Operand;

// Column nb of a wave's 128-row accumulator block: scale to the log2 domain in
// place and return (max, sum exp2(x - max)) over the 128 rows (both lane halves
// combined).  kMask: rows whose constant part 32mb + 8(i/4) + i%4 is not below
// lim are padding (-inf); the unmasked copy has no per-element compare.
template <bool kMask>
__device__ __forceinline__ float2 column_stats(f32x16 (&acc)[4][2], int nb, int lim) {
  // The masked copy takes lim through an empty asm, so its 64 row compares
  // stay inside the (rarely taken) masked branch: hoisted above it, they ran
  // for every tile and their 64-bit results spilled to VGPR lanes.
  if (kMask) asm volatile("" : "+v"(lim));
  float mx = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float y = (!kMask || 32 * mb + 8 * (i >> 2) + (i & 3) < lim) ? acc[mb][nb][i] * GPTRIG_LOG2E : -INFINITY;
      acc[mb][nb][i] = y;
      mx = fmaxf(mx, y);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float sum = 0.f;
  if (mx != -INFINITY) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) sum += fast_exp2(acc[mb][nb][i] - mx);
  }
  sum += __shfl_xor(sum, 32);
  return make_float2(mx, sum);
}

// Kept probabilities are fp16: values in (0, 1] with 3 more mantissa bits than
// bf16 (what underflows is below 2^-24 of its column's max).
typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));

typedef f16 f16x4 __attribute__((ext_vector_type(4)));

// column_stats that also stores every fp16 exp2(logit * log2(e) - max) of the
// column (this wave's 128 vocabulary rows x one token), for the rows below
// vlim (the storage vocabulary), in the kept layout: rows in groups of 4, a
// group of 32 tokens as 256 contiguous bytes, token-major (element (v, n) at
// ((n / 32) * (Vp / 4) + v / 4) * 128 + (n % 32) * 4 + v % 4, Vp = V rounded
// up to 4).  The lane's 4 consecutive accumulator rows are one 8-byte store;
// col points at its token's slot of the group holding row 0 of its block.
// Nothing is stored for a column with no real row.
template <bool kMask>
__device__ __forceinline__ float2 column_stats_keep(f32x16 (&acc)[4][2], int nb, int lim, int vlim, f16* col) {
  if (kMask) asm volatile("" : "+v"(lim), "+v"(vlim));  // (see column_stats)
  float mx = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float y = (!kMask || 32 * mb + 8 * (i >> 2) + (i & 3) < lim) ? acc[mb][nb][i] * GPTRIG_LOG2E : -INFINITY;
      acc[mb][nb][i] = y;
      mx = fmaxf(mx, y);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  float sum = 0.f;
  if (mx != -INFINITY) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f16x4 p4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float p = fast_exp2(acc[mb][nb][4 * q + t] - mx);
          sum += p;
          p4[t] = (f16)p;
        }
        const int r0 = 32 * mb + 8 * q;  // rows r0 .. r0 + 3 of the lane's block
        f16* dst = col + (r0 / 4) * 128;
        if (!kMask || r0 + 3 < vlim) {
          // Streaming store: the kept array is read back by the next launch,
          // not by this one (measured 7% faster for this launch at 65536
          // tokens than a plain store, which competes with the operand slabs
          // for L2).
          __builtin_nontemporal_store(__builtin_bit_cast(unsigned long long, p4),
                                      reinterpret_cast<unsigned long long*>(dst));
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (r0 + t < vlim) dst[t] = p4[t];
        }
      }
  }
  sum += __shfl_xor(sum, 32);
  return make_float2(mx, sum);
}

// ---------------------------------------------------------------------------
// Forward: partial (max, sum exp) in the log2 domain per token over the tile.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(gemm::THREADS)
    flce_fwd_kernel(Operand W, Operand Hd, int V, int N, int D, int sem_v, float2* __restrict__ partial) {
  __shared__ float2 xchg[4][64];
  int tm, tn;
  gemm::tile_coords(blockIdx.x, V, N, tm, tn);
  f32x16 acc[4][2];
  gemm::mainloop_pp<true, true>(acc, W, Hd, V, N, 0, D, tm * BM, tn * BN);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  const int vbase = tm * BM + 128 * wm;
  const bool full = vbase + 128 <= sem_v;  // no padding row in this wave's 128 rows
  const int lim = sem_v - vbase - 4 * hl;  // row r of the wave's block is real iff its constant part < lim
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = tn * BN + 64 * wn + 32 * nb + l32;
    const float2 st = full ? column_stats<false>(acc, nb, lim) : column_stats<true>(acc, nb, lim);
    const float mx = st.x, sum = st.y;
    if (wm == 1 && hl == 0) xchg[wn][32 * nb + l32] = make_float2(mx, sum);
    __syncthreads();
    if (wm == 0 && hl == 0 && n < N) {
      const float2 o = xchg[wn][32 * nb + l32];
      const float m2 = fmaxf(mx, o.x);
      float s2 = 0.f;
      if (m2 != -INFINITY) s2 = sum * fast_exp2(mx - m2) + o.y * fast_exp2(o.x - m2);
      partial[(size_t)tm * N + n] = make_float2(m2, s2);
    }
    __syncthreads();
  }
}

// Persistent form of the forward for d a multiple of 128 (gemm::persistent):
// one workgroup per CU walks the tiles, copying the next tile's first stages
// while this one's epilogue runs.  Same epilogue as flce_fwd_kernel, with
// LDS-only barriers (a full __syncthreads would wait for those copies).
// kKeep (the kept-softmax forward): every probability exp2(y - m) of the
// tile, m the max over its wave's 128 vocabulary rows, is also stored as fp16
// in the kept layout of column_stats_keep, and m at
// mhalf[(2 tile + half) * N + n], so the backward rescales them (in place,
// into the blocked G^T layout) instead of recomputing the logits.
template <bool kKeep>
__global__ void __launch_bounds__(gemm::THREADS)
    flce_fwd_persistent_kernel(Operand W, Operand Hd, int V, int N, int D, int sem_v, float2* __restrict__ partial,
                               f16* __restrict__ keep, float* __restrict__ mhalf) {
  __shared__ float2 xchg[4][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  const int ntiles = ((V + BM - 1) / BM) * ((N + BN - 1) / BN);
  auto coords = [&](int t, int& tm, int& tn) { gemm::tile_coords(t, V, N, tm, tn); };
  auto pre = [](int, int) {};
  auto epi = [&](f32x16(&acc)[4][2], int tm, int tn) {
    const int vbase = tm * BM + 128 * wm;
    const bool full = vbase + 128 <= sem_v;
    const int lim = sem_v - vbase - 4 * hl;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int n = tn * BN + 64 * wn + 32 * nb + l32;
      float2 st;
      if constexpr (kKeep) {
        // Tokens past N are not stored: their column points at row 0.
        const int vq = (V + 3) / 4;  // row groups per 32-token block
        f16* col = keep + (n < N ? ((size_t)(n >> 5) * vq + (vbase + 4 * hl) / 4) * 128 + (n & 31) * 4 : 0);
        const int vlim = V - vbase - 4 * hl;
        if (n < N)
          st = full ? column_stats_keep<false>(acc, nb, lim, vlim, col)
                    : column_stats_keep<true>(acc, nb, lim, vlim, col);
        else
          st = full ? column_stats<false>(acc, nb, lim) : column_stats<true>(acc, nb, lim);
        if (hl == 0 && n < N) mhalf[(size_t)(2 * tm + wm) * N + n] = st.x;
      } else {
        st = full ? column_stats<false>(acc, nb, lim) : column_stats<true>(acc, nb, lim);
      }
      const float mx = st.x, sum = st.y;
      if (wm == 1 && hl == 0) xchg[wn][32 * nb + l32] = make_float2(mx, sum);
      GPTRIG_WAIT_LGKM0();
      wg_barrier();
      if (wm == 0 && hl == 0 && n < N) {
        const float2 o = xchg[wn][32 * nb + l32];
        const float m2 = fmaxf(mx, o.x);
        float s2 = 0.f;
        if (m2 != -INFINITY) s2 = sum * fast_exp2(mx - m2) + o.y * fast_exp2(o.x - m2);
        partial[(size_t)tm * N + n] = make_float2(m2, s2);
      }
      GPTRIG_WAIT_LGKM0();
      wg_barrier();
    }
  };
  gemm::persistent<true, true>(W, Hd, V, N, D, ntiles, coords, pre, epi);
}

// Target logit h[n] . W[t[n]] (fp32 accumulation of the bf16 products), 0 for
// an invalid target: one wave per token.  Taken out of the GEMM epilogue,
// where a per-element target compare cost more than this pass.
__global__ void __launch_bounds__(256) flce_target_logit_kernel(const bf16* __restrict__ h, const bf16* __restrict__ w,
                                                              const int32_t* __restrict__ targets, int N, int D,
                                                              int sem_v, float* __restrict__ tlogit) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const int t = targets[n];
  float acc = 0.f;
  if (t >= 0 && t < sem_v) {
    for (int c = 8 * lane; c < D; c += 512) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(h + (size_t)n * D + c);
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(w + (size_t)t * D + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf((float)a[j], (float)b[j], acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) tlogit[n] = acc;
}

// lse[n] (natural log) from the per-tile partials; loss = lse - target logit,
// +inf for an invalid target (:159-172).
// One (max, sum) pair folded into another (log2 domain); empty pairs (max
// -inf, tiles past the semantic vocabulary) are skipped.
__device__ __forceinline__ void lse_fold(float& m, float& s, float pm, float ps) {
  if (pm == -INFINITY) return;
  const float m2 = fmaxf(m, pm);
  s = s * fast_exp2(m - m2) + ps * fast_exp2(pm - m2);
  m = m2;
}

// 64 tokens per workgroup (lane = token), each of the kCombineWaves waves
// folding every kCombineWaves-th tile, the partial pairs then folded through
// LDS: many waves per CU with independent loads instead of one serial chain
// per token.
template <int kCombineWaves>
__global__ void __launch_bounds__(64 * kCombineWaves)
    flce_combine_kernel(const float2* __restrict__ partial, int ntiles, int N, int sem_v,
                        const int32_t* __restrict__ targets, const float* __restrict__ tlogit,
                        float* __restrict__ lse, float* __restrict__ losses) {
  __shared__ float2 part_s[kCombineWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + lane;
  float m = -INFINITY, s = 0.f;
  if (n < N) {
    int t = wave;
    for (; t + kCombineWaves < ntiles; t += 2 * kCombineWaves) {  // two loads in flight
      const float2 p0 = partial[(size_t)t * N + n];
      const float2 p1 = partial[(size_t)(t + kCombineWaves) * N + n];
      lse_fold(m, s, p0.x, p0.y);
      lse_fold(m, s, p1.x, p1.y);
    }
    if (t < ntiles) {
      const float2 p0 = partial[(size_t)t * N + n];
      lse_fold(m, s, p0.x, p0.y);
    }
  }
  part_s[wave][lane] = float2{m, s};
  __syncthreads();
  if (wave != 0 || n >= N) return;
#pragma unroll
  for (int w = 1; w < kCombineWaves; ++w) lse_fold(m, s, part_s[w][lane].x, part_s[w][lane].y);
  const float l = (m + __log2f(s)) * GPTRIG_LN2;
  lse[n] = l;
  const int t = targets[n];
  losses[n] = (t >= 0 && t < sem_v) ? l - tlogit[n] : INFINITY;
}

// ---------------------------------------------------------------------------
// Backward K1: G^T[v - v0][n] = bf16((exp(logit - lse[n]) - [v == t]) * ct[n]),
// zero for v >= semantic vocab; ct is zero for invalid targets (:236-240).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(gemm::THREADS)
    flce_grad_kernel(Operand W, Operand Hd, int Vc, int N, int D, int v0, int sem_v,
                     const int32_t* __restrict__ targets, const float* __restrict__ lse,
                     const float* __restrict__ cot, float cot_scale, bf16* __restrict__ gt) {
  int tm, tn;
  // Two vocabulary tiles per token sweep: measured 4% faster for this launch
  // than groups of 8 (the G^T stores compete with the operand slabs for L2).
  gemm::tile_coords(blockIdx.x, Vc, N, tm, tn, 2);
  f32x16 acc[4][2];
  gemm::mainloop_pp<true, true>(acc, W, Hd, Vc, N, 0, D, tm * BM, tn * BN);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  // The bf16 G^T tile is staged through the (now idle) stage arrays, one
  // 64-row x 256-column band per array, then written out as 16-byte rows:
  // the accumulator layout would otherwise need 2-byte stores.
  wg_barrier();  // every wave is done reading the last stage
  gemm::lds_t* const band[4] = {gemm::stage_ptr<0>(), gemm::stage_ptr<1>(), gemm::stage_ptr<2>(),
                                gemm::stage_ptr<3>()};
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int nc = 64 * wn + 32 * nb + l32;  // column within the tile
    const int n = tn * BN + nc;
    const bool n_ok = n < N;
    const int t = n_ok ? targets[n] : -1;
    const bool valid_t = t >= 0 && t < sem_v;
    const float ct = valid_t ? (cot ? cot[n] : cot_scale) : 0.f;
    const float l2 = n_ok ? lse[n] * GPTRIG_LOG2E : 0.f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 128 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);  // row within the tile
        const int v = v0 + tm * BM + r;
        float g = 0.f;
        if (v < sem_v) {
          const float p = fast_exp2(acc[mb][nb][i] * GPTRIG_LOG2E - l2);
          g = (p - (v == t ? 1.f : 0.f)) * ct;
        }
        band[r >> 6][(r & 63) * 256 + nc] = (bf16)g;
      }
  }
  GPTRIG_WAIT_LGKM0();
  wg_barrier();
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int idx = tid + gemm::THREADS * j;  // 256 rows x 32 chunks of 8
    const int r = idx >> 5, c = idx & 31;
    const int vl = tm * BM + r;
    const int n = tn * BN + 8 * c;
    // Streaming (non-temporal) stores: G^T is read back by the next two
    // launches, not by this one, so it need not displace the W / h slabs
    // in L2.
    if (vl < Vc && n < N) {
      const bf16x8 g8 = *(const gemm::lds_x8*)(band[r >> 6] + (r & 63) * 256 + 8 * c);
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, g8),
                                  reinterpret_cast<u32x4*>(gt + ((size_t)(n >> 5) * Vc + vl) * 32 + (n & 31)));
    }
  }
}

// Persistent form of K1 for d a multiple of 128 (gemm::persistent), computing
// the transposed product: m = token, n = vocabulary row.  The token rows are
// read in gemm::contiguous_row order, so each lane's 16 accumulator elements
// of a 32-token block are 16 consecutive tokens of one vocabulary row, written
// to G^T as two 16-byte stores straight from registers (the stage arrays stay
// free for the next tile's copies); in the natural row order a lane held four
// runs of 4 tokens and needed four 8-byte stores (measured 0.7% slower for the
// FLCE backward).  Per-token lse / cotangent / target are staged in
// LDS, double-buffered by tile parity and loaded a tile ahead.  Tiles are
// walked four vocabulary tiles per token sweep: the 32 workgroups of an XCD
// then share 4 W slabs and 8 h slabs per round, which cuts this launch's HBM
// fetch at N = 65536 from 19.7 GB (one vocabulary tile per sweep: 32 h slabs
// per round, h re-read from HBM for every vocabulary tile) to 7.3 GB, at the
// same time (13.52 vs 13.51 ms for the whole FLCE backward; eight per sweep
// fetches 7.4 GB and takes 13.61 ms).  The launch is bound by its MFMA
// mainloop and softmax epilogue, not by HBM.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(gemm::THREADS)
    flce_grad_persistent_kernel(Operand W, Operand Hd, int Vc, int N, int D, int v0, int sem_v,
                                const int32_t* __restrict__ targets, const float* __restrict__ lse,
                                const float* __restrict__ cot, float cot_scale, bf16* __restrict__ gt) {
  __shared__ __attribute__((aligned(16))) float l2_s[2][BM];
  __shared__ __attribute__((aligned(16))) float ct_s[2][BM];
  __shared__ __attribute__((aligned(16))) int t_s[2][BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  const int ntiles = ((Vc + BM - 1) / BM) * ((N + BN - 1) / BN);
  int pre_it = 0, epi_it = 0;
  auto coords = [&](int t, int& tm, int& tn) {
    int tv, tt;
    gemm::tile_coords(t, Vc, N, tv, tt, 4);
    tm = tt;  // token tile
    tn = tv;  // vocabulary tile
  };
  auto pre = [&](int tm, int) {
    const int b = pre_it & 1;
    ++pre_it;
    if (tid < BM) {
      const int n = tm * BM + tid;
      const bool n_ok = n < N;
      const int t = n_ok ? targets[n] : -1;
      const bool valid_t = t >= 0 && t < sem_v;
      t_s[b][tid] = t;
      ct_s[b][tid] = valid_t ? (cot ? cot[n] : cot_scale) : 0.f;
      l2_s[b][tid] = n_ok ? lse[n] * GPTRIG_LOG2E : 0.f;
    }
  };
  auto epi = [&](f32x16(&acc)[4][2], int tm, int tn) {
    const int b = epi_it & 1;
    ++epi_it;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int r0 = 128 * wm + 32 * mb + 16 * hl;  // this lane's 16 consecutive tokens of the tile
      const int n = tm * BM + r0;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int vl = tn * BN + 64 * wn + 32 * nb + l32;
        const int v = v0 + vl;
        bf16* dst = gt + ((size_t)(n >> 5) * Vc + vl) * 32 + (n & 31);
#pragma unroll
        for (int h8 = 0; h8 < 2; ++h8) {
          // Per-token values re-read from LDS for each 8-token half (the
          // empty asm keeps the compiler from merging the reads across
          // halves and holding 48 registers through the epilogue).
          asm volatile("" ::: "memory");
          const int rq = r0 + 8 * h8;
          const f32x4 la = *reinterpret_cast<const f32x4*>(&l2_s[b][rq]);
          const f32x4 lb = *reinterpret_cast<const f32x4*>(&l2_s[b][rq + 4]);
          const f32x4 ca = *reinterpret_cast<const f32x4*>(&ct_s[b][rq]);
          const f32x4 cb = *reinterpret_cast<const f32x4*>(&ct_s[b][rq + 4]);
          const i32x4_t ta = *reinterpret_cast<const i32x4_t*>(&t_s[b][rq]);
          const i32x4_t tb = *reinterpret_cast<const i32x4_t*>(&t_s[b][rq + 4]);
          bf16x8 o;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float l2 = j < 4 ? la[j & 3] : lb[j & 3];
            const float ct = j < 4 ? ca[j & 3] : cb[j & 3];
            const int tt = j < 4 ? ta[j & 3] : tb[j & 3];
            float g = 0.f;
            if (v < sem_v) {
              const float p = fast_exp2(acc[mb][nb][8 * h8 + j] * GPTRIG_LOG2E - l2);
              g = (p - (v == tt ? 1.f : 0.f)) * ct;
            }
            o[j] = (bf16)g;
          }
          // n + 8 h8 is a multiple of 8, as is N: each half is wholly in or out of range.
          // (Plain stores: non-temporal ones measured 1.5% slower here.)
          if (vl < Vc && n + 8 * h8 < N) *reinterpret_cast<bf16x8*>(dst + 8 * h8) = o;
        }
      }
    }
  };
  gemm::persistent<true, true, true>(Hd, W, N, Vc, D, ntiles, coords, pre, epi);
}

// C (fp32, row-major [M][ldc]) = / += / atomic+= A B over K range of this split.
// mode 0: store, 1: accumulate (read-modify-write), 2: atomic add.
// colsum (nullable): colsum[n] atomic+= sum over this split's
// K range of B(k, n), computed from the B fragments already in registers and shared out
// over the M tiles (the bias gradient of a linear layer, fused into its
// weight gradient).
// One workgroup's tile (tm, tn) of that product over [k_begin, k_end).
template <bool AK, bool BKM>
__device__ __forceinline__ void gemm_f32_tile(Operand A, Operand B, int M, int N, int k_begin, int k_end, int tm,
                                              int tn, float* __restrict__ C, int64_t ldc, int mode,
                                              float* __restrict__ colsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  f32x16 acc[4][2];
  float csum[2] = {0.f, 0.f};
  // Every M tile of a (tn, split) sums a share of the B stages, so the
  // column sums cost each workgroup the same.
  const bool do_colsum = colsum != nullptr;
  gemm::mainloop_pp<AK, BKM, true>(acc, A, B, M, N, k_begin, k_end, tm * BM, tn * BN, csum,
                                   do_colsum ? (M + BM - 1) / BM : 0, tm);
  if (k_begin >= k_end) return;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  if (do_colsum && wm == 0) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float t = csum[nb] + __shfl_xor(csum[nb], 32);
      const int n = tn * BN + 64 * wn + 32 * nb + l32;
      if (hl == 0 && n < N) atomicAdd(colsum + n, t);
    }
  }
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = tn * BN + 64 * wn + 32 * nb + l32;
    if (n >= N) continue;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int m0 = tm * BM + 128 * wm + 32 * mb + 4 * hl;
      float* const dst = C + (int64_t)m0 * ldc + n;
      auto row = [&](int i) { return 8 * (i >> 2) + (i & 3); };
      if (mode == 1) {
        // Read-modify-write: the block's 16 reads are issued together, so
        // their latencies overlap instead of each add waiting for its read.
        float old[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) old[i] = m0 + row(i) < M ? dst[(int64_t)row(i) * ldc] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (m0 + row(i) < M) dst[(int64_t)row(i) * ldc] = old[i] + acc[mb][nb][i];
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (m0 + row(i) >= M) continue;
          if (mode == 2)
            atomicAdd(dst + (int64_t)row(i) * ldc, acc[mb][nb][i]);
          else
            dst[(int64_t)row(i) * ldc] = acc[mb][nb][i];
        }
      }
    }
  }
}

// K range [k_begin, k_end) of split `split` when K is cut into ksplit slices of whole stages.
__device__ __forceinline__ void split_range(int K, int ksplit, int split, int& k_begin, int& k_end) {
  const int kslice = ((K + ksplit - 1) / ksplit + gemm::BK - 1) / gemm::BK * gemm::BK;
  k_begin = split * kslice;
  k_end = min(K, k_begin + kslice);
}

template <bool AK, bool BKM>
__global__ void __launch_bounds__(gemm::THREADS)
    gemm_f32_kernel(Operand A, Operand B, int M, int N, int K, int ksplit, float* __restrict__ C, int64_t ldc,
                    int mode, float* __restrict__ colsum) {
  int tm, tn, split, k_begin, k_end;
  gemm::split_tile_coords(blockIdx.x, gridDim.x, M, N, tm, tn, split);
  split_range(K, ksplit, split, k_begin, k_end);
  gemm_f32_tile<AK, BKM>(A, B, M, N, k_begin, k_end, tm, tn, C, ldc, mode, colsum);
}

// The two gradient GEMMs of the kept-softmax backward in one launch, so that
// neither leaves the GPU part-empty while the other waits behind it:
//   dh (+)= G W   A(m = token, k = v) = G^T blocked (MN-major), B = W [V][d] (MN-major),
//                 split over the vocabulary into dh_split slices (fp32 atomics, or a plain
//                 store with one slice);
//   dW (+)= G^T h A = G^T blocked (K-major), B = h [n][d] (MN-major), split over the tokens
//                 into dw_split slices (mode dw_mode).
// Workgroups [0, first) run the items of the group with the longer items
// (dh_first: the dh items), the rest the other group's: the dispatcher hands
// the long items out first and the short ones fill the CUs that free up.
__global__ void __launch_bounds__(gemm::THREADS)
    flce_keep_gemms_kernel(Operand Gt, Operand Wv, Operand Hd, int n, int d, int vc, int dh_split, int dw_split,
                           float* __restrict__ dh_acc, int dh_mode, float* __restrict__ dw, int dw_mode, int n_dh,
                           int n_dw, bool dh_first) {
  const int b = blockIdx.x;
  const bool is_dh = dh_first ? b < n_dh : b >= n_dw;
  const int pid = dh_first ? (is_dh ? b : b - n_dh) : (is_dh ? b - n_dw : b);
  int tm, tn, split, k_begin, k_end;
  if (is_dh) {
    gemm::split_tile_coords(pid, n_dh, n, d, tm, tn, split);
    split_range(vc, dh_split, split, k_begin, k_end);
    gemm_f32_tile<false, false>(Gt, Wv, n, d, k_begin, k_end, tm, tn, dh_acc, d, dh_mode, nullptr);
  } else {
    gemm::split_tile_coords(pid, n_dw, vc, d, tm, tn, split);
    split_range(n, dw_split, split, k_begin, k_end);
    gemm_f32_tile<true, false>(Gt, Hd, vc, d, k_begin, k_end, tm, tn, dw, d, dw_mode, nullptr);
  }
}

// ---------------------------------------------------------------------------
// Chunked backward (more than one vocabulary chunk): pipelined launches.
//
// The workspace's bf16 [n, chunk] G^T buffer is used as two halves of C rows
// each (C = chunk / 2, a multiple of 256).  Launch c (c = 0 .. nchunks) is one
// persistent grid whose workgroups take work items from atomic counters:
//   K2 (c-1, r, dt)   dW[chunk c-1, tile r][d tile dt] += G^T[tile r, token block] h[token block][dt]
//                     (fp32 atomics, one add per token block)
//   K3 (c-1, nt, dt)  dh[token tile nt][d tile dt] (+)= G[nt, chunk c-1] W[chunk c-1][dt]
//                     (f32 store on the first chunk, no-return f32 atomics
//                     after; one conversion to bf16 after the last launch)
//   K1 (c, r, nt)     G^T tile of chunk c, into the other half
// The tokens are cut into 8 blocks of ks tokens, one per XCD: workgroup b
// takes the items of block b % 8 from that block's counter (workgroups are
// dispatched round-robin over the XCDs), so a block's h rows, G^T columns
// and dh rows are read under one L2.  Nothing in a launch depends on anything
// else in it (K1 writes the half that K2 / K3 do not read) and the stream
// orders the launches, so no workgroup ever waits for another: each takes
// items until its counter passes the block's item count and exits.  The grid
// is a multiple of 8, so every block's counter is served.
// ---------------------------------------------------------------------------
constexpr int kBlocks = 8;  // token blocks = XCDs

struct PipeLaunch {
  const bf16* h;  // [N][d]
  const bf16* w;  // [V][d]
  const int32_t* targets;
  const float* lse;
  const float* cot;
  float cot_scale;
  bf16* gt1;         // half written by K1 (chunk c1): element (v, n) at ((n / 32) * C + v) * 32 + n % 32
  const bf16* gt23;  // half read by K2 / K3 (chunk c23)
  float* dh_acc;     // f32 [N][d]
  float* dw;         // f32 [V][d]
  int* counter;      // this launch's kBlocks item counters (zero before the launch)
  int N, D, V, sem_v, C, nchunks, ks, c1, c23;
};

__host__ __device__ inline int pipe_rows(const PipeLaunch& p, int c) { return min(p.C, p.V - c * p.C); }
__host__ __device__ inline int pipe_ndt(const PipeLaunch& p) { return (p.D + BN - 1) / BN; }
// Token tiles of block q (0 past the last block).
__host__ __device__ inline int pipe_ntn(const PipeLaunch& p, int q) {
  const int len = min(p.ks, p.N - q * p.ks);
  return len > 0 ? (len + BM - 1) / BM : 0;
}
__host__ __device__ inline int pipe_k2_items(const PipeLaunch& p, int q) {
  return p.c23 < 0 || pipe_ntn(p, q) == 0 ? 0 : (pipe_rows(p, p.c23) + BM - 1) / BM * pipe_ndt(p);
}
__host__ __device__ inline int pipe_k3_items(const PipeLaunch& p, int q) {
  return p.c23 < 0 ? 0 : pipe_ntn(p, q) * pipe_ndt(p);
}
__host__ __device__ inline int pipe_k1_items(const PipeLaunch& p, int q) {
  return p.c1 < 0 ? 0 : (pipe_rows(p, p.c1) + BM - 1) / BM * pipe_ntn(p, q);
}
__host__ __device__ inline int pipe_items(const PipeLaunch& p, int q) {
  return pipe_k2_items(p, q) + pipe_k3_items(p, q) + pipe_k1_items(p, q);
}

struct PipeItem {
  int type;  // 0 = K1 (a = vocab tile, b = token tile), 1 = K2 (a = vocab tile, b = d tile),
             // 2 = K3 (a = token tile, b = d tile); token tiles are global
  int a, b;
};

// Item j of block q: the K2 items (d tile fastest, so consecutive items share
// their G^T rows), then the K3 items (d tile fastest, sharing G rows), then
// the K1 tiles (token tile fastest, sharing a W tile).
__host__ __device__ inline PipeItem pipe_decode(const PipeLaunch& p, int q, int j) {
  PipeItem it;
  const int ndt = pipe_ndt(p);
  const int nt0 = q * (p.ks / BM);
  const int n2 = pipe_k2_items(p, q), n3 = pipe_k3_items(p, q);
  if (j < n2) {
    it.type = 1;
    it.a = j / ndt;
    it.b = j % ndt;
  } else if (j < n2 + n3) {
    j -= n2;
    it.type = 2;
    it.a = nt0 + j / ndt;
    it.b = j % ndt;
  } else {
    j -= n2 + n3;
    const int ntn = pipe_ntn(p, q);
    it.type = 0;
    it.a = j / ntn;
    it.b = nt0 + j % ntn;
  }
  return it;
}

__global__ void __launch_bounds__(gemm::THREADS) flce_bwd_pipe_kernel(PipeLaunch p) {
  __shared__ int item_s;
  __shared__ __attribute__((aligned(16))) float l2_s[BM];
  __shared__ __attribute__((aligned(16))) float ct_s[BM];
  __shared__ __attribute__((aligned(16))) int t_s[BM];
  const int tid = threadIdx.x;
  const int q = blockIdx.x % kBlocks;
  const int total = pipe_items(p, q);
  for (;;) {
    if (tid == 0) item_s = atomicAdd(p.counter + q, 1);
    __syncthreads();
    // Uniform: read into a scalar register, so the decode stays in SGPRs.
    const int j = __builtin_amdgcn_readfirstlane(item_s);
    if (j >= total) break;
    const PipeItem it = pipe_decode(p, q, j);
    // Lane coordinates derived per item (see gemm::mainloop_pp's kLocalAddr);
    // the wave index stays scalar.
    int tid_l = tid;
    asm volatile("" : "+v"(tid_l));
    const int lane = tid_l & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_l >> 6);
    const int hl = lane >> 5, l32 = lane & 31;
    const int wm = wave & 1, wn = wave >> 1;
    if (it.type == 0) {
      // K1: G^T tile = (exp(logit - lse) - onehot) * ct, token tile b, vocabulary tile a of chunk c1.
      const int v0 = p.c1 * p.C, vc = pipe_rows(p, p.c1);
      const int n0 = it.b * BN;
      if (tid < BM) {
        const int n = n0 + tid;
        const bool n_ok = n < p.N;
        const int t = n_ok ? p.targets[n] : -1;
        const bool valid_t = t >= 0 && t < p.sem_v;
        t_s[tid] = t;
        ct_s[tid] = valid_t ? (p.cot ? p.cot[n] : p.cot_scale) : 0.f;
        l2_s[tid] = n_ok ? p.lse[n] * GPTRIG_LOG2E : 0.f;
      }
      f32x16 acc[4][2];
      gemm::mainloop_pp<true, true, false, true, true>(acc, Operand{p.h, p.D}, Operand{p.w + (size_t)v0 * p.D, p.D},
                                                       p.N, vc, 0, p.D, n0, it.a * BN);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int r0 = 128 * wm + 32 * mb + 16 * hl;  // this lane's 16 consecutive tokens of the tile
        const int n = n0 + r0;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int vl = it.a * BN + 64 * wn + 32 * nb + l32;
          const int v = v0 + vl;
          bf16* dst = p.gt1 + ((size_t)(n >> 5) * p.C + vl) * 32 + (n & 31);
#pragma unroll
          for (int h8 = 0; h8 < 2; ++h8) {
            asm volatile("" ::: "memory");
            const int rq = r0 + 8 * h8;
            const f32x4 la = *reinterpret_cast<const f32x4*>(&l2_s[rq]);
            const f32x4 lb = *reinterpret_cast<const f32x4*>(&l2_s[rq + 4]);
            const f32x4 ca = *reinterpret_cast<const f32x4*>(&ct_s[rq]);
            const f32x4 cb = *reinterpret_cast<const f32x4*>(&ct_s[rq + 4]);
            const i32x4_t ta = *reinterpret_cast<const i32x4_t*>(&t_s[rq]);
            const i32x4_t tb = *reinterpret_cast<const i32x4_t*>(&t_s[rq + 4]);
            bf16x8 o;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
              const float l2 = jj < 4 ? la[jj & 3] : lb[jj & 3];
              const float ct = jj < 4 ? ca[jj & 3] : cb[jj & 3];
              const int tt = jj < 4 ? ta[jj & 3] : tb[jj & 3];
              float g = 0.f;
              if (v < p.sem_v) {
                const float pr = fast_exp2(acc[mb][nb][8 * h8 + jj] * GPTRIG_LOG2E - l2);
                g = (pr - (v == tt ? 1.f : 0.f)) * ct;
              }
              o[jj] = (bf16)g;
            }
            // n + 8 h8 and N are multiples of 8: each half is wholly in or out of range.
            if (vl < vc && n + 8 * h8 < p.N) *reinterpret_cast<bf16x8*>(dst + 8 * h8) = o;
          }
        }
      }
    } else if (it.type == 1) {
      // K2: dW[chunk c23, tile a][d tile b] += G^T[tile a, token block q] h[token block q][d tile b].
      const int v0 = p.c23 * p.C, vc = pipe_rows(p, p.c23);
      const int k0 = q * p.ks, k1 = min(p.N, k0 + p.ks);
      f32x16 acc[4][2];
      gemm::mainloop_pp<true, false, false, false, true>(acc, Operand{p.gt23, p.N, p.C}, Operand{p.h, p.D}, vc, p.D,
                                                         k0, k1, it.a * BM, it.b * BN);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int n = it.b * BN + 64 * wn + 32 * nb + l32;
        if (n >= p.D) continue;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int m = it.a * BM + 128 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
            if (m < vc) atomicAdd(p.dw + (size_t)(v0 + m) * p.D + n, acc[mb][nb][i]);
          }
      }
    } else {
      // K3: dh[token tile a][d tile b] (+)= G[a, chunk c23] W[chunk c23][d tile b].
      const int v0 = p.c23 * p.C, vc = pipe_rows(p, p.c23);
      const int n0 = it.a * BM;
      f32x16 acc[4][2];
      gemm::mainloop_pp<false, false, false, false, true>(acc, Operand{p.gt23, p.N, p.C},
                                                          Operand{p.w + (size_t)v0 * p.D, p.D}, p.N, p.D, 0, vc, n0,
                                                          it.b * BN);
      // The first chunk stores; later chunks add with no-return atomics (the
      // items of one launch write disjoint tiles and the stream orders the
      // launches, so these adds never race: the atomic form only avoids a
      // load round trip per element).  dh is converted after the last launch.
      const bool first = p.c23 == 0;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int n = it.b * BN + 64 * wn + 32 * nb + l32;
        if (n >= p.D) continue;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int m = n0 + 128 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
            if (m >= p.N) continue;
            const size_t o = (size_t)m * p.D + n;
            if (first)
              p.dh_acc[o] = acc[mb][nb][i];
            else
              atomicAdd(p.dh_acc + o, acc[mb][nb][i]);
          }
      }
    }
    // Every wave is done with this item's LDS (stage arrays, per-token data
    // and item_s) before the next item is taken.
    __syncthreads();
  }
}

__global__ void f32_to_bf16_kernel(const float* __restrict__ x, bf16* __restrict__ y, int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n) {
    f32x4 v = *reinterpret_cast<const f32x4*>(x + i);
    bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
    *reinterpret_cast<bf16x4*>(y + i) = o;
  } else {
    for (; i < n; ++i) y[i] = (bf16)x[i];
  }
}

__global__ void zero_f32_kernel(float* __restrict__ x, int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n)
    *reinterpret_cast<f32x4*>(x + i) = f32x4{};
  else
    for (; i < n; ++i) x[i] = 0.f;
}

inline unsigned tiles_of(int M, int N) { return (unsigned)(ceil_div(M, BM) * ceil_div(N, BN)); }

// Default vocabulary chunk of the backward: the reference's default tile
// (rig/kernels/linear_cross_entropy.py:41, DEFAULT_VOCAB_TILE_SIZE = 2048), so
// the bf16 G^T workspace is at most [n, 2048] unless the caller asks for more.
constexpr int kDefaultChunk = 2048;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int resolve_chunk(int vocab, int vocab_chunk) {
  const int chunk = vocab_chunk > 0 ? vocab_chunk : kDefaultChunk;
  const int full = ceil_div(vocab, BM) * BM;
  return chunk > full ? full : chunk;
}

// Pipelined chunk layout: two halves of `half` vocabulary rows each inside the
// [n, chunk] G^T buffer (chunk >= 512; else one buffer of `chunk` rows and
// alternating launches), and the per-XCD token blocks of ks tokens.
struct PipeShape {
  int half, nchunks, ks;
};

PipeShape pipe_shape(int n, int vocab, int rows) {
  PipeShape s;
  s.half = rows;
  s.nchunks = ceil_div(vocab, rows);
  s.ks = ceil_div(ceil_div(n, kBlocks), BM) * BM;
  return s;
}

__global__ void zero_i32_kernel(int* __restrict__ x, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = 0;
}

// Scratch of gptrig_flce_fwd_noalloc: a file-scope device array, so that
// entry point allocates nothing.  Each GPU the library runs on holds its own
// copy, at its own address, until the process ends.  The host never passes
// the array's name to a kernel (in host code it is only a handle): the device
// address comes from hipGetSymbolAddress, taken once per device with that
// device current.
static __device__ __align__(256) unsigned char scratch[GPTRIG_FLCE_FWD_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device (nullptr if the device
// index is out of range or the runtime call fails).
void* scratch_ptr() {
  static std::once_flag once[kMaxDevices];
  static void* ptr[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::call_once(once[dev], [dev] {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) ptr[dev] = p;
  });
  return ptr[dev];
}

// The forward's launches (validated inputs, workspace of at least
// gptrig_flce_fwd_workspace_bytes), shared by the entry points; keep (with d
// a multiple of 128) also stores the kept softmax of gptrig_flce_fwd_keep.
int flce_fwd_launch(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                    void* workspace, int n, int d, int vocab, int semantic_vocab, hipStream_t s,
                    void* keep = nullptr);

// Kept-softmax buffer: the G^T array of the one-chunk backward ([ceil(n/32)]
// blocks of [vocab][32]; fp16 probabilities from the forward, rewritten in
// place as the bf16 gradient), then the f32 per-(half tile, token) maxima
// [2 ceil(vocab/256)][n].
// Rows of the kept / G^T blocks: the vocabulary rounded up to a group of 4.
int keep_rows(int vocab) { return (vocab + 3) / 4 * 4; }
size_t keep_gt_bytes(int n, int vocab) {
  return align256((size_t)keep_rows(vocab) * ceil_div(n, 32) * 32 * sizeof(bf16));
}

// Backward from the kept softmax, step 1: the per-(half tile, token) maxima m
// become the factors a = exp2(m - lse log2(e)) ct of their probabilities (in
// place), ct the token's cotangent (0 for an invalid target).
// blockIdx.y = the half tile, 4 tokens per thread (N % 8 == 0 on this path,
// so a group of 4 is wholly in or out and 16-byte aligned).
__global__ void flce_keep_alpha_kernel(float* __restrict__ mh, int halves, int N, int sem_v,
                                       const int32_t* __restrict__ targets, const float* __restrict__ lse,
                                       const float* __restrict__ cot, float cot_scale) {
  const int n0 = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (n0 >= N) return;
  float* row = mh + (size_t)blockIdx.y * N + n0;
  const f32x4 m = *reinterpret_cast<const f32x4*>(row);
  const i32x4_t t = *reinterpret_cast<const i32x4_t*>(targets + n0);  // (targets is checked 16-byte aligned)
  f32x4 a;
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // lse and cot: scalar reads, no alignment asked of the caller
    const float ct = (t[j] >= 0 && t[j] < sem_v) ? (cot ? cot[n0 + j] : cot_scale) : 0.f;
    a[j] = m[j] == -INFINITY ? 0.f : fast_exp2(m[j] - lse[n0 + j] * GPTRIG_LOG2E) * ct;
  }
  *reinterpret_cast<f32x4*>(row) = a;
}

// Step 2: G^T[v][n] = bf16(p a - [v == t] ct), zero for v >= semantic vocab
// (K1's values, from the kept fp16 p instead of recomputed logits), in place:
// each 256-byte group (4 rows x 32 tokens, token-major) becomes the same 256
// bytes of the blocked G^T layout (element (v, n) at ((n / 32) Vp + v) 32 +
// n % 32).  16 consecutive lanes take one group, 16 bytes (2 tokens x 4 rows)
// each, and all of a group's loads precede its stores (one wave, one load
// instruction), so the in-place transpose never reads a rewritten byte.
__global__ void __launch_bounds__(256)
    flce_keep_rescale_kernel(bf16* __restrict__ gt, const float* __restrict__ alpha, int N, int V, int sem_v,
                             const int32_t* __restrict__ targets, const float* __restrict__ cot, float cot_scale) {
  const int vq = (V + 3) / 4;
  const int gid = blockIdx.x * 16 + (threadIdx.x >> 4);  // row group of this 32-token block
  if (gid >= vq) return;  // whole 16-lane groups leave together
  const int blk = blockIdx.y, j = threadIdx.x & 15;
  const int n = 32 * blk + 2 * j;
  const int v0 = 4 * gid;
  bf16* grp = gt + ((size_t)blk * vq + gid) * 128;
  const f16x8 p = *reinterpret_cast<const f16x8*>(grp + 8 * j);  // tokens n, n + 1 x rows v0 .. v0 + 3
  if (n >= N) return;  // N % 8 == 0: both tokens are in or out
  bf16x2 o[4] = {};
  if (v0 < sem_v) {
    const float2 a = *reinterpret_cast<const float2*>(alpha + (size_t)(2 * (v0 >> 8) + ((v0 >> 7) & 1)) * N + n);
    const int2 t = *reinterpret_cast<const int2*>(targets + n);
    const float c0 = cot ? cot[n] : cot_scale, c1 = cot ? cot[n + 1] : cot_scale;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int v = v0 + r;
      if (v >= sem_v) continue;
      float g0 = (float)p[r] * a.x, g1 = (float)p[4 + r] * a.y;
      if (t.x == v) g0 -= c0;  // t == v < sem_v: a valid target
      if (t.y == v) g1 -= c1;
      o[r] = bf16x2{(bf16)g0, (bf16)g1};
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) *reinterpret_cast<bf16x2*>(grp + r * 32 + 2 * j) = o[r];
}

}  // namespace

extern "C" {

size_t gptrig_flce_fwd_workspace_bytes(int n, int d, int vocab) {
  (void)d;
  const size_t ntiles = (size_t)ceil_div(vocab, BM);
  return align256(ntiles * n * sizeof(float2)) + align256((size_t)n * sizeof(float));
}

int gptrig_flce_fwd(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                    void* workspace, size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab,
                    void* stream) {
  if (!hidden || !weight || !targets || !losses || !lse || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (workspace_bytes < gptrig_flce_fwd_workspace_bytes(n, d, vocab)) return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)workspace) & 15) return GPTRIG_E_SHAPE;
  return flce_fwd_launch(hidden, weight, targets, losses, lse, workspace, n, d, vocab, semantic_vocab,
                         (hipStream_t)stream);
}

int gptrig_flce_fwd_noalloc(const void* hidden, const void* weight, const int32_t* targets, float* losses,
                            float* lse, int n, int d, int vocab, int semantic_vocab, void* stream) {
  if (!hidden || !weight || !targets || !losses || !lse) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (gptrig_flce_fwd_workspace_bytes(n, d, vocab) > (size_t)GPTRIG_FLCE_FWD_NOALLOC_SCRATCH_BYTES)
    return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight) & 15) return GPTRIG_E_SHAPE;
  void* ws = scratch_ptr();
  if (!ws) return GPTRIG_E_LAUNCH;
  return flce_fwd_launch(hidden, weight, targets, losses, lse, ws, n, d, vocab, semantic_vocab, (hipStream_t)stream);
}

size_t gptrig_flce_keep_bytes(int n, int vocab) {
  if (n <= 0 || vocab <= 0) return 0;
  return keep_gt_bytes(n, vocab) + align256((size_t)2 * ceil_div(vocab, BM) * n * sizeof(float));
}

int gptrig_flce_fwd_keep(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                         void* keep, size_t keep_bytes, void* workspace, size_t workspace_bytes, int n, int d,
                         int vocab, int semantic_vocab, void* stream) {
  if (!hidden || !weight || !targets || !losses || !lse || !keep || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (d % (4 * gemm::BK)) return GPTRIG_E_UNSUPPORTED;  // the persistent forward only
  if (n % 8) return GPTRIG_E_UNSUPPORTED;                // 16-byte token groups of the backward
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (workspace_bytes < gptrig_flce_fwd_workspace_bytes(n, d, vocab)) return GPTRIG_E_WORKSPACE;
  if (keep_bytes < gptrig_flce_keep_bytes(n, vocab)) return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)workspace | (uintptr_t)keep) & 15) return GPTRIG_E_SHAPE;
  return flce_fwd_launch(hidden, weight, targets, losses, lse, workspace, n, d, vocab, semantic_vocab,
                         (hipStream_t)stream, keep);
}

}  // extern "C"

namespace {

// Work split of flce_keep_gemms_kernel, chosen by simulating the
// dispatcher: the items (dh tiles x dh_split, dW tiles x dw_split) are handed
// out in launch order to whichever CU frees up first, each costing its
// 32-deep stages (rounded up to the main loop's groups of four) plus its
// epilogue, in units of one stage: about 60 for an fp32 atomic add of a 256 KB
// tile into a large array, 20 for a read-modify-write and 10 for a plain store
// (measured at 5120 and 65536 tokens per call).  The plan with the shortest
// estimated makespan wins; plans are cached per shape.
struct KeepPlan {
  int dh_split, dw_split, dh_mode, dw_mode;
  bool dh_first;
};

double keep_makespan(int cus, unsigned dh_tiles, int dh_k, int dh_split, double dh_epi, unsigned dw_tiles, int dw_k,
                     int dw_split, double dw_epi, bool& dh_first) {
  auto len = [](int k_iters, int split) {
    const int per = ceil_div(k_iters, split);
    return (double)((per + 3) & ~3);
  };
  const double l_dh = len(dh_k, dh_split) + dh_epi, l_dw = len(dw_k, dw_split) + dw_epi;
  dh_first = l_dh >= l_dw;
  const double l1 = dh_first ? l_dh : l_dw, l2 = dh_first ? l_dw : l_dh;
  const int64_t k1 = (int64_t)(dh_first ? dh_tiles * dh_split : dw_tiles * dw_split);
  const int64_t k2 = (int64_t)(dh_first ? dw_tiles * dw_split : dh_tiles * dh_split);
  // Min-heap of CU free times (all items of a group have one length).
  std::vector<double> heap((size_t)cus, 0.0);
  auto take = [&](double l) {
    std::pop_heap(heap.begin(), heap.end(), std::greater<double>());
    heap.back() += l;
    std::push_heap(heap.begin(), heap.end(), std::greater<double>());
  };
  for (int64_t i = 0; i < k1; ++i) take(l1);
  for (int64_t i = 0; i < k2; ++i) take(l2);
  return *std::max_element(heap.begin(), heap.end());
}

KeepPlan keep_plan(int n, int d, int vocab, bool accumulate) {
  struct Entry {
    int dev, n, d, vocab;
    bool acc;
    KeepPlan plan;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
      if (e.dev == dev && e.n == n && e.d == d && e.vocab == vocab && e.acc == accumulate) return e.plan;
  }
  const int cus = gemm::device_cus();
  const unsigned dh_tiles = tiles_of(n, d), dw_tiles = tiles_of(vocab, d);
  const int dh_k = ceil_div(vocab, gemm::BK), dw_k = ceil_div(n, gemm::BK);
  KeepPlan best{1, 1, 0, accumulate ? 1 : 0, true};
  double best_cost = 1e300;
  static const int kSplits[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int sh : kSplits) {
    if (sh > 1 && dh_k / sh < 8) break;
    for (int sw : kSplits) {
      if (sw > 1 && dw_k / sw < 8) break;
      bool dh_first;
      const double cost = keep_makespan(cus, dh_tiles, dh_k, sh, sh > 1 ? 60.0 : 10.0, dw_tiles, dw_k, sw,
                                        sw > 1 ? 60.0 : (accumulate ? 20.0 : 10.0), dh_first);
      if (cost < best_cost * 0.999) {
        best_cost = cost;
        best = KeepPlan{sh, sw, sh > 1 ? 2 : 0, sw > 1 ? 2 : (accumulate ? 1 : 0), dh_first};
      }
    }
  }
  std::lock_guard<std::mutex> lock(mu);
  cache.push_back(Entry{dev, n, d, vocab, accumulate, best});
  return best;
}

int flce_fwd_launch(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                    void* workspace, int n, int d, int vocab, int semantic_vocab, hipStream_t s, void* keep) {
  const int ntiles = ceil_div(vocab, BM);
  float2* partial = (float2*)workspace;
  float* tlogit = (float*)((char*)workspace + align256((size_t)ntiles * n * sizeof(float2)));
  Operand W{(const bf16*)weight, d}, Hd{(const bf16*)hidden, d};
  if (keep) {
    const unsigned tiles = tiles_of(vocab, n), cus = (unsigned)gemm::device_cus();
    float* mh = (float*)((char*)keep + keep_gt_bytes(n, vocab));
    flce_fwd_persistent_kernel<true><<<tiles < cus ? tiles : cus, gemm::THREADS, 0, s>>>(
        W, Hd, vocab, n, d, semantic_vocab, partial, (f16*)keep, mh);
  } else if (d % (4 * gemm::BK) == 0) {
    const unsigned tiles = tiles_of(vocab, n), cus = (unsigned)gemm::device_cus();
    flce_fwd_persistent_kernel<false><<<tiles < cus ? tiles : cus, gemm::THREADS, 0, s>>>(
        W, Hd, vocab, n, d, semantic_vocab, partial, nullptr, nullptr);
  } else {
    flce_fwd_kernel<<<tiles_of(vocab, n), gemm::THREADS, 0, s>>>(W, Hd, vocab, n, d, semantic_vocab, partial);
  }
  GPTRIG_CHECK_LAUNCH();
  flce_target_logit_kernel<<<ceil_div(n, 4), 256, 0, s>>>((const bf16*)hidden, (const bf16*)weight, targets, n, d,
                                                           semantic_vocab, tlogit);
  GPTRIG_CHECK_LAUNCH();
  // 4 waves per 64 tokens; 16 when that leaves the grid short of the CUs
  // (a token chunk of a bounded run: each wave then folds a quarter as many
  // tiles, and the launch is latency-bound, not bandwidth-bound).
  if (ceil_div(n, 64) < gemm::device_cus())
    flce_combine_kernel<16><<<ceil_div(n, 64), 64 * 16, 0, s>>>(partial, ntiles, n, semantic_vocab, targets, tlogit,
                                                                lse, losses);
  else
    flce_combine_kernel<4><<<ceil_div(n, 64), 64 * 4, 0, s>>>(partial, ntiles, n, semantic_vocab, targets, tlogit,
                                                              lse, losses);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // namespace

extern "C" {

size_t gptrig_flce_bwd_workspace_bytes(int n, int d, int vocab, int vocab_chunk) {
  if (n <= 0 || d <= 0 || vocab <= 0) return 0;
  const int chunk = resolve_chunk(vocab, vocab_chunk);
  const size_t gt = align256((size_t)chunk * ceil_div(n, 32) * 32 * sizeof(bf16));
  const size_t acc = align256((size_t)n * d * sizeof(float));
  if (ceil_div(vocab, chunk) == 1) return gt + acc;
  // kBlocks work counters per launch: at most 2 ceil(vocab / 256) + 2 launches.
  return gt + acc + align256((size_t)(2 * ceil_div(vocab, BM) + 2) * kBlocks * sizeof(int));
}

int gptrig_flce_bwd(const void* hidden, const void* weight, const int32_t* targets, const float* lse,
                    const float* cotangent, float cotangent_scale, void* dhidden, float* dweight,
                    int accumulate_dweight, void* workspace, size_t workspace_bytes, int n, int d, int vocab,
                    int semantic_vocab, int vocab_chunk, void* stream) {
  if (!hidden || !weight || !targets || !lse || !dhidden || !dweight || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (vocab_chunk < 0 || vocab_chunk % 256) return GPTRIG_E_SHAPE;
  if (n % 8) return GPTRIG_E_UNSUPPORTED;  // 16-byte rows of the MN-major operands
  if (workspace_bytes < gptrig_flce_bwd_workspace_bytes(n, d, vocab, vocab_chunk)) return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)workspace | (uintptr_t)dweight) & 15)
    return GPTRIG_E_SHAPE;
  const int chunk = resolve_chunk(vocab, vocab_chunk);
  bf16* gt = (bf16*)workspace;
  const size_t gt_bytes = align256((size_t)chunk * ceil_div(n, 32) * 32 * sizeof(bf16));
  float* dh_acc = (float*)((char*)workspace + gt_bytes);
  hipStream_t s = (hipStream_t)stream;
  const bf16* Wp = (const bf16*)weight;
  const bf16* Hp = (const bf16*)hidden;
  if (!accumulate_dweight) {
    const int64_t total = (int64_t)vocab * d;
    zero_f32_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dweight, total);
    GPTRIG_CHECK_LAUNCH();
  }
  if (ceil_div(vocab, chunk) > 1) {
    // Several chunks: pipelined launches over two halves of the G^T buffer
    // (chunk >= 512), else alternating recompute / reduction launches over
    // the one buffer.
    const bool piped = chunk >= 2 * BM;
    const PipeShape ps = pipe_shape(n, vocab, piped ? chunk / 2 / BM * BM : chunk);
    const int nch = ps.nchunks;
    const int launches = piped ? nch + 1 : 2 * nch;
    int* counters = (int*)((char*)dh_acc + align256((size_t)n * d * sizeof(float)));
    zero_i32_kernel<<<ceil_div(launches * kBlocks, 256), 256, 0, s>>>(counters, launches * kBlocks);
    GPTRIG_CHECK_LAUNCH();
    const size_t half_elems = (size_t)ps.half * ceil_div(n, 32) * 32;
    PipeLaunch p;
    p.h = Hp;
    p.w = Wp;
    p.targets = targets;
    p.lse = lse;
    p.cot = cotangent;
    p.cot_scale = cotangent_scale;
    p.dh_acc = dh_acc;
    p.dw = dweight;
    p.N = n;
    p.D = d;
    p.V = vocab;
    p.sem_v = semantic_vocab;
    p.C = ps.half;
    p.nchunks = nch;
    p.ks = ps.ks;
    const int cus = gemm::device_cus();
    for (int l = 0; l < launches; ++l) {
      if (piped) {
        p.c1 = l < nch ? l : -1;
        p.c23 = l - 1;
        p.gt1 = gt + (size_t)(l & 1) * half_elems;
        p.gt23 = gt + (size_t)((l + 1) & 1) * half_elems;
      } else {
        p.c1 = (l & 1) ? -1 : l / 2;
        p.c23 = (l & 1) ? l / 2 : -1;
        p.gt1 = gt;
        p.gt23 = gt;
      }
      p.counter = counters + (size_t)l * kBlocks;
      int most = 0;
      for (int q = 0; q < kBlocks; ++q) most = pipe_items(p, q) > most ? pipe_items(p, q) : most;
      // kBlocks workgroups per XCD round at most as many as the busiest block has items.
      const int cap = cus / kBlocks > 0 ? cus / kBlocks : 1;
      const int per_block = most < 1 ? 1 : (most < cap ? most : cap);
      flce_bwd_pipe_kernel<<<per_block * kBlocks, gemm::THREADS, 0, s>>>(p);
      GPTRIG_CHECK_LAUNCH();
    }
    const int64_t total = (int64_t)n * d;
    f32_to_bf16_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, (bf16*)dhidden, total);
    GPTRIG_CHECK_LAUNCH();
    return GPTRIG_OK;
  }
  {
    const int64_t total = (int64_t)n * d;
    zero_f32_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, total);
    GPTRIG_CHECK_LAUNCH();
  }
  // One chunk (the whole vocabulary): K1, then the split-K dW and dh GEMMs.
  const int v0 = 0, vc = vocab;
  {
    Operand Wc{Wp + (size_t)v0 * d, d}, Hd{Hp, d};
    if (d % (4 * gemm::BK) == 0) {
      const unsigned tiles = tiles_of(vc, n), cus = (unsigned)gemm::device_cus();
      flce_grad_persistent_kernel<<<tiles < cus ? tiles : cus, gemm::THREADS, 0, s>>>(
          Wc, Hd, vc, n, d, v0, semantic_vocab, targets, lse, cotangent, cotangent_scale, gt);
    } else {
      flce_grad_kernel<<<tiles_of(vc, n), gemm::THREADS, 0, s>>>(Wc, Hd, vc, n, d, v0, semantic_vocab, targets, lse,
                                                                  cotangent, cotangent_scale, gt);
    }
    GPTRIG_CHECK_LAUNCH();
    // dW += G^T h : A = G^T [vc][n] (K-major), B = h [n][d] (MN-major); split over tokens.
    Operand Ag{gt, n, vc}, Bh{Hp, d};
    const int dw_split = gemm::choose_split(tiles_of(vc, d), ceil_div(n, gemm::BK));
    gemm_f32_kernel<true, false><<<tiles_of(vc, d) * dw_split, gemm::THREADS, 0, s>>>(
        Ag, Bh, vc, d, n, dw_split, dweight + (size_t)v0 * d, d, 2, nullptr);
    GPTRIG_CHECK_LAUNCH();
    // dh += G W : A(m=n, k=v) = G^T [vc][n] (MN-major), B(k=v, n=j) = W [vc][d] (MN-major).
    Operand Agt{gt, n, vc}, Bw{Wp + (size_t)v0 * d, d};
    const int dh_split = gemm::choose_split(tiles_of(n, d), ceil_div(vc, gemm::BK));
    gemm_f32_kernel<false, false><<<tiles_of(n, d) * dh_split, gemm::THREADS, 0, s>>>(Agt, Bw, n, d, vc, dh_split,
                                                                                        dh_acc, d, 2, nullptr);
    GPTRIG_CHECK_LAUNCH();
  }
  const int64_t total = (int64_t)n * d;
  f32_to_bf16_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, (bf16*)dhidden, total);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

size_t gptrig_flce_bwd_keep_workspace_bytes(int n, int d) {
  if (n <= 0 || d <= 0) return 0;
  return align256((size_t)n * d * sizeof(float));
}

// The one-chunk backward from gptrig_flce_fwd_keep's kept softmax: the G^T
// values come from rescaling the kept probabilities (two bandwidth passes)
// instead of recomputing the logits GEMM; then the same dW and dh GEMMs.
int gptrig_flce_bwd_keep(const void* hidden, const void* weight, const int32_t* targets, const float* lse,
                         const float* cotangent, float cotangent_scale, void* dhidden, float* dweight,
                         int accumulate_dweight, void* keep, size_t keep_bytes, void* workspace,
                         size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab, void* stream) {
  if (!hidden || !weight || !targets || !lse || !dhidden || !dweight || !keep || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (n % 8) return GPTRIG_E_UNSUPPORTED;
  if (keep_bytes < gptrig_flce_keep_bytes(n, vocab)) return GPTRIG_E_WORKSPACE;
  if (workspace_bytes < gptrig_flce_bwd_keep_workspace_bytes(n, d)) return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)workspace | (uintptr_t)dweight | (uintptr_t)keep |
       (uintptr_t)targets) & 15)
    return GPTRIG_E_SHAPE;  // (the rescale reads targets 16 bytes at a time)
  if (ceil_div(n, 32) > 65535) return GPTRIG_E_UNSUPPORTED;  // grid.y of the rescale
  hipStream_t s = (hipStream_t)stream;
  bf16* gt = (bf16*)keep;
  float* alpha = (float*)((char*)keep + keep_gt_bytes(n, vocab));
  float* dh_acc = (float*)workspace;
  const bf16* Wp = (const bf16*)weight;
  const bf16* Hp = (const bf16*)hidden;
  // dW (+)= G^T h and dh = G W over this call's n tokens in one launch
  // (flce_keep_gemms_kernel), split as keep_plan estimates fastest.  With few
  // tokens per call (a token chunk of a bounded run) the dW tiles are short and
  // the dh tiles long; with many, both are long enough to need no split.
  const int vc = vocab;
  const KeepPlan plan = keep_plan(n, d, vocab, accumulate_dweight != 0);
  if (!accumulate_dweight && plan.dw_mode == 2) {
    const int64_t total = (int64_t)vocab * d;
    zero_f32_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dweight, total);
    GPTRIG_CHECK_LAUNCH();
  }
  if (plan.dh_mode == 2) {
    const int64_t total = (int64_t)n * d;
    zero_f32_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, total);
    GPTRIG_CHECK_LAUNCH();
  }
  const int halves = 2 * ceil_div(vocab, BM);
  flce_keep_alpha_kernel<<<dim3((unsigned)ceil_div(n / 4, 256), (unsigned)halves), 256, 0, s>>>(
      alpha, halves, n, semantic_vocab, targets, lse, cotangent, cotangent_scale);
  GPTRIG_CHECK_LAUNCH();
  const dim3 rgrid((unsigned)ceil_div(keep_rows(vocab) / 4, 16), (unsigned)ceil_div(n, 32));
  flce_keep_rescale_kernel<<<rgrid, 256, 0, s>>>(gt, alpha, n, vocab, semantic_vocab, targets, cotangent,
                                                  cotangent_scale);
  GPTRIG_CHECK_LAUNCH();
  const unsigned n_dh = tiles_of(n, d) * (unsigned)plan.dh_split;
  const unsigned n_dw = tiles_of(vc, d) * (unsigned)plan.dw_split;
  flce_keep_gemms_kernel<<<n_dh + n_dw, gemm::THREADS, 0, s>>>(
      Operand{gt, n, keep_rows(vocab)}, Operand{Wp, d}, Operand{Hp, d}, n, d, vc, plan.dh_split, plan.dw_split, dh_acc,
      plan.dh_mode, dweight, plan.dw_mode, (int)n_dh, (int)n_dw, plan.dh_first);
  GPTRIG_CHECK_LAUNCH();
  const int64_t total = (int64_t)n * d;
  f32_to_bf16_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, (bf16*)dhidden, total);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

// dW (f32 [rows_in, cols_out], += ) = X^T dY for X bf16 [n, rows_in], dY bf16 [n, cols_out],
// and (db nullable) db (f32 [cols_out], += ) = column sums of dY: the weight and
// bias gradients of rig/nn.py:55-56 (linear).  Split over the n tokens with
// fp32 atomics so the skinny [d_in, d_out] output still fills the GPU; the
// bias sums come from the dY slabs the GEMM already stages in LDS.
int gptrig_weight_grad(const void* x, const void* dy, float* dw, float* db, int n, int rows_in, int cols_out,
                       void* stream) {
  if (!x || !dy || !dw) return GPTRIG_E_NULL;
  if (n <= 0 || rows_in <= 0 || cols_out <= 0 || rows_in % 8 || cols_out % 8) return GPTRIG_E_SHAPE;
  if (((uintptr_t)x | (uintptr_t)dy) & 15) return GPTRIG_E_SHAPE;
  const unsigned tiles = tiles_of(rows_in, cols_out);
  const int split = gemm::choose_split(tiles, ceil_div(n, gemm::BK));
  // A(m = i, k = t) = X[t][i] (MN-major), B(k = t, n = j) = dY[t][j] (MN-major).
  Operand A{(const bf16*)x, rows_in}, B{(const bf16*)dy, cols_out};
  gemm_f32_kernel<false, false><<<tiles * split, gemm::THREADS, 0, (hipStream_t)stream>>>(A, B, rows_in, cols_out, n,
                                                                                         split, dw, cols_out, 2, db);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // extern "C"
