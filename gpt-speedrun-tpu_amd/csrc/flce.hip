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
//                zero for rows >= semantic vocab (persistent when d % 128 == 0);
//            K2  dW[chunk] += G^T h     (split over tokens, fp32 atomics);
//            K3  dh_acc    += G W[chunk] (fp32 atomics, split over the chunk),
//                rounded to bf16 at the end.
#include "gemm_core.h"

#include <math.h>

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
__global__ void __launch_bounds__(gemm::THREADS)
    flce_fwd_persistent_kernel(Operand W, Operand Hd, int V, int N, int D, int sem_v, float2* __restrict__ partial) {
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
      const float2 st = full ? column_stats<false>(acc, nb, lim) : column_stats<true>(acc, nb, lim);
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
__global__ void flce_combine_kernel(const float2* __restrict__ partial, int ntiles, int N, int sem_v,
                                    const int32_t* __restrict__ targets, const float* __restrict__ tlogit,
                                    float* __restrict__ lse, float* __restrict__ losses) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float m = -INFINITY, s = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    const float2 p = partial[(size_t)t * N + n];
    if (p.x == -INFINITY) continue;
    const float m2 = fmaxf(m, p.x);
    s = s * fast_exp2(m - m2) + p.y * fast_exp2(p.x - m2);
    m = m2;
  }
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
// walked one vocabulary tile per token sweep (measured 0.7% faster for the
// FLCE backward than two per sweep, 0.8% faster than four or eight).
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
    gemm::tile_coords(t, Vc, N, tv, tt, 1);
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
template <bool AK, bool BKM>
__global__ void __launch_bounds__(gemm::THREADS)
    gemm_f32_kernel(Operand A, Operand B, int M, int N, int K, int ksplit, float* __restrict__ C, int64_t ldc,
                    int mode, float* __restrict__ colsum) {
  int tm, tn, split;
  gemm::split_tile_coords(blockIdx.x, gridDim.x, M, N, tm, tn, split);
  const int kslice = ((K + ksplit - 1) / ksplit + gemm::BK - 1) / gemm::BK * gemm::BK;
  const int k_begin = split * kslice;
  const int k_end = min(K, k_begin + kslice);
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
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = tm * BM + 128 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (m >= M) continue;
        float* dst = C + (int64_t)m * ldc + n;
        if (mode == 2)
          atomicAdd(dst, acc[mb][nb][i]);
        else
          *dst = mode ? *dst + acc[mb][nb][i] : acc[mb][nb][i];
      }
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

// Default vocabulary chunk of the backward: the whole vocabulary while the
// bf16 G^T workspace (n x chunk) fits kGradChunkBudget, else the fewest equal
// chunks (whole 256-row tiles) that fit.  One chunk measured fastest.
constexpr size_t kGradChunkBudget = size_t(8) << 30;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int resolve_chunk(int n, int vocab, int vocab_chunk) {
  int chunk = vocab_chunk;
  if (chunk <= 0) {
    const size_t bytes = size_t(2) * (size_t)n * (size_t)vocab;
    const int parts = (int)((bytes + kGradChunkBudget - 1) / kGradChunkBudget);
    chunk = ceil_div(ceil_div(vocab, parts < 1 ? 1 : parts), BM) * BM;
  }
  const int full = ceil_div(vocab, BM) * BM;
  return chunk > full ? full : chunk;
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
  const int ntiles = ceil_div(vocab, BM);
  float2* partial = (float2*)workspace;
  float* tlogit = (float*)((char*)workspace + align256((size_t)ntiles * n * sizeof(float2)));
  hipStream_t s = (hipStream_t)stream;
  Operand W{(const bf16*)weight, d}, Hd{(const bf16*)hidden, d};
  if (d % (4 * gemm::BK) == 0) {
    const unsigned tiles = tiles_of(vocab, n), cus = (unsigned)gemm::device_cus();
    flce_fwd_persistent_kernel<<<tiles < cus ? tiles : cus, gemm::THREADS, 0, s>>>(W, Hd, vocab, n, d, semantic_vocab,
                                                                                   partial);
  } else {
    flce_fwd_kernel<<<tiles_of(vocab, n), gemm::THREADS, 0, s>>>(W, Hd, vocab, n, d, semantic_vocab, partial);
  }
  GPTRIG_CHECK_LAUNCH();
  flce_target_logit_kernel<<<ceil_div(n, 4), 256, 0, s>>>((const bf16*)hidden, (const bf16*)weight, targets, n, d,
                                                           semantic_vocab, tlogit);
  GPTRIG_CHECK_LAUNCH();
  flce_combine_kernel<<<ceil_div(n, 256), 256, 0, s>>>(partial, ntiles, n, semantic_vocab, targets, tlogit, lse,
                                                        losses);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

size_t gptrig_flce_bwd_workspace_bytes(int n, int d, int vocab, int vocab_chunk) {
  const int chunk = resolve_chunk(n, vocab, vocab_chunk);
  return align256((size_t)chunk * ceil_div(n, 32) * 32 * sizeof(bf16)) + align256((size_t)n * d * sizeof(float));
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
  const int chunk = resolve_chunk(n, vocab, vocab_chunk);
  bf16* gt = (bf16*)workspace;
  float* dh_acc = (float*)((char*)workspace + align256((size_t)chunk * ceil_div(n, 32) * 32 * sizeof(bf16)));
  hipStream_t s = (hipStream_t)stream;
  const bf16* Wp = (const bf16*)weight;
  const bf16* Hp = (const bf16*)hidden;
  if (!accumulate_dweight) {
    const int64_t total = (int64_t)vocab * d;
    zero_f32_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dweight, total);
    GPTRIG_CHECK_LAUNCH();
  }
  {
    const int64_t total = (int64_t)n * d;
    zero_f32_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, total);
    GPTRIG_CHECK_LAUNCH();
  }
  for (int v0 = 0; v0 < vocab; v0 += chunk) {
    const int vc = vocab - v0 < chunk ? vocab - v0 : chunk;
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
    // dW[v0:v0+vc] += G^T h : A = G^T [vc][n] (K-major), B = h [n][d] (MN-major); split over tokens.
    Operand Ag{gt, n, vc}, Bh{Hp, d};
    const int dw_split = gemm::choose_split(tiles_of(vc, d), ceil_div(n, gemm::BK));
    gemm_f32_kernel<true, false><<<tiles_of(vc, d) * dw_split, gemm::THREADS, 0, s>>>(
        Ag, Bh, vc, d, n, dw_split, dweight + (size_t)v0 * d, d, 2, nullptr);
    GPTRIG_CHECK_LAUNCH();
    // dh += G W[v0:v0+vc] : A(m=n, k=v) = G^T [vc][n] (MN-major), B(k=v, n=j) = W [vc][d] (MN-major).
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
