// Top-k expert routing (recipes/reference_moe/train.py:1259-1273).
//
// route_topk: one thread per token.  softmax over the fp32 router logits,
//   jax.lax.top_k selection (largest value first; on equal values the lower
//   expert index first), softmax over the chosen logits.
// route_hist / route_place build the dropless bucket layout over blocks of
//   1024 slots: counts[e], and order = stable argsort(chosen.reshape(-1)) by
//   counting sort (per-block counts in the workspace, per-expert bases from
//   the totals and the blocks before, stable ranks within a block from wave
//   ballots in slot order), rows = order / top_k, position = order^-1.
//
// The routed MLP around it (:1275-1293):
//   router_logits   fp32 x @ router_w (one wave per token, weights in LDS);
//   moe_gather_rows grouped = flat[rows] (token rows in bucket order);
//   moe_gmm         grouped GEMM over the expert buckets on the MFMA GEMM core,
//                   epilogue bias (+ GELU, or x GELU' for the backward);
//   moe_combine     combined[t] = sum over the token's slots, in bucket order,
//                   of bf16(out * bf16(gate)) -- the .at[rows].add rounding;
//   moe_stats       mean probability, load, (entropy, top-1 gate, logit RMS);
// and their backward: combine_bwd, moe_gmm_dw (per-expert weight + bias
// gradients, split-K fp32 atomics), gather_bwd (the VJP of flat[rows]) and
// router_bwd (gate/probability softmax VJPs, dx and d router_w).
#include "common.h"
#include "epilogue.h"

#include <math.h>

namespace {

constexpr int kMaxExperts = 64;

__global__ void route_topk_kernel(const float* __restrict__ logits, float* __restrict__ probs,
                                  int32_t* __restrict__ chosen, float* __restrict__ gate, int T, int E, int k) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float* row = logits + (size_t)t * E;
  float mx = -INFINITY;
  for (int e = 0; e < E; ++e) mx = fmaxf(mx, row[e]);
  if (probs) {
    float s = 0.f;
    for (int e = 0; e < E; ++e) s += expf(row[e] - mx);
    for (int e = 0; e < E; ++e) probs[(size_t)t * E + e] = expf(row[e] - mx) / s;
  }
  uint64_t taken = 0;
  float vals[kMaxExperts];
  int idx[kMaxExperts];
  for (int j = 0; j < k; ++j) {
    int best = -1;
    float bv = 0.f;
    for (int e = 0; e < E; ++e) {
      if (taken >> e & 1) continue;
      const float x = row[e];
      // Strictly greater keeps the lower index on ties; NaN never wins.
      if (best < 0 || x > bv) {
        best = e;
        bv = x;
      }
    }
    taken |= 1ull << best;
    vals[j] = bv;
    idx[j] = best;
  }
  float gm = vals[0];
  for (int j = 1; j < k; ++j) gm = fmaxf(gm, vals[j]);
  float gs = 0.f;
  for (int j = 0; j < k; ++j) gs += expf(vals[j] - gm);
  for (int j = 0; j < k; ++j) {
    chosen[(size_t)t * k + j] = idx[j];
    gate[(size_t)t * k + j] = expf(vals[j] - gm) / gs;
  }
}

// Stable bucket order over blocks of kSortBlock slots, in two launches.
// route_hist: each block's per-expert counts into hist[block][e].  route_place:
// each block finds its experts' bases (all experts' totals before e, plus
// the counts of e in the blocks before it) and places its slots at base +
// rank, the rank within the block from wave ballots in slot order; block 0
// also writes counts.
constexpr int kSortBlock = 1024;

__global__ void __launch_bounds__(kSortBlock) route_hist_kernel(const int32_t* __restrict__ chosen, int n_slots,
                                                                int E, int32_t* __restrict__ hist) {
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x;
  if (tid < E) cnt[tid] = 0;
  __syncthreads();
  const int s = blockIdx.x * kSortBlock + tid;
  if (s < n_slots) atomicAdd(&cnt[chosen[s]], 1);
  __syncthreads();
  if (tid < E) hist[(size_t)blockIdx.x * E + tid] = cnt[tid];
}

__global__ void __launch_bounds__(kSortBlock) route_place_kernel(const int32_t* __restrict__ chosen, int n_slots,
                                                                 int E, int k, const int32_t* __restrict__ hist,
                                                                 int nblocks, int32_t* __restrict__ counts,
                                                                 int32_t* __restrict__ order, int32_t* __restrict__ rows,
                                                                 int32_t* __restrict__ position) {
  __shared__ int total[kMaxExperts], before[kMaxExperts], base[kMaxExperts];
  __shared__ int wave_cnt[kSortBlock / 64][kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int blk = blockIdx.x;
  if (tid < E) {
    int tot = 0, bef = 0;
    for (int b = 0; b < nblocks; ++b) {
      const int h = hist[(size_t)b * E + tid];
      tot += h;
      bef += b < blk ? h : 0;
    }
    total[tid] = tot;
    before[tid] = bef;
    if (blk == 0) counts[tid] = tot;
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      base[e] = acc + before[e];
      acc += total[e];
    }
  }
  const int s = blk * kSortBlock + tid;
  const int my_e = s < n_slots ? chosen[s] : -1;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int rank = 0;
  for (int e = 0; e < E; ++e) {
    const uint64_t m = __ballot(my_e == e);
    if (my_e == e) rank = __popcll(m & lt_mask);
    if (lane == 0) wave_cnt[wave][e] = __popcll(m);
  }
  __syncthreads();
  if (my_e >= 0) {
    int bw = 0;
    for (int w = 0; w < wave; ++w) bw += wave_cnt[w][my_e];
    const int pos = base[my_e] + bw + rank;
    order[pos] = s;
    rows[pos] = s / k;
    if (position) position[s] = pos;
  }
}

// ---------------------------------------------------------------------------
// Router logits (:1259-1264): logits[t][e] = sum_d f32(x[t][d]) * w[d][e].
// A wave takes 8 tokens at a time: lane = 8 token + g reads the token's
// 16-byte chunks g, g + 8, ... (each 8-lane group reads 128 contiguous
// bytes of one row), multiplies them by w rows from LDS, and the 8 lanes of
// a token add their partial logits with three xor exchanges.
// ---------------------------------------------------------------------------
constexpr int kMaxRouterExperts = 16;
constexpr int kRouterTokens = 16;  // tokens per wave (two passes of 8)
constexpr int kMaxRouterWidth = 4096;

// 8 bf16 of row x[t] from column d (d < D), zeros past D.
__device__ __forceinline__ void load_x8(const bf16* __restrict__ row, int d, int D, float (&xv)[8]) {
  if (d + 8 <= D && ((D & 7) == 0)) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + d);
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = (float)v[j];
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) xv[j] = d + j < D ? (float)row[d + j] : 0.f;
  }
}

template <int EP>
__global__ void __launch_bounds__(256) router_logits_kernel(const bf16* __restrict__ x, const float* __restrict__ w,
                                                            float* __restrict__ logits, int T, int D, int E) {
  extern __shared__ float wsh[];  // [D][EP], zero past E
  for (int i = threadIdx.x; i < D * EP; i += blockDim.x) {
    const int d = i / EP, e = i % EP;
    wsh[i] = e < E ? w[(size_t)d * E + e] : 0.f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tok = lane >> 3, g = lane & 7;
  const int wt0 = (blockIdx.x * 4 + wave) * kRouterTokens;
#pragma unroll 1
  for (int pass = 0; pass < kRouterTokens / 8; ++pass) {
    const int t = wt0 + 8 * pass + tok;
    float acc[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) acc[e] = 0.f;
    if (t < T) {
      const bf16* row = x + (size_t)t * D;
      for (int d = 8 * g; d < D; d += 64) {
        float xv[8];
        load_x8(row, d, D, xv);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (d + j >= D) break;
          const float* wr = wsh + (d + j) * EP;
#pragma unroll
          for (int e4 = 0; e4 < EP; e4 += 4) {
            const f32x4 w4 = *reinterpret_cast<const f32x4*>(wr + e4);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[e4 + u] = fmaf(xv[j], w4[u], acc[e4 + u]);
          }
        }
      }
    }
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      acc[e] += __shfl_xor(acc[e], 1);
      acc[e] += __shfl_xor(acc[e], 2);
      acc[e] += __shfl_xor(acc[e], 4);
    }
    if (t < T) {
#pragma unroll
      for (int e = 0; e < EP; ++e)
        if (e % 8 == g && e < E) logits[(size_t)t * E + e] = acc[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped GEMM over the expert buckets (megablox.gmm contract):
//   out[off_e + r][n] = sum_k A[off_e + r][k] * B_e(k, n),  r < counts[e],
// A K-major [R][K] (rows in bucket order), B_e either [K][N]
// (kBT = false: rhs + e*K*N) or [N][K] (kBT = true: the transpose, for dX).
// Grid: (ceil(R/256) + E) M-tile slots x ceil(N/256); surplus slots exit.
// Each 256 x 256 tile is computed transposed (features x bucket rows) and
// written through LDS in whole rows by the shared epilogue (epilogue.h),
// which also reads pre in whole rows for kMode 2.
// kMode 0: out = bf16(acc) (+ bias)
//       1: pre = bf16(bf16(acc) + bias), out = bf16(gelu(pre))
//       2: out = bf16(bf16(acc) * gelu'(pre))   (pre read, same layout as out)
// ---------------------------------------------------------------------------
template <bool kBT, int kMode>
__global__ void __launch_bounds__(gemm::THREADS)
    moe_gmm_kernel(const bf16* __restrict__ lhs, int64_t lda,
                   const bf16* __restrict__ rhs, const int32_t* __restrict__ counts, int E, int K, int N,
                   const bf16* __restrict__ bias, bf16* __restrict__ out, bf16* __restrict__ pre, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) float bias_s[gemm::BM];
  const int ntn = (N + gemm::BN - 1) / gemm::BN;
  const int tn = blockIdx.x % ntn;  // feature tile
  int tm = blockIdx.x / ntn;        // bucket-row tile of expert e
  int e = 0, off = 0;
  for (; e < E; ++e) {
    const int c = counts[e];
    const int nt = (c + gemm::BM - 1) / gemm::BM;
    if (tm < nt) break;
    tm -= nt;
    off += c;
  }
  if (e >= E) return;  // uniform: surplus slot
  const int cnt = counts[e];
  // The tile is computed transposed (rows = output features, columns =
  // bucket rows), so it leaves through the shared token-row epilogue:
  // A = the expert's weight (K-major [N][K] when transposed, else MN-major
  // [K][N]), B = the bucket's rows (K-major).
  const gemm::Operand Wop = kBT ? gemm::Operand{rhs + (int64_t)e * N * K, K} : gemm::Operand{rhs + (int64_t)e * K * N, N};
  const gemm::Operand Xop{lhs + (int64_t)off * lda, lda};
  constexpr int kEpi = kMode == 0 ? gemm_epi::kBias : kMode == 1 ? gemm_epi::kGelu : gemm_epi::kDGelu;
  if constexpr (gemm_epi::has_bias(kEpi)) gemm_epi::stage_bias(bias_s, bias ? bias + (int64_t)e * N : nullptr, tn * gemm::BM, N);
  f32x16 acc[4][2];
  gemm::mainloop_pp<kBT, true>(acc, Wop, Xop, N, cnt, 0, K, tn * gemm::BM, tm * gemm::BN);
  gemm_epi::EpiArgs ea{};
  const int64_t base = (int64_t)off * ldo;
  if (kMode == 1) {
    ea.y = pre + base;  // h = bf16(bf16(acc) + b)
    ea.act = out + base;  // gelu(h)
  } else {
    ea.y = out + base;
  }
  ea.ldy = ldo;
  ea.aux = kMode == 2 ? pre + base : nullptr;
  ea.ldaux = ldo;
  gemm_epi::linear_epilogue<kEpi>(acc, tn, tm, N, cnt, ea, bias_s);
}

// Per-expert weight (+ bias) gradients:
//   dw[e] (f32 [K][N]) += sum_{r in bucket e} A[r][k] * dy[r][n],
//   db[e] (f32 [N])    += sum_{r in bucket e} dy[r][n]          (nullable),
// A [R][K] and dy [R][N] in bucket order.  Grid:
// E x tiles(K, N) x split; bucket e's rows are split into `split` slices,
// whose partial tiles are added with fp32 atomics (measured no slower than a
// read-modify-write when a tile has one writer).
__global__ void __launch_bounds__(gemm::THREADS)
    moe_gmm_dw_kernel(const bf16* __restrict__ lhs, int64_t lda,
                      const bf16* __restrict__ dy, int64_t ldy, const int32_t* __restrict__ counts, int E, int K,
                      int N, int split, float* __restrict__ dw, float* __restrict__ db) {
  const int tiles = ((K + gemm::BM - 1) / gemm::BM) * ((N + gemm::BN - 1) / gemm::BN);
  const int e = blockIdx.x / (tiles * split);
  const int rem = blockIdx.x % (tiles * split);
  const int sp = rem / tiles;
  int tm, tn;
  gemm::tile_coords(rem % tiles, K, N, tm, tn);
  int off = 0;
  for (int i = 0; i < e; ++i) off += counts[i];
  const int cnt = counts[e];
  const int kslice = ((cnt + split - 1) / split + gemm::BK - 1) / gemm::BK * gemm::BK;
  const int k_begin = sp * kslice;
  const int k_end = min(cnt, k_begin + kslice);
  if (k_begin >= k_end) return;  // uniform
  // A(m = k-index, k = bucket row) MN-major; B(k = bucket row, n) MN-major.
  gemm::Operand A{lhs + (int64_t)off * lda, lda};
  gemm::Operand B{dy + (int64_t)off * ldy, ldy};
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  f32x16 acc[4][2];
  float csum[2] = {0.f, 0.f};
  const bool do_colsum = db != nullptr;  // shared out over the M tiles
  gemm::mainloop_pp<false, false, true>(acc, A, B, K, N, k_begin, k_end, tm * gemm::BM, tn * gemm::BN, csum,
                                        do_colsum ? (K + gemm::BM - 1) / gemm::BM : 0, tm);
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  float* dwe = dw + (int64_t)e * K * N;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = tn * gemm::BN + 64 * wn + 32 * nb + l32;
    if (n >= N) continue;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = tm * gemm::BM + 128 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (m < K) atomicAdd(dwe + (int64_t)m * N + n, acc[mb][nb][i]);
      }
  }
  if (do_colsum && wm == 0) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float t = csum[nb] + __shfl_xor(csum[nb], 32);
      const int n = tn * gemm::BN + 64 * wn + 32 * nb + l32;
      if (hl == 0 && n < N) atomicAdd(db + (int64_t)e * N + n, t);
    }
  }
}

// grouped[p] = x[rows[p]] (flat[rows], :1278): one wave per bucket row.
__global__ void __launch_bounds__(256) moe_gather_rows_kernel(const bf16* __restrict__ x, const int32_t* __restrict__ rows,
                                                              bf16* __restrict__ grouped, int R, int D) {
  const int p = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (p >= R) return;
  const int lane = threadIdx.x & 63;
  const bf16* src = x + (size_t)rows[p] * D;
  bf16* dst = grouped + (size_t)p * D;
  for (int c = lane * 8; c < D; c += 512) *reinterpret_cast<bf16x8*>(dst + c) = *reinterpret_cast<const bf16x8*>(src + c);
}

// Sort the (at most kMaxTopK) bucket positions of one token ascending.
constexpr int kMaxTopK = 8;
__device__ __forceinline__ void token_slots(const int32_t* __restrict__ position, const float* __restrict__ gate,
                                            int t, int k, int (&p)[kMaxTopK], float (&g)[kMaxTopK]) {
  for (int j = 0; j < k; ++j) {
    p[j] = position[(size_t)t * k + j];
    g[j] = gate ? (float)(bf16)gate[(size_t)t * k + j] : 0.f;
  }
  for (int a = 1; a < k; ++a)
    for (int b = a; b > 0 && p[b - 1] > p[b]; --b) {
      const int tp = p[b];
      p[b] = p[b - 1];
      p[b - 1] = tp;
      const float tg = g[b];
      g[b] = g[b - 1];
      g[b - 1] = tg;
    }
}

// combined[t] = bf16 sum, in bucket order, of bf16(out[p] * bf16(gate)):
// weighted = out * gate[order].astype(bf16); zeros.at[rows].add(weighted).
__global__ void __launch_bounds__(256) moe_combine_kernel(const bf16* __restrict__ out, const int32_t* __restrict__ position,
                                                          const float* __restrict__ gate, bf16* __restrict__ combined,
                                                          int T, int D, int k) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  int p[kMaxTopK];
  float g[kMaxTopK];
  token_slots(position, gate, t, k, p, g);
  for (int c = lane * 4; c < D; c += 256) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < k; ++j) {
      const bf16x4 v = *reinterpret_cast<const bf16x4*>(out + (size_t)p[j] * D + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = (float)(bf16)(acc[q] + (float)(bf16)((float)v[q] * g[j]));
    }
    bf16x4 o = {(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
    *reinterpret_cast<bf16x4*>(combined + (size_t)t * D + c) = o;
  }
}

// Backward of the combine: dout[p] = bf16(dcombined[t] * bf16(gate[a])),
// dgate[a] = sum_n dcombined[t][n] * out[p][n] (fp32), a = t*k + j, p = position[a].
__global__ void __launch_bounds__(256) moe_combine_bwd_kernel(const bf16* __restrict__ dcombined,
                                                              const bf16* __restrict__ out,
                                                              const int32_t* __restrict__ position,
                                                              const float* __restrict__ gate, bf16* __restrict__ dout,
                                                              float* __restrict__ dgate, int T, int D, int k) {
  const int a = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (a >= T * k) return;
  const int lane = threadIdx.x & 63;
  const int t = a / k, p = position[a];
  const float g = (float)(bf16)gate[a];
  float dot = 0.f;
  for (int c = lane * 4; c < D; c += 256) {
    const bf16x4 dc = *reinterpret_cast<const bf16x4*>(dcombined + (size_t)t * D + c);
    const bf16x4 ov = *reinterpret_cast<const bf16x4*>(out + (size_t)p * D + c);
    bf16x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[q] = (bf16)((float)dc[q] * g);
      dot = fmaf((float)dc[q], (float)ov[q], dot);
    }
    *reinterpret_cast<bf16x4*>(dout + (size_t)p * D + c) = o;
  }
  dot = wave_sum(dot);
  if (lane == 0) dgate[a] = dot;
}

// VJP of grouped = flat[rows]: dx[t] = bf16 sum, in bucket order, of dgrouped[p].
__global__ void __launch_bounds__(256) moe_gather_bwd_kernel(const bf16* __restrict__ dgrouped,
                                                             const int32_t* __restrict__ position,
                                                             bf16* __restrict__ dx, int T, int D, int k) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  int p[kMaxTopK];
  float g[kMaxTopK];
  token_slots(position, nullptr, t, k, p, g);
  for (int c = lane * 4; c < D; c += 256) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < k; ++j) {
      const bf16x4 v = *reinterpret_cast<const bf16x4*>(dgrouped + (size_t)p[j] * D + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = (float)(bf16)(acc[q] + (float)v[q]);
    }
    bf16x4 o = {(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
    *reinterpret_cast<bf16x4*>(dx + (size_t)t * D + c) = o;
  }
}

// Router statistics (:1295-1306): the sums of probabilities, entropies,
// top-1 gates and squared logits over the tokens, in three launches:
// stats_zero clears the outputs, moe_stats_kernel (one thread per token)
// adds each workgroup's sums into them with atomics, stats_finalize divides
// (and takes the root of the mean square) and writes the load.
__global__ void stats_zero_kernel(float* __restrict__ mean_probability, float* __restrict__ summary, int E) {
  const int i = threadIdx.x;
  if (i < E) mean_probability[i] = 0.f;
  if (i < 3) summary[i] = 0.f;
}

template <int EP>
__global__ void __launch_bounds__(256) moe_stats_kernel(const float* __restrict__ logits, const float* __restrict__ probs,
                                                        const float* __restrict__ gate, int T, int E, int k,
                                                        float* __restrict__ mean_probability,
                                                        float* __restrict__ summary) {
  __shared__ float red[3 + EP][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = blockIdx.x * blockDim.x + tid;
  float pe[EP], ent = 0.f, top = 0.f, sq = 0.f;
#pragma unroll
  for (int e = 0; e < EP; ++e) pe[e] = 0.f;
  if (t < T) {
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      if (e < E) {
        const float pv = probs[(size_t)t * E + e];
        const float lv = logits[(size_t)t * E + e];
        pe[e] = pv;
        ent -= pv * logf(pv + 1.0e-9f);
        sq = fmaf(lv, lv, sq);
      }
    }
    float gm = gate[(size_t)t * k];
    for (int j = 1; j < k; ++j) gm = fmaxf(gm, gate[(size_t)t * k + j]);
    top = gm;
  }
  float vals[3] = {ent, top, sq};
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const float v = wave_sum(vals[q]);
    if (lane == 0) red[q][wave] = v;
  }
#pragma unroll
  for (int e = 0; e < EP; ++e) {
    if (e < E) {
      const float v = wave_sum(pe[e]);
      if (lane == 0) red[3 + e][wave] = v;
    }
  }
  __syncthreads();
  if (tid < 3 + E) {
    const float v = red[tid][0] + red[tid][1] + red[tid][2] + red[tid][3];
    atomicAdd(tid < 3 ? summary + tid : mean_probability + (tid - 3), v);
  }
}

__global__ void stats_finalize_kernel(const int32_t* __restrict__ counts, int T, int E, int k,
                                      float* __restrict__ mean_probability, float* __restrict__ load,
                                      float* __restrict__ summary) {
  const int i = threadIdx.x;
  if (i < E) {
    mean_probability[i] = mean_probability[i] / T;
    load[i] = (float)counts[i] / (float)((long long)T * k);
  }
  if (i == 0) {
    summary[0] = summary[0] / T;
    summary[1] = summary[1] / T;
    summary[2] = sqrtf(summary[2] / ((float)T * E));
  }
}

// Router backward, per token t:
//   dchosen[j] = gate[j] * (dgate[j] - sum_i gate[i] dgate[i])        (gate softmax)
//   dprobs[e]  = dmean_probability[e] / T                              (mean over tokens)
//   dlogits[e] = probs[e] * (dprobs[e] - sum_i probs[i] dprobs[i]) + sum_{j: chosen[j]=e} dchosen[j]
//   dx[t][d]   = bf16(dx[t][d] + bf16(sum_e dlogits[e] w[d][e]))       (in place)
//   dw[d][e]  += sum_t f32(x[t][d]) dlogits[e]
// A workgroup takes a tile of kRouterBwdCols width columns x
// kRouterBwdTokens tokens.  Its threads first turn each token's gate and
// probability cotangents into dlogits (LDS); then thread (token lane tl,
// chunk c) walks tokens tl, tl + 32, ... for the 8 columns 8 c .. 8 c + 7 of
// the tile: dx[t][chunk] += bf16(dlogits[t] @ w[chunk]^T) (a 16-byte
// read-modify-write; the 8 chunk threads of a token cover 128 contiguous
// bytes) and the chunk's dw partial f32 [8][EP] in registers.  The 32 token
// lanes' partials are summed with xor exchanges and through LDS, and each
// workgroup adds one value per (column, expert) to dw with an atomic.
constexpr int kRouterBwdTokens = 1024;
constexpr int kRouterBwdCols = 64;

template <int EP>
__global__ void __launch_bounds__(256) router_bwd_kernel(const bf16* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ probs, const int32_t* __restrict__ chosen,
                                                         const float* __restrict__ gate, const float* __restrict__ dgate,
                                                         const float* __restrict__ dmean_probability,
                                                         bf16* __restrict__ dx, float* __restrict__ dw, int T, int D,
                                                         int E, int k) {
  __shared__ __attribute__((aligned(16))) float dl_s[kRouterBwdTokens][EP];
  __shared__ float red[4][kRouterBwdCols][EP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tb = blockIdx.y * kRouterBwdTokens;
  const int col0 = blockIdx.x * kRouterBwdCols;
  for (int i = tid; i < kRouterBwdTokens; i += blockDim.x) {
    const int t = tb + i;
    float dl[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) dl[e] = 0.f;
    if (t < T) {
      if (dmean_probability) {
        float pd = 0.f;
#pragma unroll
        for (int e = 0; e < EP; ++e)
          if (e < E) pd += probs[(size_t)t * E + e] * (dmean_probability[e] / T);
#pragma unroll
        for (int e = 0; e < EP; ++e)
          if (e < E) dl[e] = probs[(size_t)t * E + e] * (dmean_probability[e] / T - pd);
      }
      float gd = 0.f;
      for (int j = 0; j < k; ++j) gd += gate[(size_t)t * k + j] * dgate[(size_t)t * k + j];
      for (int j = 0; j < k; ++j) {
        const float dc = gate[(size_t)t * k + j] * (dgate[(size_t)t * k + j] - gd);
        const int ce = chosen[(size_t)t * k + j];
#pragma unroll
        for (int e = 0; e < EP; ++e)
          if (e == ce) dl[e] += dc;
      }
    }
#pragma unroll
    for (int e = 0; e < EP; ++e) dl_s[i][e] = dl[e];
  }
  __syncthreads();
  const int c = tid & 7, tl = tid >> 3;  // chunk of the tile, token lane (0 .. 31)
  const int d0 = col0 + 8 * c;
  const bool vec = (D & 7) == 0 && d0 + 8 <= D;
  float wc[8][EP], dwp[8][EP];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      wc[j][e] = (d0 + j < D && e < E) ? w[(size_t)(d0 + j) * E + e] : 0.f;
      dwp[j][e] = 0.f;
    }
  if (d0 < D) {
    for (int i = tl; i < kRouterBwdTokens; i += 32) {
      const int t = tb + i;
      if (t >= T) break;
      const bf16* xrow = x + (size_t)t * D + d0;
      bf16* drow = dx + (size_t)t * D + d0;
      float xv[8], old[8];
      if (vec) {
        const bf16x8 xx = *reinterpret_cast<const bf16x8*>(xrow);
        const bf16x8 dd = *reinterpret_cast<const bf16x8*>(drow);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          xv[j] = (float)xx[j];
          old[j] = (float)dd[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          xv[j] = d0 + j < D ? (float)xrow[j] : 0.f;
          old[j] = d0 + j < D ? (float)drow[j] : 0.f;
        }
      }
      float dl[EP];
#pragma unroll
      for (int e4 = 0; e4 < EP; e4 += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&dl_s[i][e4]);
#pragma unroll
        for (int u = 0; u < 4; ++u) dl[e4 + u] = v[u];
      }
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float sj = 0.f;
#pragma unroll
        for (int e = 0; e < EP; ++e) {
          sj = fmaf(dl[e], wc[j][e], sj);
          dwp[j][e] = fmaf(xv[j], dl[e], dwp[j][e]);
        }
        o[j] = (bf16)(old[j] + (float)(bf16)sj);
      }
      if (vec) {
        *reinterpret_cast<bf16x8*>(drow) = o;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (d0 + j < D) drow[j] = o[j];
      }
    }
  }
  // Sum the token lanes: lanes 8 m + c of a wave (m = 0..7) by xor over
  // lane bits 3..5, then the 4 waves through LDS.
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      float v = dwp[j][e];
      v += __shfl_xor(v, 8);
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (lane < 8) red[wave][8 * c + j][e] = v;
    }
  __syncthreads();
  for (int i = tid; i < kRouterBwdCols * EP; i += blockDim.x) {
    const int col = i / EP, e = i % EP;
    const float v = red[0][col][e] + red[1][col][e] + red[2][col][e] + red[3][col][e];
    if (col0 + col < D && e < E) atomicAdd(dw + (size_t)(col0 + col) * E + e, v);
  }
}

}  // namespace

extern "C" {

size_t gptrig_moe_route_workspace_bytes(int tokens, int experts, int top_k) {
  if (tokens <= 0 || experts <= 0 || top_k <= 0) return 0;
  const size_t blocks = (size_t)ceil_div((int64_t)tokens * top_k, kSortBlock);
  return (blocks * experts * sizeof(int32_t) + 255) & ~(size_t)255;
}

int gptrig_moe_route(const float* logits, float* probs, int32_t* chosen, float* gate, int32_t* counts,
                     int32_t* order, int32_t* rows, int32_t* position, void* workspace, size_t workspace_bytes,
                     int tokens, int experts, int top_k, void* stream) {
  if (!logits || !chosen || !gate || !counts || !order || !rows) return GPTRIG_E_NULL;
  if (tokens <= 0 || experts <= 0 || top_k <= 0) return GPTRIG_E_SHAPE;
  if (experts > kMaxExperts || top_k > experts) return GPTRIG_E_UNSUPPORTED;
  if ((int64_t)tokens * top_k >= (1ll << 31)) return GPTRIG_E_SHAPE;
  if (!workspace || workspace_bytes < gptrig_moe_route_workspace_bytes(tokens, experts, top_k))
    return GPTRIG_E_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  route_topk_kernel<<<ceil_div(tokens, 128), 128, 0, s>>>(logits, probs, chosen, gate, tokens, experts, top_k);
  GPTRIG_CHECK_LAUNCH();
  const int n_slots = tokens * top_k, nblocks = ceil_div(n_slots, kSortBlock);
  int32_t* hist = (int32_t*)workspace;
  route_hist_kernel<<<nblocks, kSortBlock, 0, s>>>(chosen, n_slots, experts, hist);
  GPTRIG_CHECK_LAUNCH();
  route_place_kernel<<<nblocks, kSortBlock, 0, s>>>(chosen, n_slots, experts, top_k, hist, nblocks, counts, order,
                                                    rows, position);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}


int gptrig_moe_router_logits(const void* x, const float* router_w, float* logits, int tokens, int width, int experts,
                             void* stream) {
  if (!x || !router_w || !logits) return GPTRIG_E_NULL;
  if (tokens <= 0 || width <= 0 || experts <= 0) return GPTRIG_E_SHAPE;
  if (experts > kMaxRouterExperts || (size_t)width * experts * sizeof(float) > 32768) return GPTRIG_E_UNSUPPORTED;
  const int ep = experts <= 4 ? 4 : experts <= 8 ? 8 : 16;
  if ((size_t)width * ep * sizeof(float) > 65536) return GPTRIG_E_UNSUPPORTED;
  const size_t smem = (size_t)width * ep * sizeof(float);
  const unsigned grid = (unsigned)ceil_div(tokens, 4 * kRouterTokens);
  hipStream_t s = (hipStream_t)stream;
  if (ep == 4)
    router_logits_kernel<4><<<grid, 256, smem, s>>>((const bf16*)x, router_w, logits, tokens, width, experts);
  else if (ep == 8)
    router_logits_kernel<8><<<grid, 256, smem, s>>>((const bf16*)x, router_w, logits, tokens, width, experts);
  else
    router_logits_kernel<16><<<grid, 256, smem, s>>>((const bf16*)x, router_w, logits, tokens, width, experts);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_gather_rows(const void* x, const int32_t* rows, void* grouped, int n_rows, int width, void* stream) {
  if (!x || !rows || !grouped) return GPTRIG_E_NULL;
  if (n_rows <= 0 || width <= 0 || width % 8) return GPTRIG_E_SHAPE;
  if (((uintptr_t)x | (uintptr_t)grouped) & 15) return GPTRIG_E_SHAPE;
  moe_gather_rows_kernel<<<ceil_div(n_rows, 4), 256, 0, (hipStream_t)stream>>>((const bf16*)x, rows, (bf16*)grouped,
                                                                               n_rows, width);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_gmm(const void* lhs, int64_t lda, const void* rhs, int rhs_transposed, const int32_t* counts,
                   const void* bias, int mode, void* out, void* pre, int64_t ldo, int rows, int k, int n, int experts,
                   void* stream) {
  if (!lhs || !rhs || !counts || !out) return GPTRIG_E_NULL;
  if ((mode == 1 || mode == 2) && !pre) return GPTRIG_E_NULL;
  if (rows <= 0 || k <= 0 || n <= 0 || experts <= 0 || mode < 0 || mode > 2) return GPTRIG_E_SHAPE;
  if (k % 8 || n % 8 || lda % 8 || lda < k || ldo < n || ldo % 8) return GPTRIG_E_SHAPE;
  if (((uintptr_t)lhs | (uintptr_t)rhs | (uintptr_t)out | (uintptr_t)pre) & 15) return GPTRIG_E_SHAPE;
  if (experts > kMaxExperts) return GPTRIG_E_UNSUPPORTED;
  const unsigned grid = (unsigned)((ceil_div(rows, gemm::BM) + experts) * ceil_div(n, gemm::BN));
  hipStream_t s = (hipStream_t)stream;
  const bf16* L = (const bf16*)lhs;
  const bf16* Rh = (const bf16*)rhs;
  const bf16* Bi = (const bf16*)bias;
  bf16* O = (bf16*)out;
  bf16* P = (bf16*)pre;
#define GPTRIG_GMM(BT, MODE)                                                                                     \
  moe_gmm_kernel<BT, MODE><<<grid, gemm::THREADS, 0, s>>>(L, lda, Rh, counts, experts, k, n, Bi, O, P, ldo)
  if (rhs_transposed) {
    if (mode == 0) GPTRIG_GMM(true, 0);
    else if (mode == 1) GPTRIG_GMM(true, 1);
    else GPTRIG_GMM(true, 2);
  } else {
    if (mode == 0) GPTRIG_GMM(false, 0);
    else if (mode == 1) GPTRIG_GMM(false, 1);
    else GPTRIG_GMM(false, 2);
  }
#undef GPTRIG_GMM
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_gmm_dw(const void* lhs, int64_t lda, const void* dy, int64_t ldy, const int32_t* counts, float* dw,
                      float* db, int rows, int k, int n, int experts, void* stream) {
  if (!lhs || !dy || !counts || !dw) return GPTRIG_E_NULL;
  if (rows <= 0 || k <= 0 || n <= 0 || experts <= 0) return GPTRIG_E_SHAPE;
  if (k % 8 || n % 8 || lda % 8 || ldy % 8 || lda < k || ldy < n) return GPTRIG_E_SHAPE;
  if (((uintptr_t)lhs | (uintptr_t)dy) & 15) return GPTRIG_E_SHAPE;
  if (experts > kMaxExperts) return GPTRIG_E_UNSUPPORTED;
  const unsigned tiles = (unsigned)(ceil_div(k, gemm::BM) * ceil_div(n, gemm::BN));
  // No split once E x tiles fills the GPU (every split adds an atomic
  // epilogue per tile); below that, short split blocks, which in the training
  // step also leave room for the main stream's kernels beside this one (on
  // the weight-gradient stream): config E measured 46.6 ms/step with them
  // against 49.2 ms with 144 unsplit blocks, and 60.7 against 62.5 ms with
  // 288 unsplit blocks instead of split ones.
  const int64_t cells = (int64_t)tiles * experts;
  const int split = cells >= gemm::device_cus() ? 1 : gemm::choose_split(tiles * experts,
                                                                         ceil_div(ceil_div(rows, experts), gemm::BK));
  moe_gmm_dw_kernel<<<tiles * experts * split, gemm::THREADS, 0, (hipStream_t)stream>>>(
      (const bf16*)lhs, lda, (const bf16*)dy, ldy, counts, experts, k, n, split, dw, db);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_combine(const void* out, const int32_t* position, const float* gate, void* combined, int tokens,
                       int width, int top_k, void* stream) {
  if (!out || !position || !gate || !combined) return GPTRIG_E_NULL;
  if (tokens <= 0 || width <= 0 || top_k <= 0 || width % 8) return GPTRIG_E_SHAPE;
  if (top_k > kMaxTopK) return GPTRIG_E_UNSUPPORTED;
  moe_combine_kernel<<<ceil_div(tokens, 4), 256, 0, (hipStream_t)stream>>>((const bf16*)out, position, gate,
                                                                          (bf16*)combined, tokens, width, top_k);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_combine_bwd(const void* dcombined, const void* out, const int32_t* position, const float* gate,
                           void* dout, float* dgate, int tokens, int width, int top_k, void* stream) {
  if (!dcombined || !out || !position || !gate || !dout || !dgate) return GPTRIG_E_NULL;
  if (tokens <= 0 || width <= 0 || top_k <= 0 || width % 8) return GPTRIG_E_SHAPE;
  if (top_k > kMaxTopK) return GPTRIG_E_UNSUPPORTED;
  moe_combine_bwd_kernel<<<ceil_div((long long)tokens * top_k, 4), 256, 0, (hipStream_t)stream>>>(
      (const bf16*)dcombined, (const bf16*)out, position, gate, (bf16*)dout, dgate, tokens, width, top_k);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_gather_bwd(const void* dgrouped, const int32_t* position, void* dx, int tokens, int width, int top_k,
                          void* stream) {
  if (!dgrouped || !position || !dx) return GPTRIG_E_NULL;
  if (tokens <= 0 || width <= 0 || top_k <= 0 || width % 8) return GPTRIG_E_SHAPE;
  if (top_k > kMaxTopK) return GPTRIG_E_UNSUPPORTED;
  moe_gather_bwd_kernel<<<ceil_div(tokens, 4), 256, 0, (hipStream_t)stream>>>((const bf16*)dgrouped, position,
                                                                             (bf16*)dx, tokens, width, top_k);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_stats(const float* logits, const float* probs, const float* gate, const int32_t* counts, int tokens,
                     int experts, int top_k, float* mean_probability, float* load, float* summary, void* stream) {
  if (!logits || !probs || !gate || !counts || !mean_probability || !load || !summary) return GPTRIG_E_NULL;
  if (tokens <= 0 || experts <= 0 || top_k <= 0 || top_k > experts) return GPTRIG_E_SHAPE;
  if (experts > kMaxRouterExperts) return GPTRIG_E_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  stats_zero_kernel<<<1, 64, 0, s>>>(mean_probability, summary, experts);
  GPTRIG_CHECK_LAUNCH();
  const unsigned grid = (unsigned)ceil_div(tokens, 256);
  if (experts <= 4)
    moe_stats_kernel<4><<<grid, 256, 0, s>>>(logits, probs, gate, tokens, experts, top_k, mean_probability, summary);
  else if (experts <= 8)
    moe_stats_kernel<8><<<grid, 256, 0, s>>>(logits, probs, gate, tokens, experts, top_k, mean_probability, summary);
  else
    moe_stats_kernel<16><<<grid, 256, 0, s>>>(logits, probs, gate, tokens, experts, top_k, mean_probability, summary);
  GPTRIG_CHECK_LAUNCH();
  stats_finalize_kernel<<<1, 64, 0, s>>>(counts, tokens, experts, top_k, mean_probability, load, summary);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_moe_router_bwd(const void* x, const float* router_w, const float* probs, const int32_t* chosen,
                          const float* gate, const float* dgate, const float* dmean_probability, void* dx,
                          float* dw_router, int tokens, int width, int experts, int top_k, void* stream) {
  if (!x || !router_w || !probs || !chosen || !gate || !dgate || !dx || !dw_router) return GPTRIG_E_NULL;
  if (tokens <= 0 || width <= 0 || experts <= 0 || top_k <= 0 || top_k > experts) return GPTRIG_E_SHAPE;
  if (experts > kMaxRouterExperts || (size_t)width * experts * sizeof(float) > 32768) return GPTRIG_E_UNSUPPORTED;
  const dim3 grid((unsigned)ceil_div(width, kRouterBwdCols), (unsigned)ceil_div(tokens, kRouterBwdTokens));
  hipStream_t s = (hipStream_t)stream;
  if (experts <= 4)
    router_bwd_kernel<4><<<grid, 256, 0, s>>>((const bf16*)x, router_w, probs, chosen, gate, dgate, dmean_probability,
                                              (bf16*)dx, dw_router, tokens, width, experts, top_k);
  else if (experts <= 8)
    router_bwd_kernel<8><<<grid, 256, 0, s>>>((const bf16*)x, router_w, probs, chosen, gate, dgate, dmean_probability,
                                              (bf16*)dx, dw_router, tokens, width, experts, top_k);
  else
    router_bwd_kernel<16><<<grid, 256, 0, s>>>((const bf16*)x, router_w, probs, chosen, gate, dgate,
                                               dmean_probability, (bf16*)dx, dw_router, tokens, width, experts, top_k);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // extern "C"
