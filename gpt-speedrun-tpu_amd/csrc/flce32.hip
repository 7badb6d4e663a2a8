// Fused linear cross-entropy with float32 compute (compute_dtype=float32 of
// rig/kernels/linear_cross_entropy.py:38-41): the same algorithm as the bf16
// kernels of flce.hip -- tiled logits with a per-tile (max, sum exp) in the
// forward, the logits recomputed one vocabulary chunk at a time in the
// backward -- with every product and sum in float32, as the reference's
// einsums with compute_dtype float32 (`_tile_logits`, :92-112; the backward,
// :220-302).  The [n, vocab] logits never exist; the backward's working set is
// one float32 [n, chunk] logit gradient, the reference's own [n,
// vocab_tile_size] bound.
//
// Everything runs on one float32 GEMM tile kernel (64 x 64 outputs per
// 256-thread workgroup, k in steps of 16 through LDS, 4 x 4 outputs per
// thread, the vector ALU's fused multiply-add) with four epilogues.  The
// bf16 path carries the training step; this one serves the API's float32
// mode and its tests, so it favours plain code over peak rate.
#include "common.h"

#include <math.h>

namespace {

constexpr int kT = 64;   // tile edge
constexpr int kK = 16;   // k per LDS stage

// Element (r, c) at p[r * rs + c * cs]; one of the strides is 1.
struct Mat {
  const float* p;
  int64_t rs, cs;
};

enum { kStats = 0, kGrad = 1, kStore = 2, kAccum = 3 };

struct Epi32 {
  float* out;         // kGrad: G [M][ld]; kStore / kAccum: C [M][ld]
  int64_t ld;
  float2* partial;    // kStats: [column tile][M] = (max, sum exp(logit - max)), natural units
  int col0;           // vocabulary row of output column 0 (masks, targets)
  int sem_v;          // vocabulary rows >= sem_v are not classes
  const int32_t* targets;
  const float* lse;
  const float* cot;   // per-row cotangent (nullable: cot_scale for every row)
  float cot_scale;
};

template <int kEpi>
__global__ void __launch_bounds__(256) gemm32_kernel(Mat A, Mat B, int M, int N, int K, Epi32 e) {
  __shared__ float As[kK][kT + 4], Bs[kK][kT + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.x * kT, n0 = blockIdx.y * kT;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  const bool a_k_inner = A.cs == 1, b_k_inner = B.rs == 1;
  for (int k0 = 0; k0 < K; k0 += kK) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int idx = tid + 256 * r;
      // Consecutive threads walk the unit-stride dimension.
      const int mm = a_k_inner ? idx >> 4 : idx & 63, ka = a_k_inner ? idx & 15 : idx >> 6;
      const int nn = b_k_inner ? idx >> 4 : idx & 63, kb = b_k_inner ? idx & 15 : idx >> 6;
      const int m = m0 + mm, n = n0 + nn, k1 = k0 + ka, k2 = k0 + kb;
      As[ka][mm] = (m < M && k1 < K) ? A.p[m * A.rs + k1 * A.cs] : 0.f;
      Bs[kb][nn] = (n < N && k2 < K) ? B.p[k2 * B.rs + n * B.cs] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = As[kk][4 * ty + i];
        b[i] = Bs[kk][4 * tx + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 4 * ty + i;
    if constexpr (kEpi == kStats) {
      // Row statistics over the tile's 64 columns: the 16 threads of a row
      // group are lanes 16 q .. 16 q + 15 of one wave.
      float y[4], mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int v = e.col0 + n0 + 4 * tx + j;
        y[j] = (n0 + 4 * tx + j < N && v < e.sem_v) ? acc[i][j] : -INFINITY;
        mx = fmaxf(mx, y[j]);
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      float s = 0.f;
      if (mx != -INFINITY) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s += expf(y[j] - mx);
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o);
      if (tx == 0 && m < M) e.partial[(size_t)blockIdx.y * M + m] = make_float2(mx, s);
    } else {
      if (m >= M) continue;
      float ct = 0.f, l = 0.f;
      int t = -1;
      if constexpr (kEpi == kGrad) {
        t = e.targets[m];
        const bool valid = t >= 0 && t < e.sem_v;
        ct = valid ? (e.cot ? e.cot[m] : e.cot_scale) : 0.f;
        l = e.lse[m];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + 4 * tx + j;
        if (n >= N) continue;
        float* dst = e.out + (int64_t)m * e.ld + n;
        if constexpr (kEpi == kGrad) {
          const int v = e.col0 + n;
          // (exp(logit - lse) - [v == t]) * ct, zero for non-class rows
          // (linear_cross_entropy.py:255-266).
          *dst = v < e.sem_v ? (expf(acc[i][j] - l) - (v == t ? 1.f : 0.f)) * ct : 0.f;
        } else if constexpr (kEpi == kStore) {
          *dst = acc[i][j];
        } else {
          *dst += acc[i][j];
        }
      }
    }
  }
}

// Target logit h[n] . W[t[n]] in float32 (0 for an invalid target): one wave per token.
__global__ void __launch_bounds__(256) target32_kernel(const float* __restrict__ h, const float* __restrict__ w,
                                                       const int32_t* __restrict__ targets, int N, int D, int sem_v,
                                                       float* __restrict__ tlogit) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const int t = targets[n];
  float acc = 0.f;
  if (t >= 0 && t < sem_v)
    for (int c = lane; c < D; c += 64) acc = fmaf(h[(size_t)n * D + c], w[(size_t)t * D + c], acc);
  acc = wave_sum(acc);
  if (lane == 0) tlogit[n] = acc;
}

// lse = max + log(sum) over the column tiles' partials; loss = lse - target
// logit, +inf for an invalid target.  One thread per token.
__global__ void combine32_kernel(const float2* __restrict__ partial, int ntiles, int N, int sem_v,
                                 const int32_t* __restrict__ targets, const float* __restrict__ tlogit,
                                 float* __restrict__ lse, float* __restrict__ losses) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float m = -INFINITY;
  for (int t = 0; t < ntiles; ++t) m = fmaxf(m, partial[(size_t)t * N + n].x);
  float s = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    const float2 p = partial[(size_t)t * N + n];
    if (p.x != -INFINITY) s += p.y * expf(p.x - m);
  }
  const float l = m + logf(s);
  lse[n] = l;
  const int t = targets[n];
  losses[n] = (t >= 0 && t < sem_v) ? l - tlogit[n] : INFINITY;
}

__global__ void zero32_kernel(float* __restrict__ x, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = 0.f;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int chunk32(int vocab, int vocab_chunk) {
  const int c = vocab_chunk <= 0 ? 2048 : (vocab_chunk + kT - 1) / kT * kT;
  return c < vocab ? c : (vocab + kT - 1) / kT * kT;
}

dim3 grid_of(int M, int N) { return dim3((unsigned)((M + kT - 1) / kT), (unsigned)((N + kT - 1) / kT)); }

}  // namespace

extern "C" {

size_t gptrig_flce32_fwd_workspace_bytes(int n, int d, int vocab) {
  (void)d;
  if (n <= 0 || vocab <= 0) return 0;
  const size_t ntiles = (size_t)((vocab + kT - 1) / kT);
  return align256(ntiles * n * sizeof(float2)) + align256((size_t)n * sizeof(float));
}

int gptrig_flce32_fwd(const float* hidden, const float* weight, const int32_t* targets, float* losses, float* lse,
                      void* workspace, size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab,
                      void* stream) {
  if (!hidden || !weight || !targets || !losses || !lse || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (workspace_bytes < gptrig_flce32_fwd_workspace_bytes(n, d, vocab)) return GPTRIG_E_WORKSPACE;
  if ((int64_t)n * d >= (1ll << 31) || (int64_t)vocab * d >= (1ll << 31)) return GPTRIG_E_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int ntiles = (vocab + kT - 1) / kT;
  float2* partial = (float2*)workspace;
  float* tlogit = (float*)((char*)workspace + align256((size_t)ntiles * n * sizeof(float2)));
  Epi32 e{};
  e.partial = partial;
  e.sem_v = semantic_vocab;
  // logits[token][v] = sum_d h[token][d] W[v][d]
  gemm32_kernel<kStats><<<grid_of(n, vocab), 256, 0, s>>>(Mat{hidden, d, 1}, Mat{weight, 1, d}, n, vocab, d, e);
  GPTRIG_CHECK_LAUNCH();
  target32_kernel<<<(unsigned)((n + 3) / 4), 256, 0, s>>>(hidden, weight, targets, n, d, semantic_vocab, tlogit);
  GPTRIG_CHECK_LAUNCH();
  combine32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(partial, ntiles, n, semantic_vocab, targets, tlogit,
                                                                lse, losses);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

size_t gptrig_flce32_bwd_workspace_bytes(int n, int d, int vocab, int vocab_chunk) {
  (void)d;
  if (n <= 0 || vocab <= 0) return 0;
  return align256((size_t)n * chunk32(vocab, vocab_chunk) * sizeof(float));
}

int gptrig_flce32_bwd(const float* hidden, const float* weight, const int32_t* targets, const float* lse,
                      const float* cotangent, float cotangent_scale, float* dhidden, float* dweight,
                      int accumulate_dweight, void* workspace, size_t workspace_bytes, int n, int d, int vocab,
                      int semantic_vocab, int vocab_chunk, void* stream) {
  if (!hidden || !weight || !targets || !lse || !dhidden || !dweight || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || vocab_chunk < 0) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (workspace_bytes < gptrig_flce32_bwd_workspace_bytes(n, d, vocab, vocab_chunk)) return GPTRIG_E_WORKSPACE;
  if ((int64_t)n * d >= (1ll << 31) || (int64_t)vocab * d >= (1ll << 31)) return GPTRIG_E_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int C = chunk32(vocab, vocab_chunk);
  float* G = (float*)workspace;
  zero32_kernel<<<(unsigned)(((int64_t)n * d + 255) / 256), 256, 0, s>>>(dhidden, (int64_t)n * d);
  GPTRIG_CHECK_LAUNCH();
  for (int v0 = 0; v0 < vocab; v0 += C) {
    const int c = vocab - v0 < C ? vocab - v0 : C;
    const float* Wc = weight + (int64_t)v0 * d;
    Epi32 g{};
    g.out = G;
    g.ld = c;
    g.col0 = v0;
    g.sem_v = semantic_vocab;
    g.targets = targets;
    g.lse = lse;
    g.cot = cotangent;
    g.cot_scale = cotangent_scale;
    // G[token][v] = (exp(logit - lse) - onehot) * ct for the chunk's rows.
    gemm32_kernel<kGrad><<<grid_of(n, c), 256, 0, s>>>(Mat{hidden, d, 1}, Mat{Wc, 1, d}, n, c, d, g);
    GPTRIG_CHECK_LAUNCH();
    // dh += G W[chunk]  (the reference's grad_hidden carry, :247)
    Epi32 a{};
    a.out = dhidden;
    a.ld = d;
    gemm32_kernel<kAccum><<<grid_of(n, d), 256, 0, s>>>(Mat{G, c, 1}, Mat{Wc, d, 1}, n, d, c, a);
    GPTRIG_CHECK_LAUNCH();
    // dW[chunk] (+)= G^T h  (the dynamic_update_slice of :279-283)
    Epi32 w{};
    w.out = dweight + (int64_t)v0 * d;
    w.ld = d;
    if (accumulate_dweight)
      gemm32_kernel<kAccum><<<grid_of(c, d), 256, 0, s>>>(Mat{G, 1, c}, Mat{hidden, d, 1}, c, d, n, w);
    else
      gemm32_kernel<kStore><<<grid_of(c, d), 256, 0, s>>>(Mat{G, 1, c}, Mat{hidden, d, 1}, c, d, n, w);
    GPTRIG_CHECK_LAUNCH();
  }
  return GPTRIG_OK;
}

}  // extern "C"
