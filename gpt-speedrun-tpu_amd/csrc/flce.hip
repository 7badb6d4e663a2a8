// Fused linear cross-entropy for gfx950 (rig/kernels/linear_cross_entropy.py).
//
// All contractions run through one bf16 MFMA GEMM template (fp32 accumulate,
// 128x128x32 workgroup tiles, LDS double buffering) with fused epilogues:
//
//   forward  (:115-179)  logits^T tile = W_tile h^T  -> per-row partial
//            (max, sum exp) over the tile's 128 vocabulary rows + the target
//            logit; a combine pass gives lse and loss = lse - target_logit.
//            The [n, vocab] logits never exist.
//   backward (:220-302)  per vocabulary chunk (bounded workspace, like the
//            reference's [n, tile] live logits):
//            K1  recompute logits^T, write G^T = ((exp(logit-lse) - onehot)*ct)
//                as bf16 [chunk, n] (zero for rows >= semantic vocab);
//            K2  dW[chunk] = G^T h          (fp32, store or accumulate);
//            K3  dh_acc   += G W[chunk]     (fp32), rounded to bf16 at the end.
//
// The GEMM computes C[m][n] = sum_k A(m,k) B(k,n).  Each operand is either
// K-major (A[m*ld+k], B[n*ld+k]) or MN-major (A[k*ld+m], B[k*ld+n]); an
// MN-major operand is transposed while being written to LDS so every MFMA
// fragment read is one 16-byte LDS load.
#include "common.h"

#include <math.h>

namespace {

constexpr int TM = 128, TN = 128, TK = 32;
constexpr int LDK = TK + 8;  // LDS row stride (elements): 80-byte rows
constexpr int kGroupM = 8;

struct Operand {
  const bf16* p;
  int64_t ld;
};

// Global -> registers: one 128 x 32 tile slab, two 16-byte chunks per thread.
template <bool KMAJOR>
__device__ __forceinline__ void load_slab(bf16x8 (&st)[2], Operand op, int mn0, int k0, int MN, int K, int tid) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = tid + 256 * r;
    if (KMAJOR) {
      const int row = idx >> 2, kc = (idx & 3) * 8;
      const int m = mn0 + row, k = k0 + kc;
      st[r] = (m < MN && k < K) ? *reinterpret_cast<const bf16x8*>(op.p + (int64_t)m * op.ld + k) : bf16x8{};
    } else {
      const int kk = idx >> 4, mc = (idx & 15) * 8;
      const int m = mn0 + mc, k = k0 + kk;
      st[r] = (m < MN && k < K) ? *reinterpret_cast<const bf16x8*>(op.p + (int64_t)k * op.ld + m) : bf16x8{};
    }
  }
}

template <bool KMAJOR>
__device__ __forceinline__ void store_slab(bf16* lds, const bf16x8 (&st)[2], int tid) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = tid + 256 * r;
    if (KMAJOR) {
      const int row = idx >> 2, kc = (idx & 3) * 8;
      *reinterpret_cast<bf16x8*>(lds + row * LDK + kc) = st[r];
    } else {
      const int kk = idx >> 4, mc = (idx & 15) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) lds[(mc + j) * LDK + kk] = st[r][j];
    }
  }
}

__device__ __forceinline__ void tile_coords(int M, int N, int& tm, int& tn) {
  const int mt = (M + TM - 1) / TM, nt = (N + TN - 1) / TN;
  const int pid = blockIdx.x;
  const int in_group = kGroupM * nt;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsize = min(mt - first_m, kGroupM);
  tm = first_m + (pid % in_group) % gsize;
  tn = (pid % in_group) / gsize;
}

// Main loop: acc[mb][nb] is the wave's 64x64 sub-tile as 2x2 MFMA blocks;
// element i of acc[mb][nb] is C[m0 + 32mb + 8(i/4) + 4(lane/32) + i%4][n0 + 32nb + lane%32].
template <bool AK, bool BK>
__device__ __forceinline__ void gemm_mainloop(f32x16 (&acc)[2][2], Operand A, Operand B, int M, int N, int K,
                                              int tm0, int tn0, bf16* lds_a, bf16* lds_b) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm0 = 64 * (wave & 1), wn0 = 64 * (wave >> 1);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};
  const int nk = (K + TK - 1) / TK;
  bf16x8 sa[2], sb[2];
  load_slab<AK>(sa, A, tm0, 0, M, K, tid);
  load_slab<BK>(sb, B, tn0, 0, N, K, tid);
  store_slab<AK>(lds_a, sa, tid);
  store_slab<BK>(lds_b, sb, tid);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    bf16* la = lds_a + buf * TM * LDK;
    bf16* lb = lds_b + buf * TN * LDK;
    if (kt + 1 < nk) {
      load_slab<AK>(sa, A, tm0, (kt + 1) * TK, M, K, tid);
      load_slab<BK>(sb, B, tn0, (kt + 1) * TK, N, K, tid);
    }
#pragma unroll
    for (int kc = 0; kc < TK / 16; ++kc) {
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        fa[mb] = *reinterpret_cast<const bf16x8*>(la + (wm0 + 32 * mb + l32) * LDK + 16 * kc + 8 * hl);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        fb[nb] = *reinterpret_cast<const bf16x8*>(lb + (wn0 + 32 * nb + l32) * LDK + 16 * kc + 8 * hl);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(fa[mb], fb[nb], acc[mb][nb]);
    }
    if (kt + 1 < nk) {
      store_slab<AK>(lds_a + (buf ^ 1) * TM * LDK, sa, tid);
      store_slab<BK>(lds_b + (buf ^ 1) * TN * LDK, sb, tid);
    }
    __syncthreads();
  }
}

#define GEMM_SMEM                                                   \
  __shared__ __attribute__((aligned(16))) bf16 lds_a[2 * TM * LDK]; \
  __shared__ __attribute__((aligned(16))) bf16 lds_b[2 * TN * LDK];

// ---------------------------------------------------------------------------
// Forward: C = logits^T (m = vocab row, n = token).  Partial (max, sum exp)
// over the tile's vocabulary rows in the log2 domain, per token.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256, 2)
    flce_fwd_kernel(Operand W, Operand Hd, int V, int N, int D, int sem_v, const int32_t* __restrict__ targets,
                    float2* __restrict__ partial, float* __restrict__ tlogit) {
  GEMM_SMEM
  __shared__ float2 xchg[2][64];
  int tm, tn;
  tile_coords(V, N, tm, tn);
  f32x16 acc[2][2];
  gemm_mainloop<true, true>(acc, W, Hd, V, N, D, tm * TM, tn * TN, lds_a, lds_b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  const int vbase = tm * TM + 64 * wm;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = tn * TN + 64 * wn + 32 * nb + l32;
    const int t = n < N ? targets[n] : -1;
    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = vbase + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
        const float x = acc[mb][nb][i];
        if (v == t && n < N) tlogit[n] = x;
        const float y = v < sem_v ? x * GPTRIG_LOG2E : -INFINITY;
        acc[mb][nb][i] = y;
        mx = fmaxf(mx, y);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    float sum = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) sum += fast_exp2(acc[mb][nb][i] - mx);
    }
    sum += __shfl_xor(sum, 32);
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
__global__ void __launch_bounds__(256, 2)
    flce_grad_kernel(Operand W, Operand Hd, int Vc, int N, int D, int v0, int V, int sem_v,
                     const int32_t* __restrict__ targets, const float* __restrict__ lse,
                     const float* __restrict__ cot, float cot_scale, bf16* __restrict__ gt) {
  GEMM_SMEM
  int tm, tn;
  tile_coords(Vc, N, tm, tn);
  f32x16 acc[2][2];
  gemm_mainloop<true, true>(acc, W, Hd, Vc, N, D, tm * TM, tn * TN, lds_a, lds_b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = tn * TN + 64 * wn + 32 * nb + l32;
    if (n >= N) continue;
    const int t = targets[n];
    const bool valid_t = t >= 0 && t < sem_v;
    const float ct = valid_t ? (cot ? cot[n] : cot_scale) : 0.f;
    const float l2 = lse[n] * GPTRIG_LOG2E;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int vl = tm * TM + 64 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
        const int v = v0 + vl;
        if (vl >= Vc) continue;
        float g = 0.f;
        if (v < sem_v) {
          const float p = fast_exp2(acc[mb][nb][i] * GPTRIG_LOG2E - l2);
          g = (p - (v == t ? 1.f : 0.f)) * ct;
        }
        gt[(size_t)vl * N + n] = (bf16)g;
      }
  }
}

// C stored as fp32 row-major [M][ldc] (overwrite or accumulate).
template <bool AK, bool BK>
__global__ void __launch_bounds__(256, 2)
    gemm_f32_kernel(Operand A, Operand B, int M, int N, int K, float* __restrict__ C, int64_t ldc, int accumulate) {
  GEMM_SMEM
  int tm, tn;
  tile_coords(M, N, tm, tn);
  f32x16 acc[2][2];
  gemm_mainloop<AK, BK>(acc, A, B, M, N, K, tm * TM, tn * TN, lds_a, lds_b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = tn * TN + 64 * wn + 32 * nb + l32;
    if (n >= N) continue;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = tm * TM + 64 * wm + 32 * mb + 8 * (i >> 2) + 4 * hl + (i & 3);
        if (m >= M) continue;
        float* dst = C + (int64_t)m * ldc + n;
        *dst = accumulate ? *dst + acc[mb][nb][i] : acc[mb][nb][i];
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

__global__ void zero_rows_kernel(float* __restrict__ x, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = 0.f;
}

inline unsigned grid_for(int M, int N) { return (unsigned)(ceil_div(M, TM) * ceil_div(N, TN)); }

constexpr int kDefaultChunk = 4096;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

size_t gptrig_flce_fwd_workspace_bytes(int n, int d, int vocab) {
  (void)d;
  const size_t ntiles = (size_t)ceil_div(vocab, TM);
  return align256(ntiles * n * sizeof(float2)) + align256((size_t)n * sizeof(float));
}

int gptrig_flce_fwd(const void* hidden, const void* weight, const int32_t* targets, float* losses, float* lse,
                    void* workspace, size_t workspace_bytes, int n, int d, int vocab, int semantic_vocab,
                    void* stream) {
  if (!hidden || !weight || !targets || !losses || !lse || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (workspace_bytes < gptrig_flce_fwd_workspace_bytes(n, d, vocab)) return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight) & 15) return GPTRIG_E_SHAPE;
  const int ntiles = ceil_div(vocab, TM);
  float2* partial = (float2*)workspace;
  float* tlogit = (float*)((char*)workspace + align256((size_t)ntiles * n * sizeof(float2)));
  hipStream_t s = (hipStream_t)stream;
  Operand W{(const bf16*)weight, d}, Hd{(const bf16*)hidden, d};
  flce_fwd_kernel<<<grid_for(vocab, n), 256, 0, s>>>(W, Hd, vocab, n, d, semantic_vocab, targets, partial, tlogit);
  GPTRIG_CHECK_LAUNCH();
  flce_combine_kernel<<<ceil_div(n, 256), 256, 0, s>>>(partial, ntiles, n, semantic_vocab, targets, tlogit, lse,
                                                        losses);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

size_t gptrig_flce_bwd_workspace_bytes(int n, int d, int vocab, int vocab_chunk) {
  if (vocab_chunk <= 0) vocab_chunk = kDefaultChunk;
  if (vocab_chunk > vocab) vocab_chunk = ceil_div(vocab, TM) * TM;
  return align256((size_t)vocab_chunk * n * sizeof(bf16)) + align256((size_t)n * d * sizeof(float));
}

int gptrig_flce_bwd(const void* hidden, const void* weight, const int32_t* targets, const float* lse,
                    const float* cotangent, float cotangent_scale, void* dhidden, float* dweight,
                    int accumulate_dweight, void* workspace, size_t workspace_bytes, int n, int d, int vocab,
                    int semantic_vocab, int vocab_chunk, void* stream) {
  if (!hidden || !weight || !targets || !lse || !dhidden || !dweight || !workspace) return GPTRIG_E_NULL;
  if (n <= 0 || d <= 0 || vocab <= 0 || d % 64) return GPTRIG_E_SHAPE;
  if (semantic_vocab <= 0 || semantic_vocab > vocab) return GPTRIG_E_SHAPE;
  if (vocab_chunk < 0 || vocab_chunk % 256) return GPTRIG_E_SHAPE;
  if (n % 8) return GPTRIG_E_UNSUPPORTED;  // MN-major 16-byte loads of h and G^T rows
  if (workspace_bytes < gptrig_flce_bwd_workspace_bytes(n, d, vocab, vocab_chunk)) return GPTRIG_E_WORKSPACE;
  if (((uintptr_t)hidden | (uintptr_t)weight | (uintptr_t)workspace) & 15) return GPTRIG_E_SHAPE;
  int chunk = vocab_chunk <= 0 ? kDefaultChunk : vocab_chunk;
  if (chunk > vocab) chunk = ceil_div(vocab, TM) * TM;
  bf16* gt = (bf16*)workspace;
  float* dh_acc = (float*)((char*)workspace + align256((size_t)chunk * n * sizeof(bf16)));
  hipStream_t s = (hipStream_t)stream;
  const bf16* Wp = (const bf16*)weight;
  const bf16* Hp = (const bf16*)hidden;
  for (int v0 = 0; v0 < vocab; v0 += chunk) {
    const int vc = vocab - v0 < chunk ? vocab - v0 : chunk;
    Operand Wc{Wp + (size_t)v0 * d, d}, Hd{Hp, d};
    flce_grad_kernel<<<grid_for(vc, n), 256, 0, s>>>(Wc, Hd, vc, n, d, v0, vocab, semantic_vocab, targets, lse,
                                                      cotangent, cotangent_scale, gt);
    GPTRIG_CHECK_LAUNCH();
    // dW[v0:v0+vc] = G^T h : A = G^T [vc][n] (K-major), B = h [n][d] (MN-major).
    Operand Ag{gt, n}, Bh{Hp, d};
    gemm_f32_kernel<true, false><<<grid_for(vc, d), 256, 0, s>>>(Ag, Bh, vc, d, n, dweight + (size_t)v0 * d, d,
                                                                 accumulate_dweight);
    GPTRIG_CHECK_LAUNCH();
    // dh += G W[v0:v0+vc] : A(m=n, k=v) = G^T [vc][n] (MN-major), B(k=v, n=j) = W [vc][d] (MN-major).
    Operand Agt{gt, n}, Bw{Wp + (size_t)v0 * d, d};
    gemm_f32_kernel<false, false><<<grid_for(n, d), 256, 0, s>>>(Agt, Bw, n, d, vc, dh_acc, d, v0 > 0);
    GPTRIG_CHECK_LAUNCH();
  }
  const int64_t total = (int64_t)n * d;
  f32_to_bf16_kernel<<<ceil_div(ceil_div(total, 4), 256), 256, 0, s>>>(dh_acc, (bf16*)dhidden, total);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // extern "C"
