// Dense linear layers of the GPT block (rig/nn.py:55-56, `linear`) on the
// GEMM core, with the elementwise pass that follows each of them fused into
// the epilogue.
//
// The output tile is computed transposed: MFMA rows are output features and
// MFMA columns are tokens (A = the weight as [feature][k], B = the
// activations [token][k], both K-major when the weight is stored [out][in]),
// so each lane holds four consecutive features of one token; the tile is then
// written out through LDS in whole token rows.  Epilogues, in the reference's
// rounding order:
//   kPlain  y  = bf16(acc)                                  (input gradient)
//   kBias   y  = bf16(bf16(acc) + b)                        (linear)
//   kGelu   h  = bf16(bf16(acc) + b), g = bf16(gelu(h))     (MLP up-projection
//                                                             then jax.nn.gelu,
//                                                             train.py:1170-1171)
//   kRope   y  = bf16(bf16(acc) + b), then the interleaved RoPE rotation of
//                 features < rope_cols (QKV projection then apply_rotary on q
//                 and k, train.py:1136-1142, rig/nn.py:36-52)
//   kDGelu  dh = bf16(bf16(acc) * gelu'(h))                 (input gradient of
//                                                             the down-projection
//                                                             times the GELU VJP)
// bf16(acc) + b and the rotation round exactly as the standalone passes
// (gelu_fwd / gelu_bwd / rope kernels) do on a bf16 GEMM output.
//
// K a multiple of 128: the persistent main loop (one workgroup per CU walking
// the tiles, the next tile's operands in flight during each epilogue).  Other
// K: one workgroup per 256 x 256 tile, on the ping-pong main loop.
#include "epilogue.h"

namespace {

using gemm::BM;
using gemm::BN;
using gemm::Operand;
using namespace gemm_epi;

template <int kEpi, bool kWK>
__global__ void __launch_bounds__(gemm::THREADS)
    linear_tile_kernel(Operand W, Operand X, int F, int N, int K, int group, EpiArgs e) {
  __shared__ __attribute__((aligned(16))) float bias_s[BM];
  int tm, tn;
  gemm::tile_coords(blockIdx.x, F, N, tm, tn, group);
  // Visible to every wave after the main loop's first barrier.
  if constexpr (has_bias(kEpi)) stage_bias(bias_s, e.bias, tm * BM, F);
  f32x16 acc[4][2];
  gemm::mainloop_pp<kWK, true>(acc, W, X, F, N, 0, K, tm * BM, tn * BN);
  linear_epilogue<kEpi>(acc, tm, tn, F, N, e, bias_s);
}

// ---- persistent form ----
//
// One workgroup per CU walks tiles blockIdx.x, blockIdx.x + gridDim.x, ...;
// the next tile's first four stages are copied while the current tile's
// epilogue runs (gemm::persistent), so no tile pays the operand latency of a
// fresh launch.  The stage ring is then busy during the epilogue, so the tile
// leaves through a 32 KB band of its own, one 64-feature band at a time: band
// p holds features 32p .. 32p + 31 of both M halves (accumulator block mb =
// p of every wave) for all 256 tokens.  Band row r (a token) is 128 bytes =
// 8 chunks of 8 features; chunk c (features 128 (c / 4) + 32p + 8 (c % 4))
// sits at position c ^ (r % 8).
constexpr int kBandFeat = 64;

__device__ __forceinline__ int band_feature(int tm, int p, int c) {
  return tm * BM + 128 * (c >> 2) + 32 * p + 8 * (c & 3);
}

template <int kEpi, bool kWK>
__global__ void __launch_bounds__(gemm::THREADS)
    linear_persistent_kernel(Operand W, Operand X, int F, int N, int K, int group, EpiArgs e) {
  __shared__ __attribute__((aligned(1024))) bf16 band_s[BN * kBandFeat];
  typedef __attribute__((address_space(3))) bf16 lds_bf16;
  lds_bf16* const band = (lds_bf16*)band_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31, wm = wave & 1, wn = wave >> 1;
  const int ntiles = ((F + BM - 1) / BM) * ((N + BN - 1) / BN);
  // Read-phase position of this thread: chunk c of rows r0 + 64 it.
  const int c = tid & 7, r0 = tid >> 3;
  auto coords = [&](int t, int& tm, int& tn) { gemm::tile_coords(t, F, N, tm, tn, group); };
  auto pre = [](int, int) {};
  auto epi = [&](f32x16(&acc)[4][2], int tm, int tn) {
    // Per-pass inputs loaded one pass ahead: the saved pre-activation (kDGelu).
    bf16x8 aux[2][4];
    auto load_aux = [&](int p, bf16x8(&dst)[4]) {
      if constexpr (kEpi == kDGelu) {
        const int f = band_feature(tm, p, c);
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const int tok = tn * BN + r0 + 64 * it;
          dst[it] = (tok < N && f < F) ? *reinterpret_cast<const bf16x8*>(e.aux + (int64_t)tok * e.ldaux + f)
                                       : bf16x8{};
        }
      }
    };
    load_aux(0, aux[0]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (p < 3) load_aux(p + 1, aux[(p + 1) & 1]);
      const int f = band_feature(tm, p, c);
      bf16x8 b8{};
      if constexpr (has_bias(kEpi))
        if (e.bias && f < F)  // (the bias may sit at any 2-byte offset)
#pragma unroll
          for (int j = 0; j < 8; ++j) b8[j] = e.bias[f + j];
      // Write phase: bf16(acc) of block mb = p into the band.
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int r = 64 * wn + 32 * nb + l32;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bf16x4 o;
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = (bf16)acc[p][nb][4 * q + j];
          *(__attribute__((address_space(3))) bf16x4*)(band + r * kBandFeat + 8 * ((4 * wm + q) ^ (r & 7)) + 4 * hl) =
              o;
        }
      }
      GPTRIG_WAIT_LGKM0();
      wg_barrier();
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = r0 + 64 * it;
        const int tok = tn * BN + r;
        bf16x8 v = *(const __attribute__((address_space(3))) bf16x8*)(band + r * kBandFeat + 8 * (c ^ (r & 7)));
        if (tok >= N || f >= F) continue;  // F % 8 == 0: f < F covers f .. f+7
        if constexpr (has_bias(kEpi)) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = (bf16)((float)v[j] + (float)b8[j]);
        }
        if constexpr (kEpi == kGelu) {
          bf16x8 g;
#pragma unroll
          for (int j = 0; j < 8; ++j) g[j] = (bf16)gelu_f((float)v[j]);
          *reinterpret_cast<bf16x8*>(e.act + (int64_t)tok * e.ldy + f) = g;
        } else if constexpr (kEpi == kDGelu) {
          const bf16x8 h = aux[p & 1][it];
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = (bf16)((float)v[j] * gelu_grad_f((float)h[j]));
        } else if constexpr (kEpi == kRope) {
          if (f < e.rope_cols) {
            const int half = e.head_dim >> 1;
            const int i0 = (f % e.head_dim) >> 1;
            const int64_t t0 = (int64_t)(tok % e.seq) * half + i0;
            const bf16x4 c4 = *reinterpret_cast<const bf16x4*>(e.rcs + t0);
            const bf16x4 s4 = *reinterpret_cast<const bf16x4*>(e.rsn + t0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const bf16x2 rr = rope_pair((float)v[2 * j], (float)v[2 * j + 1], (float)c4[j], (float)s4[j]);
              v[2 * j] = rr[0];
              v[2 * j + 1] = rr[1];
            }
          }
        }
        *reinterpret_cast<bf16x8*>(e.y + (int64_t)tok * e.ldy + f) = v;
      }
      GPTRIG_WAIT_LGKM0();
      wg_barrier();  // every wave has read the band before the next pass writes it
    }
  };
  gemm::persistent<kWK, true>(W, X, F, N, K, ntiles, coords, pre, epi);
}

template <int kEpi>
int launch_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, int n, int k, int f,
                  const EpiArgs& e, hipStream_t s) {
  if (!x || !w || !e.y) return GPTRIG_E_NULL;
  if (n <= 0 || k <= 0 || f <= 0) return GPTRIG_E_SHAPE;
  if (k % 8 || f % 8 || ldx % 8 || ldw % 8 || e.ldy % 8 || ldx < k || e.ldy < f) return GPTRIG_E_SHAPE;
  if (w_kmajor ? ldw < k : ldw < f) return GPTRIG_E_SHAPE;
  if (((uintptr_t)x | (uintptr_t)w) & 15) return GPTRIG_E_SHAPE;
  if ((uintptr_t)e.y & 15) return GPTRIG_E_SHAPE;
  const Operand W{(const bf16*)w, ldw}, X{(const bf16*)x, ldx};
  const unsigned tiles = (unsigned)(ceil_div(f, BM) * ceil_div(n, BN));
  const int group = gemm::kGroupM;
  if (k % (4 * gemm::BK) == 0) {
    const unsigned grid = tiles < (unsigned)gemm::device_cus() ? tiles : (unsigned)gemm::device_cus();
    const int pgroup = ceil_div(f, BM) <= 16 ? ceil_div(f, BM) : group;
    if (w_kmajor)
      linear_persistent_kernel<kEpi, true><<<grid, gemm::THREADS, 0, s>>>(W, X, f, n, k, pgroup, e);
    else
      linear_persistent_kernel<kEpi, false><<<grid, gemm::THREADS, 0, s>>>(W, X, f, n, k, pgroup, e);
    GPTRIG_CHECK_LAUNCH();
    return GPTRIG_OK;
  }
  if (w_kmajor)
    linear_tile_kernel<kEpi, true><<<tiles, gemm::THREADS, 0, s>>>(W, X, f, n, k, group, e);
  else
    linear_tile_kernel<kEpi, false><<<tiles, gemm::THREADS, 0, s>>>(W, X, f, n, k, group, e);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

EpiArgs make_args(void* y, int64_t ldy, const void* bias) {
  EpiArgs e{};
  e.y = (bf16*)y;
  e.ldy = ldy;
  e.bias = (const bf16*)bias;
  e.seq = 1;
  e.head_dim = 4;
  return e;
}

}  // namespace

extern "C" {

int gptrig_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias, void* y,
                  int64_t ldy, int n, int k, int f, void* stream) {
  const EpiArgs e = make_args(y, ldy, bias);
  if (bias) return launch_linear<kBias>(x, ldx, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
  return launch_linear<kPlain>(x, ldx, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
}

int gptrig_linear_gelu(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias,
                       void* h, void* g, int64_t ldy, int n, int k, int f, void* stream) {
  if (!g) return GPTRIG_E_NULL;
  if ((uintptr_t)g & 15) return GPTRIG_E_SHAPE;
  EpiArgs e = make_args(h, ldy, bias);
  e.act = (bf16*)g;
  return launch_linear<kGelu>(x, ldx, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
}

int gptrig_linear_rope(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias,
                       void* y, int64_t ldy, int n, int k, int f, const void* cos_table, const void* sin_table,
                       int seq, int rope_cols, int head_dim, void* stream) {
  if (!cos_table || !sin_table) return GPTRIG_E_NULL;
  if (seq <= 0 || head_dim <= 0 || head_dim % 8 || rope_cols < 0 || rope_cols % head_dim || rope_cols > f)
    return GPTRIG_E_SHAPE;
  if (((uintptr_t)cos_table | (uintptr_t)sin_table) & 7) return GPTRIG_E_SHAPE;
  EpiArgs e = make_args(y, ldy, bias);
  e.rcs = (const bf16*)cos_table;
  e.rsn = (const bf16*)sin_table;
  e.seq = seq;
  e.rope_cols = rope_cols;
  e.head_dim = head_dim;
  return launch_linear<kRope>(x, ldx, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
}

int gptrig_linear_dgelu(const void* dy, int64_t lddy, const void* w, int64_t ldw, int w_kmajor, const void* h,
                        int64_t ldh, void* dx, int64_t lddx, int n, int k, int f, void* stream) {
  if (!h) return GPTRIG_E_NULL;
  if (ldh % 8 || ldh < f || ((uintptr_t)h & 15)) return GPTRIG_E_SHAPE;
  EpiArgs e = make_args(dx, lddx, nullptr);
  e.aux = (const bf16*)h;
  e.ldaux = ldh;
  return launch_linear<kDGelu>(dy, lddy, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
}

}  // extern "C"
