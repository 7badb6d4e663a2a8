// Dense linear layers of the GPT block (rig/nn.py:55-56, `linear`) on the
// GEMM core, with the elementwise pass that follows each of them fused into
// the epilogue.
//
// The output tile is computed transposed: MFMA rows are output features and
// MFMA columns are tokens (A = the weight as [feature][k], B = the
// activations [token][k], both K-major when the weight is stored [out][in]),
// so each lane holds four consecutive features of one token and writes them
// with one 8-byte store.  Epilogues, in the reference's rounding order:
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
// K a multiple of 128 with a K-major weight runs gemm::persistent (one
// workgroup per CU walking the tiles, the next tile's operands in flight
// during the epilogue); other shapes run one workgroup per tile.
#include "gemm_core.h"

namespace {

using gemm::BM;
using gemm::BN;
using gemm::Operand;

enum { kPlain = 0, kBias = 1, kGelu = 2, kRope = 3, kDGelu = 4 };

struct EpiArgs {
  bf16* y;
  int64_t ldy;
  const bf16* bias;   // kBias, kGelu, kRope (nullable: zero bias)
  bf16* act;          // kGelu: gelu(h), leading dimension ldy
  const bf16* aux;    // kDGelu: h
  int64_t ldaux;
  const bf16* rcs;    // kRope: bf16 cos / sin tables [seq][head_dim / 2]
  const bf16* rsn;
  int seq, rope_cols, head_dim;
};

constexpr bool has_bias(int e) { return e == kBias || e == kGelu || e == kRope; }

__device__ __forceinline__ void stage_bias(float* dst, const bf16* bias, int f_base, int F) {
  const int tid = threadIdx.x;
  if (tid < BM) {
    const int f = f_base + tid;
    dst[tid] = (bias && f < F) ? (float)bias[f] : 0.f;
  }
}

// acc[mb][nb][4q + j] = out[token tn*BN + 64wn + 32nb + l32][feature tm*BM + 128wm + 32mb + 8q + 4hl + j].
template <int kEpi>
__device__ __forceinline__ void linear_epilogue(const f32x16 (&acc)[4][2], int tm, int tn, int F, int N,
                                                const EpiArgs& e, const float* bias_s) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int tok = tn * BN + 64 * wn + 32 * nb + l32;
    if (tok >= N) continue;
    const int pos = kEpi == kRope ? tok % e.seq : 0;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int fl = 128 * wm + 32 * mb + 8 * q + 4 * hl;
        const int f0 = tm * BM + fl;
        // F is a multiple of 4 and f0 of 4, so f0 < F covers f0 .. f0+3.
        if (f0 >= F) continue;
        bf16x4 o;
        if constexpr (kEpi == kPlain) {
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = (bf16)acc[mb][nb][4 * q + j];
        } else if constexpr (kEpi == kDGelu) {
          const bf16x4 h = *reinterpret_cast<const bf16x4*>(e.aux + (int64_t)tok * e.ldaux + f0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            o[j] = (bf16)((float)(bf16)acc[mb][nb][4 * q + j] * gelu_grad_f((float)h[j]));
        } else {
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(bias_s + fl);
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = (bf16)((float)(bf16)acc[mb][nb][4 * q + j] + b4[j]);
          if constexpr (kEpi == kGelu) {
            bf16x4 g;
#pragma unroll
            for (int j = 0; j < 4; ++j) g[j] = (bf16)gelu_f((float)o[j]);
            *reinterpret_cast<bf16x4*>(e.act + (int64_t)tok * e.ldy + f0) = g;
          }
          if constexpr (kEpi == kRope) {
            if (f0 < e.rope_cols) {
              // Pairs (f0, f0+1) and (f0+2, f0+3); head_dim % 4 == 0 keeps the
              // pair index even, so the two table entries are one 4-byte load.
              const int half = e.head_dim >> 1;
              const int i0 = (f0 % e.head_dim) >> 1;
              const bf16x2 c2 = *reinterpret_cast<const bf16x2*>(e.rcs + (int64_t)pos * half + i0);
              const bf16x2 s2 = *reinterpret_cast<const bf16x2*>(e.rsn + (int64_t)pos * half + i0);
              const bf16x2 r0 = rope_pair((float)o[0], (float)o[1], (float)c2[0], (float)s2[0]);
              const bf16x2 r1 = rope_pair((float)o[2], (float)o[3], (float)c2[1], (float)s2[1]);
              o = bf16x4{r0[0], r0[1], r1[0], r1[1]};
            }
          }
        }
        *reinterpret_cast<bf16x4*>(e.y + (int64_t)tok * e.ldy + f0) = o;
      }
  }
}

template <int kEpi, bool kWK>
__global__ void __launch_bounds__(gemm::THREADS)
    linear_persistent_kernel(Operand W, Operand X, int F, int N, int K, int group, EpiArgs e) {
  __shared__ __attribute__((aligned(16))) float bias_s[2][BM];
  const int ntiles = ((F + BM - 1) / BM) * ((N + BN - 1) / BN);
  int pre_it = 0, epi_it = 0;
  auto coords = [&](int t, int& tm, int& tn) { gemm::tile_coords(t, F, N, tm, tn, group); };
  // The bias of the next tile is staged after the current tile's epilogue,
  // into the other buffer (other waves may still be reading this one).
  auto pre = [&](int tm, int) {
    if constexpr (has_bias(kEpi)) stage_bias(bias_s[pre_it & 1], e.bias, tm * BM, F);
    ++pre_it;
  };
  auto epi = [&](f32x16(&acc)[4][2], int tm, int tn) {
    linear_epilogue<kEpi>(acc, tm, tn, F, N, e, bias_s[epi_it & 1]);
    ++epi_it;
  };
  gemm::persistent<kWK, true>(W, X, F, N, K, ntiles, coords, pre, epi);
}

template <int kEpi, bool kWK>
__global__ void __launch_bounds__(gemm::THREADS)
    linear_tile_kernel(Operand W, Operand X, int F, int N, int K, int group, EpiArgs e) {
  __shared__ __attribute__((aligned(16))) float bias_s[BM];
  int tm, tn;
  gemm::tile_coords(blockIdx.x, F, N, tm, tn, group);
  // Visible to every wave after the mainloop's first barrier.
  if constexpr (has_bias(kEpi)) stage_bias(bias_s, e.bias, tm * BM, F);
  f32x16 acc[4][2];
  gemm::mainloop<kWK, true>(acc, W, X, F, N, 0, K, tm * BM, tn * BN);
  linear_epilogue<kEpi>(acc, tm, tn, F, N, e, bias_s);
}

template <int kEpi>
int launch_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, int n, int k, int f,
                  const EpiArgs& e, hipStream_t s) {
  if (!x || !w || !e.y) return GPTRIG_E_NULL;
  if (n <= 0 || k <= 0 || f <= 0) return GPTRIG_E_SHAPE;
  if (k % 8 || f % 8 || ldx % 8 || ldw % 8 || e.ldy % 4 || ldx < k || e.ldy < f) return GPTRIG_E_SHAPE;
  if (w_kmajor ? ldw < k : ldw < f) return GPTRIG_E_SHAPE;
  if (((uintptr_t)x | (uintptr_t)w) & 15) return GPTRIG_E_SHAPE;
  if ((uintptr_t)e.y & 7) return GPTRIG_E_SHAPE;
  const Operand W{(const bf16*)w, ldw}, X{(const bf16*)x, ldx};
  const unsigned tiles = (unsigned)(ceil_div(f, BM) * ceil_div(n, BN));
  const int group = gemm::kGroupM;
  // (The persistent form is kept to K-major weights: with an MN-major weight
  // its epilogues spill, and a scratch reload waits for every copy in flight.)
  if (k % 128 == 0 && w_kmajor) {
    const unsigned cus = (unsigned)gemm::device_cus();
    const unsigned grid = tiles < cus ? tiles : cus;
    linear_persistent_kernel<kEpi, true><<<grid, gemm::THREADS, 0, s>>>(W, X, f, n, k, group, e);
  } else {
    if (w_kmajor)
      linear_tile_kernel<kEpi, true><<<tiles, gemm::THREADS, 0, s>>>(W, X, f, n, k, group, e);
    else
      linear_tile_kernel<kEpi, false><<<tiles, gemm::THREADS, 0, s>>>(W, X, f, n, k, group, e);
  }
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
  if ((uintptr_t)g & 7) return GPTRIG_E_SHAPE;
  EpiArgs e = make_args(h, ldy, bias);
  e.act = (bf16*)g;
  return launch_linear<kGelu>(x, ldx, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
}

int gptrig_linear_rope(const void* x, int64_t ldx, const void* w, int64_t ldw, int w_kmajor, const void* bias,
                       void* y, int64_t ldy, int n, int k, int f, const void* cos_table, const void* sin_table,
                       int seq, int rope_cols, int head_dim, void* stream) {
  if (!cos_table || !sin_table) return GPTRIG_E_NULL;
  if (seq <= 0 || head_dim <= 0 || head_dim % 4 || rope_cols < 0 || rope_cols % head_dim || rope_cols > f)
    return GPTRIG_E_SHAPE;
  if (((uintptr_t)cos_table | (uintptr_t)sin_table) & 3) return GPTRIG_E_SHAPE;
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
  if (ldh % 4 || ldh < f || ((uintptr_t)h & 7)) return GPTRIG_E_SHAPE;
  EpiArgs e = make_args(dx, lddx, nullptr);
  e.aux = (const bf16*)h;
  e.ldaux = ldh;
  return launch_linear<kDGelu>(dy, lddy, w, ldw, w_kmajor, n, k, f, e, (hipStream_t)stream);
}

}  // extern "C"
