// Output stage shared by the transposed-tile GEMM kernels (csrc/linear.hip
// and the grouped expert GEMM of csrc/moe.hip): MFMA rows are output
// features, columns are tokens, and the tile leaves through LDS in whole
// token rows with the elementwise pass that follows the product fused in.
#pragma once

#include "gemm_core.h"

namespace gemm_epi {

using gemm::BM;
using gemm::BN;

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

// The output tile goes out through the stage arrays, which the main loop no
// longer needs: each lane first writes its four consecutive features of one
// token (acc[mb][nb][4q + j] = out[token tn*BN + 64wn + 32nb + l32][feature
// tm*BM + 128wm + 32mb + 8q + 4hl + j]) as bf16 into a [token][feature] tile,
// then every thread takes 16-byte runs of 8 features of one token, so each
// wave writes whole 512-byte token rows (the register layout would scatter
// every store instruction over 32 rows).  The GELU, its derivative and the
// RoPE rotation run in that second pass, on 8 features of one token.
// Tile row r (a token) sits in stage array r / 64 at (r % 64) * 256; its
// 16-byte chunk c at position c ^ (r % 32), so the 32 tokens a store
// instruction covers spread over the banks.
__device__ __forceinline__ gemm::lds_t* tile_row(int r) {
  gemm::lds_t* const band[4] = {gemm::stage_ptr<0>(), gemm::stage_ptr<1>(), gemm::stage_ptr<2>(),
                                gemm::stage_ptr<3>()};
  return band[r >> 6] + (r & 63) * 256;
}

template <int kEpi>
__device__ __forceinline__ void linear_epilogue(const f32x16 (&acc)[4][2], int tm, int tn, int F, int N,
                                                const EpiArgs& e, const float* bias_s) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  wg_barrier();  // every wave is done with the last stage
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int r = 64 * wn + 32 * nb + l32;
    gemm::lds_t* const row = tile_row(r);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int fl = 128 * wm + 32 * mb + 8 * q + 4 * hl;
        bf16x4 o;
        if constexpr (has_bias(kEpi)) {
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(bias_s + fl);
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = (bf16)((float)(bf16)acc[mb][nb][4 * q + j] + b4[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = (bf16)acc[mb][nb][4 * q + j];
        }
        *(__attribute__((address_space(3))) bf16x4*)(row + 8 * ((fl >> 3) ^ (r & 31)) + 4 * hl) = o;
      }
  }
  GPTRIG_WAIT_LGKM0();
  wg_barrier();
#pragma unroll 4
  for (int it = 0; it < BM * BN / 8 / gemm::THREADS; ++it) {
    const int idx = tid + gemm::THREADS * it;
    const int r = idx >> 5, c = idx & 31;
    const int tok = tn * BN + r, f = tm * BM + 8 * c;
    // F is a multiple of 8, so f < F covers f .. f+7.
    if (tok >= N || f >= F) continue;
    bf16x8 v = *(const gemm::lds_x8*)(tile_row(r) + 8 * (c ^ (r & 31)));
    if constexpr (kEpi == kGelu) {
      bf16x8 g;
#pragma unroll
      for (int j = 0; j < 8; ++j) g[j] = (bf16)gelu_f((float)v[j]);
      *reinterpret_cast<bf16x8*>(e.act + (int64_t)tok * e.ldy + f) = g;
    } else if constexpr (kEpi == kDGelu) {
      const bf16x8 h = *reinterpret_cast<const bf16x8*>(e.aux + (int64_t)tok * e.ldaux + f);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (bf16)((float)v[j] * gelu_grad_f((float)h[j]));
    } else if constexpr (kEpi == kRope) {
      if (f < e.rope_cols) {
        // Four pairs of one head; head_dim % 8 == 0 keeps them in one head and
        // their four table entries in one 8-byte load.
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
}


}  // namespace gemm_epi
