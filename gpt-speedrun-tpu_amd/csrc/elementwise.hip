// HBM-bound passes of the training step: RMSNorm, GELU(tanh), interleaved RoPE,
// embedding gather/scatter, fused AdamW with the gradient-norm reduction, and
// small reductions.  Every kernel streams 16-byte vectors where the shape
// allows and falls back to a scalar tail otherwise.
#include "common.h"

#include <math.h>

namespace {

constexpr int kWave = 64;

__global__ void fill_f32_kernel(float* __restrict__ x, int64_t n, float value) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = value;
}

// ----------------------------------------------------------------------------
// RMSNorm  (rig/nn.py:26-33)
//   n  = bf16(x * rsqrt(mean(x^2) + 1e-5))      statistic in fp32
//   y  = bf16(n * scale_bf16)
// One wave per row, 4-element (8-byte) vectors; a lane always owns the same
// columns (c = lane + 64t), so the backward keeps its dscale partial in
// registers across rows.  kMaxChunks bounds the per-lane row cache (d <= 2048).
// ----------------------------------------------------------------------------
constexpr int kMaxChunks = 8;

// kAdd: the row is first formed as sum = bf16(x + bf16(branch * branch_scale))
// (the residual add in front of the norm) and written to sum_out, which may
// be x itself (each lane reads its chunks before writing them).
template <bool kAdd>
__global__ void __launch_bounds__(256) rmsnorm_fwd_kernel(const bf16* x, const bf16* __restrict__ scale,
                                                          bf16* __restrict__ y, float* __restrict__ rstd, int rows,
                                                          int d, const bf16* __restrict__ branch, float branch_scale,
                                                          bf16* sum_out, const bf16* __restrict__ branch_bias) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const bf16* xr = x + (size_t)row * d;
  bf16* yr = y + (size_t)row * d;
  const int chunks = d / 4;
  bf16x4 xv[kMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < kMaxChunks; ++t) {
    const int c = lane + kWave * t;
    if (c < chunks) {
      xv[t] = *reinterpret_cast<const bf16x4*>(xr + 4 * c);
      if (kAdd) {
        bf16x4 bv = *reinterpret_cast<const bf16x4*>(branch + (size_t)row * d + 4 * c);
        if (branch_bias) {  // the linear's own bias add, rounded before the residual add
          const bf16x4 bb = *reinterpret_cast<const bf16x4*>(branch_bias + 4 * c);
#pragma unroll
          for (int j = 0; j < 4; ++j) bv[j] = (bf16)((float)bv[j] + (float)bb[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[t][j] = (bf16)((float)xv[t][j] + (float)(bf16)((float)bv[j] * branch_scale));
        *reinterpret_cast<bf16x4*>(sum_out + (size_t)row * d + 4 * c) = xv[t];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += (float)xv[t][j] * (float)xv[t][j];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)d + 1.0e-5f);
  if (lane == 0 && rstd) rstd[row] = r;
#pragma unroll
  for (int t = 0; t < kMaxChunks; ++t) {
    const int c = lane + kWave * t;
    if (c < chunks) {
      bf16x4 sv = *reinterpret_cast<const bf16x4*>(scale + 4 * c);
      bf16x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (bf16)((float)(bf16)((float)xv[t][j] * r) * (float)sv[j]);
      *reinterpret_cast<bf16x4*>(yr + 4 * c) = o;
    }
  }
}

// The same for d % 8 == 0 with 16-byte accesses: chunk c (8 values) of a row
// is lane c % 64's (c / 64)-th, C8 = ceil(d / 512) chunks per lane.
template <bool kAdd, int C8>
__global__ void __launch_bounds__(256) rmsnorm_fwd8_kernel(const bf16* x, const bf16* __restrict__ scale,
                                                           bf16* __restrict__ y, float* __restrict__ rstd, int rows,
                                                           int d, const bf16* __restrict__ branch, float branch_scale,
                                                           bf16* sum_out, const bf16* __restrict__ branch_bias) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const bf16* xr = x + (size_t)row * d;
  bf16* yr = y + (size_t)row * d;
  const int chunks = d / 8;
  bf16x8 xv[C8];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < C8; ++t) {
    const int c = lane + kWave * t;
    if (c < chunks) {
      xv[t] = *reinterpret_cast<const bf16x8*>(xr + 8 * c);
      if (kAdd) {
        bf16x8 bv = *reinterpret_cast<const bf16x8*>(branch + (size_t)row * d + 8 * c);
        if (branch_bias) {  // the linear's own bias add, rounded before the residual add
          const bf16x8 bb = *reinterpret_cast<const bf16x8*>(branch_bias + 8 * c);
#pragma unroll
          for (int j = 0; j < 8; ++j) bv[j] = (bf16)((float)bv[j] + (float)bb[j]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[t][j] = (bf16)((float)xv[t][j] + (float)(bf16)((float)bv[j] * branch_scale));
        *reinterpret_cast<bf16x8*>(sum_out + (size_t)row * d + 8 * c) = xv[t];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += (float)xv[t][j] * (float)xv[t][j];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)d + 1.0e-5f);
  if (lane == 0 && rstd) rstd[row] = r;
#pragma unroll
  for (int t = 0; t < C8; ++t) {
    const int c = lane + kWave * t;
    if (c < chunks) {
      const bf16x8 sv = *reinterpret_cast<const bf16x8*>(scale + 8 * c);
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (bf16)((float)(bf16)((float)xv[t][j] * r) * (float)sv[j]);
      *reinterpret_cast<bf16x8*>(yr + 8 * c) = o;
    }
  }
}

// Launch of the forward: the 16-byte form when every row, the scale and the
// bias are 16-byte aligned and d <= 2048, else the 8-byte one.
template <bool kAdd>
static void launch_rmsnorm_fwd(const bf16* x, const bf16* scale, bf16* y, float* rstd, int rows, int d,
                               const bf16* branch, float branch_scale, bf16* sum, const bf16* bias, hipStream_t s) {
  const uintptr_t al = (uintptr_t)x | (uintptr_t)scale | (uintptr_t)y | (uintptr_t)branch | (uintptr_t)sum |
                       (uintptr_t)bias;
  const int c8 = ceil_div(d / 8, 64);
  const dim3 grid(ceil_div(rows, 4));
  if (d % 8 == 0 && (al & 15) == 0 && c8 <= 4) {
    if (c8 == 1) rmsnorm_fwd8_kernel<kAdd, 1><<<grid, 256, 0, s>>>(x, scale, y, rstd, rows, d, branch, branch_scale, sum, bias);
    else if (c8 == 2) rmsnorm_fwd8_kernel<kAdd, 2><<<grid, 256, 0, s>>>(x, scale, y, rstd, rows, d, branch, branch_scale, sum, bias);
    else if (c8 == 3) rmsnorm_fwd8_kernel<kAdd, 3><<<grid, 256, 0, s>>>(x, scale, y, rstd, rows, d, branch, branch_scale, sum, bias);
    else rmsnorm_fwd8_kernel<kAdd, 4><<<grid, 256, 0, s>>>(x, scale, y, rstd, rows, d, branch, branch_scale, sum, bias);
  } else {
    rmsnorm_fwd_kernel<kAdd><<<grid, 256, 0, s>>>(x, scale, y, rstd, rows, d, branch, branch_scale, sum, bias);
  }
}

// Backward of rms_norm by the chain rule through the two roundings:
//   dn = bf16(dy * scale)                       (cotangent of the bf16 product)
//   dx = r*dn - (r^3/d) * x * sum_j(dn_j x_j)   (fp32), rounded to bf16
//   dx += dresidual (bf16 add), if given
//   partial[block][j] = sum over the block's rows of dy_j * n_j
__global__ void __launch_bounds__(256) rmsnorm_bwd_kernel(const bf16* __restrict__ dy, const bf16* __restrict__ x,
                                                          const bf16* __restrict__ scale,
                                                          const float* __restrict__ rstd,
                                                          const bf16* __restrict__ dres, bf16* __restrict__ dx,
                                                          float* __restrict__ partial, int rows, int d) {
  extern __shared__ float smem[];  // [waves][d]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int chunks = d / 4;
  f32x4 dsc[kMaxChunks];
  bf16x4 sv[kMaxChunks];
#pragma unroll
  for (int t = 0; t < kMaxChunks; ++t) {
    dsc[t] = f32x4{};
    const int c = lane + kWave * t;
    if (c < chunks) sv[t] = *reinterpret_cast<const bf16x4*>(scale + 4 * c);
  }
  for (int row = blockIdx.x * waves + wave; row < rows; row += gridDim.x * waves) {
    const bf16* xr = x + (size_t)row * d;
    const bf16* gr = dy + (size_t)row * d;
    const float r = rstd[row];
    bf16x4 xv[kMaxChunks], gv[kMaxChunks];
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < kMaxChunks; ++t) {
      const int c = lane + kWave * t;
      if (c < chunks) {
        xv[t] = *reinterpret_cast<const bf16x4*>(xr + 4 * c);
        gv[t] = *reinterpret_cast<const bf16x4*>(gr + 4 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) dot += (float)(bf16)((float)gv[t][j] * (float)sv[t][j]) * (float)xv[t][j];
      }
    }
    dot = wave_sum(dot);
    const float coef = r * r * r * dot / (float)d;
    bf16* o = dx + (size_t)row * d;
#pragma unroll
    for (int t = 0; t < kMaxChunks; ++t) {
      const int c = lane + kWave * t;
      if (c < chunks) {
        bf16x4 rv;
        if (dres) rv = *reinterpret_cast<const bf16x4*>(dres + (size_t)row * d + 4 * c);
        bf16x4 ov;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xf = (float)xv[t][j], g = (float)gv[t][j];
          const float dn = (float)(bf16)(g * (float)sv[t][j]);
          float v = (float)(bf16)(r * dn - coef * xf);
          if (dres) v += (float)rv[j];
          ov[j] = (bf16)v;
          dsc[t][j] += g * (float)(bf16)(xf * r);
        }
        *reinterpret_cast<bf16x4*>(o + 4 * c) = ov;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kMaxChunks; ++t) {
    const int c = lane + kWave * t;
    if (c < chunks) *reinterpret_cast<f32x4*>(smem + (size_t)wave * d + 4 * c) = dsc[t];
  }
  __syncthreads();
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    float s = 0.f;
    for (int w = 0; w < waves; ++w) s += smem[(size_t)w * d + j];
    partial[(size_t)blockIdx.x * d + j] = s;
  }
}

// out[j] (+)= sum_p partial[p][j]: 64 columns x 4 part-slices per block, the
// part range split over gridDim.y, one atomic per column per block.
// Row width a multiple of 8 (at most 2048): one wave per row, 16-byte loads
// (lane l holds chunks l, l+64, ... of 8 elements), two rows per iteration so
// the loads of both rows (x, dy and the residual gradient) are in flight
// before either row's reduction.  The three inputs are read once: non-temporal
// loads (about 6% faster at 65536 x 768).
constexpr int kMaxC8 = 4;
template <int C>
__global__ void __launch_bounds__(256) rmsnorm_bwd8_kernel(const bf16* __restrict__ dy, const bf16* __restrict__ x,
                                                           const bf16* __restrict__ scale,
                                                           const float* __restrict__ rstd,
                                                           const bf16* __restrict__ dres, bf16* __restrict__ dx,
                                                           float* __restrict__ partial, int rows, int d) {
  __shared__ float red[4][kMaxC8 * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c8 = d >> 3;
  float dsc[C][8];
  bf16x8 sv[C];
#pragma unroll
  for (int t = 0; t < C; ++t) {
#pragma unroll
    for (int j = 0; j < 8; ++j) dsc[t][j] = 0.f;
    const int c = lane + 64 * t;
    if (c < c8) sv[t] = *reinterpret_cast<const bf16x8*>(scale + 8 * c);
  }
  const int stride = gridDim.x * 4;
  for (int row0 = blockIdx.x * 4 + wave; row0 < rows; row0 += 2 * stride) {
    bf16x8 xv[2][C], gv[2][C], rv[2][C];
    float r[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = row0 + u * stride;
      r[u] = row < rows ? rstd[row] : 0.f;
#pragma unroll
      for (int t = 0; t < C; ++t) {
        const int c = lane + 64 * t;
        if (row < rows && c < c8) {
          const size_t o = (size_t)row * d + 8 * c;
          xv[u][t] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(x + o));
          gv[u][t] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(dy + o));
          if (dres) rv[u][t] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(dres + o));
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = row0 + u * stride;
      if (row >= rows) break;  // uniform across the wave
      float dot = 0.f;
#pragma unroll
      for (int t = 0; t < C; ++t)
        if (lane + 64 * t < c8)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            dot += (float)(bf16)((float)gv[u][t][j] * (float)sv[t][j]) * (float)xv[u][t][j];
      dot = wave_sum(dot);
      const float coef = r[u] * r[u] * r[u] * dot / (float)d;
#pragma unroll
      for (int t = 0; t < C; ++t) {
        const int c = lane + 64 * t;
        if (c < c8) {
          bf16x8 ov;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float xf = (float)xv[u][t][j], g = (float)gv[u][t][j];
            const float dn = (float)(bf16)(g * (float)sv[t][j]);
            float v = (float)(bf16)(r[u] * dn - coef * xf);
            if (dres) v += (float)rv[u][t][j];
            ov[j] = (bf16)v;
            dsc[t][j] += g * (float)(bf16)(xf * r[u]);
          }
          *reinterpret_cast<bf16x8*>(dx + (size_t)row * d + 8 * c) = ov;
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < C; ++t) {
    const int c = lane + 64 * t;
    if (c < c8)
#pragma unroll
      for (int j = 0; j < 8; ++j) red[wave][8 * c + j] = dsc[t][j];
  }
  __syncthreads();
  for (int j = threadIdx.x; j < d; j += blockDim.x)
    partial[(size_t)blockIdx.x * d + j] = red[0][j] + red[1][j] + red[2][j] + red[3][j];
}

// Row width a multiple of 256 (at most 1024): one half-wave per row, lane l
// of the half holding chunks l, l + 32, ... of 8 elements, so every lane
// carries C chunks (with a wave per row, d = 768 left half the lanes idle on
// the second chunk, and the VALU work of that chunk cost a full-width
// instruction).  The two halves of a wave take consecutive rows; per-row sums
// reduce over the 32 lanes of a half.  Same arithmetic and rounding as
// rmsnorm_bwd8_kernel.
template <int C>
__global__ void __launch_bounds__(256) rmsnorm_bwd_hw_kernel(const bf16* __restrict__ dy, const bf16* __restrict__ x,
                                                             const bf16* __restrict__ scale,
                                                             const float* __restrict__ rstd,
                                                             const bf16* __restrict__ dres, bf16* __restrict__ dx,
                                                             float* __restrict__ partial, int rows, int d) {
  __shared__ float red[8][C * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  float dsc[C][8];
  bf16x8 sv[C];
#pragma unroll
  for (int t = 0; t < C; ++t) {
#pragma unroll
    for (int j = 0; j < 8; ++j) dsc[t][j] = 0.f;
    sv[t] = *reinterpret_cast<const bf16x8*>(scale + 8 * (l32 + 32 * t));
  }
  // Row pair p (uniform per wave) covers rows 2p and 2p + 1.
  const int pstride = gridDim.x * 4;
  for (int p = blockIdx.x * 4 + wave; 2 * p < rows; p += pstride) {
    const int row = 2 * p + hl;
    const bool ok = row < rows;
    bf16x8 xv[C], gv[C], rv[C];
    const float r = ok ? rstd[row] : 0.f;
#pragma unroll
    for (int t = 0; t < C; ++t) {
      const size_t o = (size_t)(ok ? row : 0) * d + 8 * (l32 + 32 * t);
      xv[t] = ok ? __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(x + o)) : bf16x8{};
      gv[t] = ok ? __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(dy + o)) : bf16x8{};
      if (dres) rv[t] = ok ? __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(dres + o)) : bf16x8{};
    }
    float dot = 0.f;
#pragma unroll
    for (int t = 0; t < C; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) dot += (float)(bf16)((float)gv[t][j] * (float)sv[t][j]) * (float)xv[t][j];
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
    const float coef = r * r * r * dot / (float)d;
    if (ok) {
#pragma unroll
      for (int t = 0; t < C; ++t) {
        bf16x8 ov;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xf = (float)xv[t][j], g = (float)gv[t][j];
          const float dn = (float)(bf16)(g * (float)sv[t][j]);
          float v = (float)(bf16)(r * dn - coef * xf);
          if (dres) v += (float)rv[t][j];
          ov[j] = (bf16)v;
          dsc[t][j] += g * (float)(bf16)(xf * r);
        }
        *reinterpret_cast<bf16x8*>(dx + (size_t)row * d + 8 * (l32 + 32 * t)) = ov;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < C; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[2 * wave + hl][8 * (l32 + 32 * t) + j] = dsc[t][j];
  __syncthreads();
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    float acc = 0.f;
#pragma unroll
    for (int h = 0; h < 8; ++h) acc += red[h][j];
    partial[(size_t)blockIdx.x * d + j] = acc;
  }
}

__global__ void __launch_bounds__(256) column_sum_kernel(const float* __restrict__ partial, int parts, int d,
                                                         float* __restrict__ out) {
  __shared__ float red[4][64];
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  const int slice = threadIdx.x >> 6;
  const int per = (parts + gridDim.y - 1) / gridDim.y;
  const int p0 = blockIdx.y * per, p1 = min(parts, p0 + per);
  float s = 0.f;
  if (col < d)
    for (int p = p0 + slice; p < p1; p += 4) s += partial[(size_t)p * d + col];
  red[slice][threadIdx.x & 63] = s;
  __syncthreads();
  if (slice == 0 && col < d) atomicAdd(out + col, red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] +
                                                      red[3][threadIdx.x]);
}

// Bias gradient: db[j] += sum_rows dy[row][j] in fp32 (the transpose of the
// broadcast bias add of rig/nn.py:55-56).  8 columns per thread, 64 column
// chunks x 4 row slices per block, rows split over gridDim.y.
__global__ void __launch_bounds__(256) bias_grad_kernel(const bf16* __restrict__ dy, int rows, int cols,
                                                        float* __restrict__ db) {
  __shared__ f32x4 red[4][64][2];
  const int cc = blockIdx.x * 64 + (threadIdx.x & 63);  // 8-column chunk
  const int slice = threadIdx.x >> 6;
  const int per = (rows + gridDim.y - 1) / gridDim.y;
  const int r0 = blockIdx.y * per, r1 = min(rows, r0 + per);
  f32x4 a = f32x4{}, b = f32x4{};
  if (8 * cc < cols) {
#pragma unroll 8
    for (int r = r0 + slice; r < r1; r += 4) {
      bf16x8 v = *reinterpret_cast<const bf16x8*>(dy + (size_t)r * cols + 8 * cc);
      a[0] += (float)v[0]; a[1] += (float)v[1]; a[2] += (float)v[2]; a[3] += (float)v[3];
      b[0] += (float)v[4]; b[1] += (float)v[5]; b[2] += (float)v[6]; b[3] += (float)v[7];
    }
  }
  red[slice][threadIdx.x & 63][0] = a;
  red[slice][threadIdx.x & 63][1] = b;
  __syncthreads();
  if (slice == 0 && 8 * cc < cols) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f32x4 t = red[0][threadIdx.x][h];
#pragma unroll
      for (int s2 = 1; s2 < 4; ++s2) {
        f32x4 u = red[s2][threadIdx.x][h];
        t[0] += u[0]; t[1] += u[1]; t[2] += u[2]; t[3] += u[3];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) atomicAdd(db + 8 * cc + 4 * h + j, t[j]);
    }
  }
}

// ----------------------------------------------------------------------------
// GELU, tanh approximation (jax.nn.gelu(approximate=True), train.py:1171)
// ----------------------------------------------------------------------------
// With a bias (the up-projection's, rig/nn.py:55-56): the GEMM output x gets
// bf16(x + b[column]) first, the rounding of the linear's bias add, and the
// backward recomputes that pre-activation instead of reading it back.
// `cols` (a multiple of 8) is the row width, so an 8-value chunk never
// straddles two rows.
template <bool kBias>
__global__ void bias_gelu_fwd_kernel(const bf16* __restrict__ x, const bf16* __restrict__ bias, bf16* __restrict__ y,
                                     int64_t n, int cols) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;
  bf16x8 v = *reinterpret_cast<const bf16x8*>(x + i);
  if (kBias) {
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(bias + i % cols);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (bf16)((float)v[j] + (float)b[j]);
  }
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = (bf16)gelu_f((float)v[j]);
  *reinterpret_cast<bf16x8*>(y + i) = o;
}

__global__ void bias_gelu_bwd_kernel(const bf16* __restrict__ dy, const bf16* __restrict__ x,
                                     const bf16* __restrict__ bias, bf16* __restrict__ dx, int64_t n, int cols) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;
  bf16x8 v = *reinterpret_cast<const bf16x8*>(x + i);
  const bf16x8 b = *reinterpret_cast<const bf16x8*>(bias + i % cols);
  const bf16x8 g = *reinterpret_cast<const bf16x8*>(dy + i);
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float h = (float)(bf16)((float)v[j] + (float)b[j]);
    o[j] = (bf16)((float)g[j] * gelu_grad_f(h));
  }
  *reinterpret_cast<bf16x8*>(dx + i) = o;
}

__global__ void gelu_fwd_kernel(const bf16* __restrict__ x, bf16* __restrict__ y, int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i + 8 <= n) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(x + i);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (bf16)gelu_f((float)v[j]);
    *reinterpret_cast<bf16x8*>(y + i) = o;
  } else {
    for (; i < n; ++i) y[i] = (bf16)gelu_f((float)x[i]);
  }
}

__global__ void gelu_bwd_kernel(const bf16* __restrict__ dy, const bf16* __restrict__ x, bf16* __restrict__ dx,
                                int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i + 8 <= n) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(x + i);
    bf16x8 g = *reinterpret_cast<const bf16x8*>(dy + i);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (bf16)((float)g[j] * gelu_grad_f((float)v[j]));
    *reinterpret_cast<bf16x8*>(dx + i) = o;
  } else {
    for (; i < n; ++i) dx[i] = (bf16)((float)dy[i] * gelu_grad_f((float)x[i]));
  }
}

// ----------------------------------------------------------------------------
// Interleaved RoPE, base 10000  (rig/nn.py:36-52)
// Table: inv_freq = 10000^(-2i/D), angle = pos*inv_freq (fp32), cos/sin -> bf16.
// In place on rows of a [rows, row_stride] buffer; position = row % seq; the
// first `heads` head-sized column groups of each row are rotated.
// ----------------------------------------------------------------------------
__global__ void rope_table_kernel(bf16* __restrict__ cs, bf16* __restrict__ sn, int seq, int half, int head_dim) {
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= seq * half) return;
  int p = idx / half, i = idx % half;
  float fraction = (float)(2 * i) / (float)head_dim;
  float inv = powf(10000.0f, -fraction);
  float angle = (float)p * inv;
  cs[idx] = (bf16)cosf(angle);
  sn[idx] = (bf16)sinf(angle);
}

// kBias: columns [0, cols) of each row first get bf16(x + bias[column]) (the
// bias add of the linear that produced the rows, rig/nn.py:55-56), and only
// the first heads * head_dim of them are then rotated: the q / k / v rows of
// the fused projection in one pass.  Without it cols = heads * head_dim.
template <bool kBackward, bool kBias = false>
__global__ void rope_kernel(bf16* __restrict__ x, int64_t row_stride, int rows, int seq, int heads, int head_dim,
                            const bf16* __restrict__ cs, const bf16* __restrict__ sn,
                            const bf16* __restrict__ bias = nullptr, int cols = 0) {
  const int half = head_dim / 2;
  const int rotated = heads * head_dim;
  const int chunks_per_row = (kBias ? cols : rotated) / 8;  // 4 pairs (8 values) per thread
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * chunks_per_row) return;
  int row = (int)(t / chunks_per_row);
  const int c0 = 8 * (int)(t % chunks_per_row);  // first column of the chunk
  bf16* p = x + (size_t)row * row_stride + c0;
  bf16x8 v = *reinterpret_cast<bf16x8*>(p);
  if (kBias) {
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(bias + c0);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (bf16)((float)v[j] + (float)b[j]);
    if (c0 >= rotated) {
      *reinterpret_cast<bf16x8*>(p) = v;
      return;
    }
  }
  const int i0 = (c0 % head_dim) / 2;  // pairs are (even, odd) columns of a head
  int pos = row % seq;
  bf16x4 c4 = *reinterpret_cast<const bf16x4*>(cs + (size_t)pos * half + i0);
  bf16x4 s4 = *reinterpret_cast<const bf16x4*>(sn + (size_t)pos * half + i0);
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float s = (float)s4[j];
    if (kBackward) s = -s;
    const bf16x2 r = rope_pair((float)v[2 * j], (float)v[2 * j + 1], (float)c4[j], s);
    o[2 * j] = r[0];
    o[2 * j + 1] = r[1];
  }
  *reinterpret_cast<bf16x8*>(p) = o;
}

// ----------------------------------------------------------------------------
// Embedding gather (train.py:1107) and its transpose (fp32 scatter-add).
// ----------------------------------------------------------------------------
__global__ void embedding_fwd_kernel(const int32_t* __restrict__ tok, const bf16* __restrict__ table,
                                     bf16* __restrict__ out, int n, int d, int vocab) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int chunks = d / 8;
  if (t >= (int64_t)n * chunks) return;
  int row = (int)(t / chunks), c = (int)(t % chunks);
  int id = tok[row];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  *reinterpret_cast<bf16x8*>(out + (size_t)row * d + 8 * c) =
      *reinterpret_cast<const bf16x8*>(table + (size_t)id * d + 8 * c);
}

// One wave per token row; lane l adds elements l, l+64, ...: each atomic
// instruction covers 64 consecutive floats (two 128-byte lines), not 64
// scattered 32-byte strides.
__global__ void __launch_bounds__(256) embedding_bwd_kernel(const int32_t* __restrict__ tok,
                                                            const bf16* __restrict__ dout,
                                                            float* __restrict__ dtable, int n, int d, int vocab) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const int id = tok[row];
  if (id < 0 || id >= vocab) return;
  const int lane = threadIdx.x & 63;
  const bf16* src = dout + (size_t)row * d;
  float* dst = dtable + (size_t)id * d;
  for (int e = lane; e < d; e += 64) atomicAdd(dst + e, (float)src[e]);
}

// ----------------------------------------------------------------------------
// AdamW over a flat fp32 arena (train.py:1386-1445).  Tensors start on
// `chunk`-element boundaries, so every chunk belongs to exactly one tensor;
// chunk_tensor[c] names it and hparams[t] = {lr_mult, eps, decay} where
// eps = adam_eps * eps_horizon * eps_mult and decay = wd * decay_horizon *
// decay_mult (0 when the role is not decayed).  Also emits the block partial of
// sum(g^2) (the pre-clip gradient norm, train.py:1387-1391) and the bf16
// shadow of the updated parameter used by the next step's matmuls.
// ----------------------------------------------------------------------------
__global__ void __launch_bounds__(256) adamw_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v,
                                                    bf16* __restrict__ shadow,
                                                    const int32_t* __restrict__ chunk_tensor,
                                                    const float* __restrict__ hparams, int chunk, float lr,
                                                    float beta1, float beta2, float bc1, float bc2,
                                                    const float* __restrict__ clip_scale,
                                                    float* __restrict__ sq_partial) {
  __shared__ float red[4];
  const int c = blockIdx.x;
  const int t = chunk_tensor[c];
  const float lr_t = lr * hparams[3 * t + 0];
  const float eps = hparams[3 * t + 1];
  const float decay = hparams[3 * t + 2];
  const float clip = clip_scale ? *clip_scale : 1.0f;
  const size_t base = (size_t)c * chunk;
  float sq = 0.f;
  // kAdamUnroll groups of 4 elements per thread and round, every load of the
  // round issued before the first update, so each thread keeps
  // 16 kAdamUnroll loads in flight (the pass is bound by HBM).  The four f32
  // streams are read and written once per step: non-temporal accesses keep
  // them from displacing cached data (about 6% faster than plain ones).
  constexpr int kAdamUnroll = 4;
  for (int i0 = threadIdx.x * 4; i0 < chunk; i0 += kAdamUnroll * blockDim.x * 4) {
    f32x4 gv[kAdamUnroll], pv[kAdamUnroll], mv[kAdamUnroll], vv[kAdamUnroll];
#pragma unroll
    for (int u = 0; u < kAdamUnroll; ++u) {
      const int i = i0 + u * blockDim.x * 4;
      if (i < chunk) {
        const size_t k = base + i;
        gv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g + k));
        pv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + k));
        mv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(m + k));
        vv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(v + k));
      }
    }
#pragma unroll
    for (int u = 0; u < kAdamUnroll; ++u) {
      const int i = i0 + u * blockDim.x * 4;
      if (i >= chunk) break;
      const size_t k = base + i;
      bf16x4 sv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float gr = gv[u][j];
        sq += gr * gr;
        float gj = gr * clip;
        float mj = beta1 * mv[u][j] + (1.0f - beta1) * gj;
        float vj = beta2 * vv[u][j] + (1.0f - beta2) * gj * gj;
        float adam = (mj / bc1) / (sqrtf(vj / bc2) + eps);
        float pj = pv[u][j] - lr_t * (adam + decay * pv[u][j]);
        mv[u][j] = mj;
        vv[u][j] = vj;
        pv[u][j] = pj;
        sv[j] = (bf16)pj;
      }
      __builtin_nontemporal_store(pv[u], reinterpret_cast<f32x4*>(p + k));
      __builtin_nontemporal_store(mv[u], reinterpret_cast<f32x4*>(m + k));
      __builtin_nontemporal_store(vv[u], reinterpret_cast<f32x4*>(v + k));
      if (shadow) *reinterpret_cast<bf16x4*>(shadow + k) = sv;
    }
  }
  if (sq_partial) {
    sq = wave_sum(sq);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = sq;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = 0.f;
      for (int w = 0; w < (int)(blockDim.x / 64); ++w) s += red[w];
      sq_partial[c] = s;
    }
  }
}

__global__ void __launch_bounds__(256) sq_partial_kernel(const float* __restrict__ x, int chunk,
                                                         float* __restrict__ partial) {
  __shared__ float red[4];
  const size_t base = (size_t)blockIdx.x * chunk;
  float sq = 0.f;
  for (int i = threadIdx.x * 4; i < chunk; i += blockDim.x * 4) {
    f32x4 gv = *reinterpret_cast<const f32x4*>(x + base + i);
    sq += gv[0] * gv[0] + gv[1] * gv[1] + gv[2] * gv[2] + gv[3] * gv[3];
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = sq;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < (int)(blockDim.x / 64); ++w) s += red[w];
    partial[blockIdx.x] = s;
  }
}

// Sum the partials in fp64 (one block), write the norm, the clip scale
// min(1, clip/(norm+1e-6)) and, when given, the history row (loss, lr, norm).
__global__ void __launch_bounds__(256) finalize_norm_kernel(const float* __restrict__ partial, int parts,
                                                            float grad_clip, float* __restrict__ norm_out,
                                                            float* __restrict__ clip_out,
                                                            const float* __restrict__ loss, float lr,
                                                            float* __restrict__ history_row) {
  __shared__ double red[256];
  double s = 0.0;
  for (int i = threadIdx.x; i < parts; i += blockDim.x) s += (double)partial[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float norm = (float)sqrt(red[0]);
    if (norm_out) *norm_out = norm;
    if (clip_out) *clip_out = grad_clip > 0.f ? fminf(1.0f, grad_clip / (norm + 1.0e-6f)) : 1.0f;
    if (history_row) {
      history_row[0] = loss ? *loss : 0.f;
      history_row[1] = lr;
      history_row[2] = norm;
    }
  }
}

__global__ void cast_f32_bf16_kernel(const float* __restrict__ x, bf16* __restrict__ y, int64_t n) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n) {
    f32x4 v = *reinterpret_cast<const f32x4*>(x + i);
    bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
    *reinterpret_cast<bf16x4*>(y + i) = o;
  } else {
    for (; i < n; ++i) y[i] = (bf16)x[i];
  }
}

// out += weight * sum(x)  (fp32 atomics, one per block)
__global__ void __launch_bounds__(256) weighted_sum_kernel(const float* __restrict__ x, int64_t n, float weight,
                                                           float* __restrict__ out) {
  __shared__ float red[4];
  float s = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    s += x[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(out, weight * (red[0] + red[1] + red[2] + red[3]));
}

// out[0] += sum(x * mask), out[1] += sum(mask): the masked loss sum and target
// count of eval_step (recipes/reference/train.py:1519-1524), fp32 throughout
// (an infinite loss under a zero mask gives NaN, as x * mask does there).
__global__ void __launch_bounds__(256) masked_sum_kernel(const float* __restrict__ x, const float* __restrict__ mask,
                                                         int64_t n, float* __restrict__ out) {
  __shared__ float red[2][4];
  float s = 0.f, c = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float m = mask[i];
    s += x[i] * m;
    c += m;
  }
  s = wave_sum(s);
  c = wave_sum(c);
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x / 64] = s;
    red[1][threadIdx.x / 64] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    atomicAdd(out, red[0][0] + red[0][1] + red[0][2] + red[0][3]);
    atomicAdd(out + 1, red[1][0] + red[1][1] + red[1][2] + red[1][3]);
  }
}

}  // namespace

// ----------------------------------------------------------------------------
// bf16 transpose, dst[c][r] = src[r][c]: 64 x 64 tiles through LDS (one
// padding column), 16-byte loads along src rows, 2-byte stores along dst rows
// grouped so a wave writes 64 consecutive elements.
// ----------------------------------------------------------------------------
__global__ void __launch_bounds__(256) transpose_bf16_kernel(const bf16* __restrict__ src, bf16* __restrict__ dst,
                                                             int rows, int cols) {
  __shared__ bf16 tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + 256 * i;  // 512 chunks of 8
    const int r = idx >> 3, c8 = (idx & 7) * 8;
    if (r0 + r < rows) {
      if (c0 + c8 + 8 <= cols) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(src + (size_t)(r0 + r) * cols + c0 + c8);
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[r][c8 + j] = v[j];
      } else {
        for (int j = 0; j < 8 && c0 + c8 + j < cols; ++j) tile[r][c8 + j] = src[(size_t)(r0 + r) * cols + c0 + c8 + j];
      }
    }
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6;
  for (int c = w; c < 64; c += 4) {
    if (c0 + c < cols && r0 + lane < rows) dst[(size_t)(c0 + c) * rows + r0 + lane] = tile[lane][c];
  }
}

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

int gptrig_rmsnorm_fwd(const void* x, const void* scale, void* y, float* rstd, int rows, int d, void* stream) {
  if (!x || !scale || !y) return GPTRIG_E_NULL;
  if (rows < 0 || d <= 0 || d % 4) return GPTRIG_E_SHAPE;
  if (d > 4 * 64 * kMaxChunks) return GPTRIG_E_UNSUPPORTED;
  if (rows == 0) return GPTRIG_OK;
  launch_rmsnorm_fwd<false>((const bf16*)x, (const bf16*)scale, (bf16*)y, rstd, rows, d, nullptr, 1.0f, nullptr, nullptr,
                            (hipStream_t)stream);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_add_bias_rmsnorm_fwd(const void* x, const void* branch, const void* branch_bias, float branch_scale,
                                const void* scale, void* sum, void* y, float* rstd, int rows, int d, void* stream) {
  if (!x || !branch || !scale || !sum || !y) return GPTRIG_E_NULL;
  if (rows < 0 || d <= 0 || d % 4) return GPTRIG_E_SHAPE;
  if (d > 4 * 64 * kMaxChunks) return GPTRIG_E_UNSUPPORTED;
  if (y == x || y == sum || y == branch || sum == branch) return GPTRIG_E_SHAPE;
  if ((uintptr_t)branch_bias & 7) return GPTRIG_E_SHAPE;  // 8-byte vector reads
  if (rows == 0) return GPTRIG_OK;
  launch_rmsnorm_fwd<true>((const bf16*)x, (const bf16*)scale, (bf16*)y, rstd, rows, d, (const bf16*)branch,
                           branch_scale, (bf16*)sum, (const bf16*)branch_bias, (hipStream_t)stream);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_add_rmsnorm_fwd(const void* x, const void* branch, float branch_scale, const void* scale, void* sum,
                           void* y, float* rstd, int rows, int d, void* stream) {
  return gptrig_add_bias_rmsnorm_fwd(x, branch, nullptr, branch_scale, scale, sum, y, rstd, rows, d, stream);
}

static int rmsnorm_bwd_blocks(int rows) {
  // Eight rows per workgroup pass (two per wave), at most 1024 workgroups:
  // enough loads in flight to cover HBM latency, and few dscale partials.
  const int b = ceil_div(rows, 8);
  return b < 1 ? 1 : (b > 1024 ? 1024 : b);
}

size_t gptrig_rmsnorm_bwd_workspace_bytes(int rows, int d) {
  return (size_t)rmsnorm_bwd_blocks(rows) * d * sizeof(float);
}

int gptrig_rmsnorm_bwd(const void* dy, const void* x, const void* scale, const float* rstd, const void* dresidual,
                       void* dx, float* dscale, int accumulate_dscale, void* workspace, size_t workspace_bytes,
                       int rows, int d, void* stream) {
  if (!dy || !x || !scale || !rstd || !dx || !dscale || !workspace) return GPTRIG_E_NULL;
  if (rows <= 0 || d <= 0 || d % 4) return GPTRIG_E_SHAPE;
  if (d > 4 * 64 * kMaxChunks) return GPTRIG_E_UNSUPPORTED;
  if (workspace_bytes < gptrig_rmsnorm_bwd_workspace_bytes(rows, d)) return GPTRIG_E_WORKSPACE;
  const int blocks = rmsnorm_bwd_blocks(rows);
  hipStream_t s = (hipStream_t)stream;
  if (!accumulate_dscale) {
    fill_f32_kernel<<<ceil_div(d, 256), 256, 0, s>>>(dscale, d, 0.f);
    GPTRIG_CHECK_LAUNCH();
  }
  const int c8 = ceil_div(d / 8, 64);
  if (d % 256 == 0 && d <= 1024) {
    const int c = d / 256;
#define GPTRIG_RMSHW(C)                                                                                           \
  rmsnorm_bwd_hw_kernel<C><<<blocks, 256, 0, s>>>((const bf16*)dy, (const bf16*)x, (const bf16*)scale, rstd,        \
                                                  (const bf16*)dresidual, (bf16*)dx, (float*)workspace, rows, d)
    if (c == 1) GPTRIG_RMSHW(1);
    else if (c == 2) GPTRIG_RMSHW(2);
    else if (c == 3) GPTRIG_RMSHW(3);
    else GPTRIG_RMSHW(4);
#undef GPTRIG_RMSHW
  } else if (d % 8 == 0 && c8 <= kMaxC8) {
#define GPTRIG_RMS8(C)                                                                                          \
  rmsnorm_bwd8_kernel<C><<<blocks, 256, 0, s>>>((const bf16*)dy, (const bf16*)x, (const bf16*)scale, rstd,        \
                                                (const bf16*)dresidual, (bf16*)dx, (float*)workspace, rows, d)
    if (c8 == 1) GPTRIG_RMS8(1);
    else if (c8 == 2) GPTRIG_RMS8(2);
    else if (c8 == 3) GPTRIG_RMS8(3);
    else GPTRIG_RMS8(4);
#undef GPTRIG_RMS8
  } else
    rmsnorm_bwd_kernel<<<blocks, 256, 4 * d * sizeof(float), s>>>((const bf16*)dy, (const bf16*)x,
                                                                    (const bf16*)scale, rstd,
                                                                    (const bf16*)dresidual, (bf16*)dx,
                                                                    (float*)workspace, rows, d);
  GPTRIG_CHECK_LAUNCH();
  column_sum_kernel<<<dim3(ceil_div(d, 64), 16), 256, 0, s>>>((const float*)workspace, blocks, d, dscale);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_bias_grad(const void* dy, int rows, int cols, float* db, void* stream) {
  if (!dy || !db) return GPTRIG_E_NULL;
  if (rows < 0 || cols <= 0 || cols % 8) return GPTRIG_E_SHAPE;
  if (rows == 0) return GPTRIG_OK;
  const int ysplit = (rows + 127) / 128;
  bias_grad_kernel<<<dim3(ceil_div(cols / 8, 64), ysplit), 256, 0, (hipStream_t)stream>>>((const bf16*)dy, rows,
                                                                                          cols, db);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_transpose_bf16(const void* src, void* dst, int rows, int cols, void* stream) {
  if (!src || !dst) return GPTRIG_E_NULL;
  if (rows <= 0 || cols <= 0 || cols % 8) return GPTRIG_E_SHAPE;
  if (((uintptr_t)src) & 15) return GPTRIG_E_SHAPE;
  transpose_bf16_kernel<<<dim3(ceil_div(cols, 64), ceil_div(rows, 64)), 256, 0, (hipStream_t)stream>>>(
      (const bf16*)src, (bf16*)dst, rows, cols);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_gelu_fwd(const void* x, void* y, int64_t n, void* stream) {
  if (!x || !y) return GPTRIG_E_NULL;
  if (n < 0) return GPTRIG_E_SHAPE;
  if (n == 0) return GPTRIG_OK;
  gelu_fwd_kernel<<<ceil_div(ceil_div(n, 8), 256), 256, 0, (hipStream_t)stream>>>((const bf16*)x, (bf16*)y, n);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_gelu_bwd(const void* dy, const void* x, void* dx, int64_t n, void* stream) {
  if (!dy || !x || !dx) return GPTRIG_E_NULL;
  if (n < 0) return GPTRIG_E_SHAPE;
  if (n == 0) return GPTRIG_OK;
  gelu_bwd_kernel<<<ceil_div(ceil_div(n, 8), 256), 256, 0, (hipStream_t)stream>>>((const bf16*)dy, (const bf16*)x,
                                                                                   (bf16*)dx, n);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_bias_gelu_fwd(const void* x, const void* bias, void* y, int rows, int cols, void* stream) {
  if (!x || !bias || !y) return GPTRIG_E_NULL;
  if (rows < 0 || cols <= 0 || cols % 8) return GPTRIG_E_SHAPE;
  if (((uintptr_t)x | (uintptr_t)bias | (uintptr_t)y) & 15) return GPTRIG_E_SHAPE;  // 16-byte vector accesses
  if (rows == 0) return GPTRIG_OK;
  const int64_t n = (int64_t)rows * cols;
  bias_gelu_fwd_kernel<true><<<ceil_div(n / 8, 256), 256, 0, (hipStream_t)stream>>>(
      (const bf16*)x, (const bf16*)bias, (bf16*)y, n, cols);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_bias_gelu_bwd(const void* dy, const void* x, const void* bias, void* dx, int rows, int cols,
                         void* stream) {
  if (!dy || !x || !bias || !dx) return GPTRIG_E_NULL;
  if (rows < 0 || cols <= 0 || cols % 8) return GPTRIG_E_SHAPE;
  if (((uintptr_t)dy | (uintptr_t)x | (uintptr_t)bias | (uintptr_t)dx) & 15) return GPTRIG_E_SHAPE;
  if (rows == 0) return GPTRIG_OK;
  const int64_t n = (int64_t)rows * cols;
  bias_gelu_bwd_kernel<<<ceil_div(n / 8, 256), 256, 0, (hipStream_t)stream>>>(
      (const bf16*)dy, (const bf16*)x, (const bf16*)bias, (bf16*)dx, n, cols);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_rope_table(void* cos_table, void* sin_table, int seq, int head_dim, void* stream) {
  if (!cos_table || !sin_table) return GPTRIG_E_NULL;
  if (seq <= 0 || head_dim <= 0 || (head_dim & 1)) return GPTRIG_E_SHAPE;
  int half = head_dim / 2;
  rope_table_kernel<<<ceil_div((long long)seq * half, 256), 256, 0, (hipStream_t)stream>>>(
      (bf16*)cos_table, (bf16*)sin_table, seq, half, head_dim);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

static int rope_launch(bool backward, void* x, int64_t row_stride, int rows, int seq, int heads, int head_dim,
                       const void* cs, const void* sn, void* stream) {
  if (!x || !cs || !sn) return GPTRIG_E_NULL;
  if (rows < 0 || seq <= 0 || heads <= 0 || head_dim <= 0) return GPTRIG_E_SHAPE;
  if (head_dim % 8 || row_stride % 8 || row_stride < (int64_t)heads * head_dim) return GPTRIG_E_SHAPE;
  if (rows == 0) return GPTRIG_OK;
  long long threads = (long long)rows * heads * (head_dim / 2) / 4;
  if (backward)
    rope_kernel<true><<<ceil_div(threads, 256), 256, 0, (hipStream_t)stream>>>(
        (bf16*)x, row_stride, rows, seq, heads, head_dim, (const bf16*)cs, (const bf16*)sn);
  else
    rope_kernel<false><<<ceil_div(threads, 256), 256, 0, (hipStream_t)stream>>>(
        (bf16*)x, row_stride, rows, seq, heads, head_dim, (const bf16*)cs, (const bf16*)sn);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_rope_fwd(void* x, int64_t row_stride, int rows, int seq, int heads, int head_dim, const void* cos_table,
                    const void* sin_table, void* stream) {
  return rope_launch(false, x, row_stride, rows, seq, heads, head_dim, cos_table, sin_table, stream);
}

int gptrig_bias_rope_fwd(void* x, int64_t row_stride, int rows, int cols, const void* bias, int seq, int heads,
                         int head_dim, const void* cos_table, const void* sin_table, void* stream) {
  if (!x || !bias || !cos_table || !sin_table) return GPTRIG_E_NULL;
  if (rows < 0 || seq <= 0 || heads <= 0 || head_dim <= 0) return GPTRIG_E_SHAPE;
  if (head_dim % 8 || cols % 8 || row_stride % 8 || cols < heads * head_dim || row_stride < cols)
    return GPTRIG_E_SHAPE;
  if (((uintptr_t)x | (uintptr_t)bias) & 15) return GPTRIG_E_SHAPE;  // 16-byte vector accesses
  if (rows == 0) return GPTRIG_OK;
  const long long threads = (long long)rows * (cols / 8);
  rope_kernel<false, true><<<ceil_div(threads, 256), 256, 0, (hipStream_t)stream>>>(
      (bf16*)x, row_stride, rows, seq, heads, head_dim, (const bf16*)cos_table, (const bf16*)sin_table,
      (const bf16*)bias, cols);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_rope_bwd(void* dx, int64_t row_stride, int rows, int seq, int heads, int head_dim,
                    const void* cos_table, const void* sin_table, void* stream) {
  return rope_launch(true, dx, row_stride, rows, seq, heads, head_dim, cos_table, sin_table, stream);
}

int gptrig_embedding_fwd(const int32_t* tokens, const void* table, void* out, int n, int d, int vocab,
                         void* stream) {
  if (!tokens || !table || !out) return GPTRIG_E_NULL;
  if (n < 0 || d <= 0 || d % 8 || vocab <= 0) return GPTRIG_E_SHAPE;
  if (n == 0) return GPTRIG_OK;
  embedding_fwd_kernel<<<ceil_div((long long)n * (d / 8), 256), 256, 0, (hipStream_t)stream>>>(
      tokens, (const bf16*)table, (bf16*)out, n, d, vocab);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_embedding_bwd(const int32_t* tokens, const void* dout, float* dtable, int n, int d, int vocab,
                         void* stream) {
  if (!tokens || !dout || !dtable) return GPTRIG_E_NULL;
  if (n < 0 || d <= 0 || d % 8 || vocab <= 0) return GPTRIG_E_SHAPE;
  if (n == 0) return GPTRIG_OK;
  embedding_bwd_kernel<<<ceil_div(n, 4), 256, 0, (hipStream_t)stream>>>(tokens, (const bf16*)dout, dtable, n, d,
                                                                        vocab);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_adamw(float* param, const float* grad, float* m, float* v, void* param_bf16, const int32_t* chunk_tensor,
                 const float* tensor_hparams, int64_t n_chunks, int chunk, float lr, float beta1, float beta2,
                 int step, const float* clip_scale, float* sq_partials, void* stream) {
  if (!param || !grad || !m || !v || !chunk_tensor || !tensor_hparams) return GPTRIG_E_NULL;
  if (n_chunks < 0 || chunk <= 0 || chunk % 1024 || step <= 0) return GPTRIG_E_SHAPE;
  if (n_chunks == 0) return GPTRIG_OK;
  // The reference divides by float32 bias corrections 1 - beta^step.
  float bc1 = 1.0f - powf(beta1, (float)step);
  float bc2 = 1.0f - powf(beta2, (float)step);
  adamw_kernel<<<(unsigned)n_chunks, 256, 0, (hipStream_t)stream>>>(param, grad, m, v, (bf16*)param_bf16,
                                                                      chunk_tensor, tensor_hparams, chunk, lr, beta1,
                                                                      beta2, bc1, bc2, clip_scale,
                                                                      sq_partials);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_sq_norm_partials(const float* x, int64_t n_chunks, int chunk, float* partials, void* stream) {
  if (!x || !partials) return GPTRIG_E_NULL;
  if (n_chunks < 0 || chunk <= 0 || chunk % 1024) return GPTRIG_E_SHAPE;
  if (n_chunks == 0) return GPTRIG_OK;
  sq_partial_kernel<<<(unsigned)n_chunks, 256, 0, (hipStream_t)stream>>>(x, chunk, partials);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_finalize_norm(const float* partials, int parts, float grad_clip, float* norm_out, float* clip_out,
                         const float* loss, float lr, float* history_row, void* stream) {
  if (!partials) return GPTRIG_E_NULL;
  if (parts <= 0) return GPTRIG_E_SHAPE;
  finalize_norm_kernel<<<1, 256, 0, (hipStream_t)stream>>>(partials, parts, grad_clip, norm_out, clip_out, loss, lr,
                                                          history_row);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_cast_f32_bf16(const float* x, void* y, int64_t n, void* stream) {
  if (!x || !y) return GPTRIG_E_NULL;
  if (n < 0) return GPTRIG_E_SHAPE;
  if (n == 0) return GPTRIG_OK;
  cast_f32_bf16_kernel<<<ceil_div(ceil_div(n, 4), 256), 256, 0, (hipStream_t)stream>>>(x, (bf16*)y, n);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_weighted_sum(const float* x, int64_t n, float weight, float* out, void* stream) {
  if (!x || !out) return GPTRIG_E_NULL;
  if (n <= 0) return GPTRIG_E_SHAPE;
  int blocks = ceil_div(n, 256);
  if (blocks > 1024) blocks = 1024;
  weighted_sum_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(x, n, weight, out);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_masked_sum(const float* x, const float* mask, int64_t n, float* out, void* stream) {
  if (!x || !mask || !out) return GPTRIG_E_NULL;
  if (n <= 0) return GPTRIG_E_SHAPE;
  int blocks = ceil_div(n, 256);
  if (blocks > 1024) blocks = 1024;
  masked_sum_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(x, mask, n, out);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

int gptrig_fill_f32(float* x, int64_t n, float value, void* stream) {
  if (!x) return GPTRIG_E_NULL;
  if (n < 0) return GPTRIG_E_SHAPE;
  if (n == 0) return GPTRIG_OK;
  fill_f32_kernel<<<ceil_div(n, 256), 256, 0, (hipStream_t)stream>>>(x, n, value);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // extern "C"
