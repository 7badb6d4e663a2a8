// Causal flash attention for gfx950: bf16 MFMA (v_mfma_f32_32x32x16_bf16),
// fp32 online softmax in the exp2 domain, LDS-staged K/V tiles.
//
// Semantics follow rig/kernels/tpu_flash_attention.py:
//   forward  (:236-348)  O = softmax(scale*QK^T masked) V, LSE = log sum exp
//   dQ       (:479-575)  dQ = (P o (dO V^T - Delta)) * scale  K
//   dK/dV    (:578-701)  dV = P^T dO,  dK = dS^T Q
// with P recomputed from the saved LSE, Delta = rowsum(O o dO), and the
// probability / dS operands rounded to bf16 before their products.
//
// Forward mapping: a workgroup owns 128 queries (4 waves x 32).  Each wave
// computes S^T = K Q^T so that MFMA lane l holds query l%32 and 16 keys: the
// row max/sum are lane-local (+ one xor-32 exchange) and P^T is already the
// B operand of O^T = V^T P^T, so probabilities never leave registers.
//
// Backward mapping (KV-owned): a workgroup owns a block of keys and walks
// the causal query blocks (64 queries per step).  Each wave computes S = Q K^T
// and dP = dO V^T with lane l holding key l%32, accumulates dV^T += dO^T P and
// dK^T += Q^T dS in registers, and publishes bf16 dS to LDS; dQ = dS K over
// the workgroup's keys is added to an fp32 accumulator with atomics, and a
// last pass rounds dQ to bf16.  head_dim 64: 256 keys as 8 waves x 32 (two
// waves per SIMD).  head_dim 128: 128 keys as 4 waves x 32 (one wave per
// SIMD), double-buffered query blocks and dS^T with the previous block's dQ
// computed after the current block's scores.
#include "attn64.h"

#include <type_traits>

namespace {

constexpr int kBlockM = 128;  // forward: queries per workgroup
constexpr int kBlockN = 64;   // forward: keys per LDS tile
constexpr int kBwd64Threads = 512;  // backward (head_dim 64): 8 waves of 32 keys
constexpr int kBwd64Keys = 256;     // backward (head_dim 64): keys per workgroup
constexpr int kBwdM = 64;     // backward: queries per step
constexpr float kMinusBig = -1.0e30f;

struct View {
  const bf16* p;
  int64_t sb, sh, ss;
  __device__ __forceinline__ const bf16* row(int b, int h, int s) const { return p + b * sb + h * sh + s * ss; }
};
struct MutView {
  bf16* p;
  int64_t sb, sh, ss;
  __device__ __forceinline__ bf16* row(int b, int h, int s) const { return p + b * sb + h * sh + s * ss; }
};

// Workgroup id -> (batch*head, block rank), rank-major: every head's rank-0
// block (its heaviest causal share, see the callers) is dispatched before any
// rank-1 block, and so on, so the last workgroups to start are the light ones
// and the tail stays short.  Workgroups are dispatched round-robin over the 8
// XCDs; with batch*heads a multiple of 8 all blocks of one head land on the
// same XCD, which keeps that head's K/V (forward) or Q/dO/dQ (backward) in one
// L2.
__device__ __forceinline__ void xcd_map(int id, int nblocks, int bh_total, int& bh, int& blk) {
  (void)nblocks;
  bh = id % bh_total;
  blk = id / bh_total;
}

// ============================================================================
// Backward passes around the main kernels: Delta (and the dQ accumulator
// zeroed) before, the dQ conversion to bf16 after
// ============================================================================
template <int D>
__global__ void attn_bwd_pre_kernel(View O, View dO, float* __restrict__ delta, float* __restrict__ dq_acc, int B,
                                    int H, int S) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = t >> 3;
  const int part = t & 7;
  if (row >= (int64_t)B * H * S) return;
  const int s = (int)(row % S);
  const int bh = (int)(row / S);
  const int b = bh / H, h = bh % H;
  const bf16* o = O.row(b, h, s);
  const bf16* g = dO.row(b, h, s);
  float acc = 0.f;
#pragma unroll
  for (int c = part; c < D / 8; c += 8) {
    bf16x8 ov = *reinterpret_cast<const bf16x8*>(o + 8 * c);
    bf16x8 gv = *reinterpret_cast<const bf16x8*>(g + 8 * c);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += (float)ov[j] * (float)gv[j];
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  if (part == 0) delta[row] = acc;
  float* dq = dq_acc + row * D;
#pragma unroll
  for (int c = part; c < D / 4; c += 8) *reinterpret_cast<f32x4*>(dq + 4 * c) = f32x4{};
}

template <int D>
// rcs / rsn (nullable): RoPE tables [S][D/2]; when given, the bf16 dQ is
// passed back through the transposed rotation (the RoPE VJP) before the store.
__global__ void attn_dq_convert_kernel(const float* __restrict__ dq_acc, MutView dQ, int B, int H, int S,
                                       const bf16* __restrict__ rcs, const bf16* __restrict__ rsn) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = t / (D / 8);
  const int c = (int)(t % (D / 8));
  if (row >= (int64_t)B * H * S) return;
  const int s = (int)(row % S);
  const int bh = (int)(row / S);
  const float* src = dq_acc + row * D + 8 * c;
  f32x4 a = *reinterpret_cast<const f32x4*>(src);
  f32x4 bb = *reinterpret_cast<const f32x4*>(src + 4);
  bf16x8 o = {(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3], (bf16)bb[0], (bf16)bb[1], (bf16)bb[2], (bf16)bb[3]};
  if (rcs) {
    const bf16x4 c4 = *reinterpret_cast<const bf16x4*>(rcs + (size_t)s * (D / 2) + 4 * c);
    const bf16x4 s4 = *reinterpret_cast<const bf16x4*>(rsn + (size_t)s * (D / 2) + 4 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 r = rope_pair((float)o[2 * j], (float)o[2 * j + 1], (float)c4[j], -(float)s4[j]);
      o[2 * j] = r[0];
      o[2 * j + 1] = r[1];
    }
  }
  *reinterpret_cast<bf16x8*>(dQ.row(bh / H, bh % H, s) + 8 * c) = o;
}

// ============================================================================
// Kernels on swizzled row-major LDS tiles (attn64.h)
// ============================================================================

typedef __attribute__((address_space(3))) void lds_void;

// Forward (head_dim 64 and 128): K/V tiles of 64 keys are copied global ->
// LDS by the DMA path (buffer_load_dwordx4 ... lds) into double-buffered
// swizzled tiles, one LDS array per buffer and operand so the compiler can see
// that the copy into one buffer never aliases reads of the other; V^T
// operands come from transposed reads with the accumulator's row order.  A
// head_dim-128 tile is kept as two 64-wide swizzled tiles (d 0..63, then d
// 64..127) so the same swizzle and reads serve it.  A tile is consumed in two
// halves of 32 keys (online softmax per half): at head_dim 64 that keeps the
// wave under 128 VGPRs (four waves per SIMD hide the LDS and exp latencies),
// at head_dim 128 (twice the O accumulator and Q operands) two workgroups
// share a CU.
template <int D, bool kSeg>
__device__ __forceinline__ void attn_fwd_swz(View Q, View K, View V, MutView O, float* __restrict__ lse,
                                             const int32_t* __restrict__ seg, int B, int H, int S, float scale_log2) {
  constexpr int KC = D / 16, DB = D / 32;
  // Element offset of 16-byte chunk c16 of tile row `row` (64 rows per tile).
  auto tofs = [](int row, int c16) { return (c16 >> 3) * 64 * 64 + at64::swz(row, c16 & 7); };
  __shared__ __attribute__((aligned(16))) bf16 fk0[64 * D];
  __shared__ __attribute__((aligned(16))) bf16 fk1[64 * D];
  __shared__ __attribute__((aligned(16))) bf16 fv0[64 * D];
  __shared__ __attribute__((aligned(16))) bf16 fv1[64 * D];

  const int nq = (S + kBlockM - 1) / kBlockM;
  int bh, qb;
  xcd_map(blockIdx.x, nq, B * H, bh, qb);
  qb = nq - 1 - qb;
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63;
  // Scalar, so the per-wave mask decisions below are uniform branches.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, l32 = lane & 31;
  const int q0 = qb * kBlockM;
  const int qw0 = q0 + wave * 32;
  const int my_q = qw0 + l32;
  const int last_q = min(q0 + kBlockM, S) - 1;
  const int ntiles = last_q / kBlockN + 1;

  bf16x8 qreg[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
    qreg[kc] = my_q < S ? *reinterpret_cast<const bf16x8*>(Q.row(b, h, my_q) + 16 * kc + 8 * hl) : bf16x8{};
  const int seg_q = (kSeg && my_q < S) ? seg[(size_t)b * S + my_q] : 0;

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  float m_run = kMinusBig, l_run = 0.f;

  // Wave w fills 1 KB blocks 2w, 2w+1 (8 rows each) of the K and V tiles
  // through buffer resources of this (b, h): 32-bit per-lane offsets, and
  // rows at or past S read as zeros.
  const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(K.row(b, h, 0), (uint32_t)(S * K.ss * 2));
  const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(V.row(b, h, 0), (uint32_t)(S * V.ss * 2));
  // Wave w fills 1 KB blocks NBW*w .. NBW*w + NBW-1 of each tile: block blk
  // holds rows 8*(blk % 8) .. +7 of the 64-wide tile blk / 8.
  constexpr int NBW = D / 32;
  const int kss2 = (int)K.ss * 2, vss2 = (int)V.ss * 2;
  int koff[NBW], voff[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int blk = NBW * wave + j;
    const int row = 8 * (blk & 7) + (lane >> 3);
    const int t = (row >> 1) & 7;
    const int c = 8 * (blk >> 3) + ((lane & 7) ^ (((t & 1) << 2) | (t >> 1)));
    koff[j] = row * kss2 + 16 * c;
    voff[j] = row * vss2 + 16 * c;
  }
  auto fill = [&](at64::lds_t* kt, at64::lds_t* vt, int kv0) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int blk = NBW * wave + j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(k_rs, (lds_void*)(kt + blk * 512), 16, koff[j] + kv0 * kss2, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(v_rs, (lds_void*)(vt + blk * 512), 16, voff[j] + kv0 * vss2, 0, 0, 0);
    }
  };

  // One 32-key half of a tile in buffer (kt, vt).
  auto half = [&](const at64::lds_t* kt, const at64::lds_t* vt, int kv0, int sb) __attribute__((always_inline)) {
    f32x16 s = f32x16{};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      s = mfma32(*(const at64::lds_x8*)(kt + tofs(32 * sb + l32, 2 * kc + hl)), qreg[kc], s);
    // Row max on raw scores (scale > 0); masked scores become -inf.
    const int kh0 = kv0 + 32 * sb;
    float mraw = -INFINITY;
    if constexpr (kSeg) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kh0 + 8 * (i >> 2) + 4 * hl + (i & 3);
        bool vis = key <= my_q && key < S;
        if (vis) vis = seg[(size_t)b * S + key] == seg_q;
        s[i] = vis ? s[i] : -INFINITY;
        mraw = fmaxf(mraw, s[i]);
      }
    } else {
      // One uniform branch per half: element i holds key kh0 + 4hl + c_i,
      // c_i = 8 (i / 4) + i % 4, visible while c_i <= min(my_q, S - 1) - kh0 - 4hl.
      if ((kh0 + 31 > qw0) || (kh0 + 32 > S)) {
        const int lim = min(my_q, S - 1) - kh0 - 4 * hl;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 8 * (i >> 2) + (i & 3) <= lim ? s[i] : -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) mraw = fmaxf(mraw, s[i]);
    }
    mraw = fmaxf(mraw, __shfl_xor(mraw, 32));
    // Lazy rescaling: the running max (log2 units) only moves when a row's
    // max exceeds it by more than 8, so probabilities stay <= 2^8 and the
    // accumulator rescale is skipped on most halves.  O = acc / l and
    // lse = m + log2(l) hold for any consistent m.
    const float m_tile = mraw * scale_log2;
    const bool grow = m_tile > m_run + 8.0f;
    const float m_new = grow ? m_tile : m_run;
    if (__builtin_amdgcn_read_exec() & __ballot(grow)) {
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[db][i] *= alpha;
    }
    m_run = m_new;
    float lsum = 0.f;
    bf16x8 pb[2];
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = fast_exp2(fmaf(s[8 * c2 + j], scale_log2, -m_new));
        lsum += p;
        pb[c2][j] = (bf16)p;
      }
    l_run += lsum;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
      for (int db = 0; db < DB; ++db)
        acc[db] = mfma32(at64::trfrag<true>(vt + (db >> 1) * 64 * 64, 32 * (db & 1), 16 * (2 * sb + c2), lane),
                         pb[c2], acc[db]);
  };

  auto tile = [&](const at64::lds_t* kt, const at64::lds_t* vt, at64::lds_t* nkt, at64::lds_t* nvt, int it) {
    const int kv0 = it * kBlockN;
    if (it + 1 < ntiles) fill(nkt, nvt, kv0 + kBlockN);
    // Halves whose every key lies past the wave's last query add nothing.
    if (kv0 <= qw0 + 31) half(kt, vt, kv0, 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the halves' live ranges apart
    if (kv0 + 32 <= qw0 + 31) half(kt, vt, kv0, 1);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the next tile has landed
    __syncthreads();
  };

  at64::lds_t* const k0s = gemm::lds_cast(fk0);
  at64::lds_t* const k1s = gemm::lds_cast(fk1);
  at64::lds_t* const v0s = gemm::lds_cast(fv0);
  at64::lds_t* const v1s = gemm::lds_cast(fv1);
  fill(k0s, v0s, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  for (int it = 0; it < ntiles; it += 2) {
    tile(k0s, v0s, k1s, v1s, it);
    if (it + 1 < ntiles) tile(k1s, v1s, k0s, v0s, it + 1);
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (my_q < S) {
    const float inv = 1.0f / l_tot;
    bf16* orow = O.row(b, h, my_q);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bf16x4 o4;
#pragma unroll
        for (int t = 0; t < 4; ++t) o4[t] = (bf16)(acc[db][4 * r + t] * inv);
        *reinterpret_cast<bf16x4*>(orow + 32 * db + 8 * r + 4 * hl) = o4;
      }
    if (hl == 0) lse[((size_t)b * H + h) * S + my_q] = (m_run + __log2f(l_tot)) * GPTRIG_LN2;
  }
}

template <bool kSeg>
__global__ void __launch_bounds__(256, 4)
    attn_fwd64_kernel(View Q, View K, View V, MutView O, float* __restrict__ lse, const int32_t* __restrict__ seg,
                      int B, int H, int S, float scale_log2) {
  attn_fwd_swz<64, kSeg>(Q, K, V, O, lse, seg, B, H, S, scale_log2);
}

template <bool kSeg>
__global__ void __launch_bounds__(256, 2)
    attn_fwd128_kernel(View Q, View K, View V, MutView O, float* __restrict__ lse, const int32_t* __restrict__ seg,
                       int B, int H, int S, float scale_log2) {
  attn_fwd_swz<128, kSeg>(Q, K, V, O, lse, seg, B, H, S, scale_log2);
}

// Backward: KV-owned, 256 keys per workgroup (32 per wave), 64 queries per
// step.  Q/dO/K/V tiles are swizzled row-major; Q^T, dO^T, K^T and dS come
// from transposed reads, so nothing is written to LDS transposed.  dS is
// stored as dS^T [key][query] (8-byte writes) and dQ = dS K is added to an
// fp32 accumulator with buffer atomics.  The loop body keeps no spills: a
// scratch reload would make the compiler wait for every outstanding vector
// memory operation, the previous step's dQ atomics included.
template <bool kSeg>
__global__ void __launch_bounds__(kBwd64Threads, 2)
    attn_bwd64_kernel(View Q, View K, View V, View dO, const float* __restrict__ lse,
                      const float* __restrict__ delta, const int32_t* __restrict__ seg, float* __restrict__ dq_acc,
                      MutView dK, MutView dV, int B, int H, int S, float scale, float scale_log2,
                      const bf16* __restrict__ rcs, const bf16* __restrict__ rsn) {
  constexpr int D = 64, KC = 4, DB = 2, NT = kBwd64Threads, NK = kBwd64Keys;
  __shared__ __attribute__((aligned(16))) bf16 smem[(64 + 64 + 3 * NK) * 64];
  __shared__ __attribute__((aligned(16))) float lse_s[kBwdM], delta_s[kBwdM];
  __shared__ int seg_s[kBwdM];
  // RoPE tables (cos, sin) of the workgroup's keys, read by the dK epilogue
  // when the RoPE VJP is fused; staged here so their loads overlap the loop.
  __shared__ __attribute__((aligned(16))) bf16 rope_s[2][NK * (D / 2)];
  at64::lds_t* const Qs = gemm::lds_cast(smem);
  at64::lds_t* const dOs = Qs + 64 * 64;
  at64::lds_t* const Ks = dOs + 64 * 64;
  at64::lds_t* const dSt = Ks + NK * 64;
  at64::lds_t* const Vs = dSt + NK * 64;

  const int nkv = (S + NK - 1) / NK;
  int bh, kb;
  xcd_map(blockIdx.x, nkv, B * H, bh, kb);
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int k0 = kb * NK;
  const int kw0 = k0 + 32 * wave;
  const int my_k = kw0 + l32;
  const bool k_ok = my_k < S;

  const int seg_k = (kSeg && k_ok) ? seg[(size_t)b * S + my_k] : 0;

  {
    // (Branch-free, so these loads issue together with the K / V loads below.)
    constexpr int kChunks = NK * (D / 2) / 8;  // 16-byte chunks per table
#pragma unroll
    for (int r = 0; r < kChunks / NT; ++r) {
      const int idx = tid + NT * r;
      const int key = idx / (D / 16), c = idx % (D / 16);
      const bool ok = rcs != nullptr && k0 + key < S;
      const size_t off = ok ? (size_t)(k0 + key) * (D / 2) + 8 * c : 0;
      *reinterpret_cast<bf16x8*>(&rope_s[0][8 * idx]) = ok ? *reinterpret_cast<const bf16x8*>(rcs + off) : bf16x8{};
      *reinterpret_cast<bf16x8*>(&rope_s[1][8 * idx]) = ok ? *reinterpret_cast<const bf16x8*>(rsn + off) : bf16x8{};
    }
  }
  // K and V tiles of the workgroup's keys (row-major, swizzled).  K feeds
  // dQ = dS K (transposed reads) and, like V, the per-key MFMA operands of
  // S = Q K^T and dP = dO V^T, which are re-read from LDS every step rather
  // than held in 32 registers for the whole loop.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int idx = tid + NT * r;
    const int row = idx >> 3, c = idx & 7;
    const bool ok = k0 + row < S;
    const bf16x8 kv = ok ? *reinterpret_cast<const bf16x8*>(K.row(b, h, k0 + row) + 8 * c) : bf16x8{};
    const bf16x8 vv = ok ? *reinterpret_cast<const bf16x8*>(V.row(b, h, k0 + row) + 8 * c) : bf16x8{};
    *(at64::lds_x8*)(Ks + at64::swz(row, c)) = kv;
    *(at64::lds_x8*)(Vs + at64::swz(row, c)) = vv;
  }

  f32x16 dv_acc[DB], dk_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dv_acc[db] = f32x16{};
    dk_acc[db] = f32x16{};
  }
  // Per-(b, h) buffer resources: scalar bases, 32-bit per-lane offsets, and
  // zeros / dropped writes past the end of the sequence instead of branches.
  const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(Q.row(b, h, 0), (uint32_t)(S * Q.ss * 2));
  const __amdgpu_buffer_rsrc_t g_rs = make_rsrc(dO.row(b, h, 0), (uint32_t)(S * dO.ss * 2));
  const __amdgpu_buffer_rsrc_t lse_rs = make_rsrc(lse + (size_t)bh * S, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t delta_rs = make_rsrc(delta + (size_t)bh * S, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t seg_rs =
      make_rsrc(kSeg ? (const void*)(seg + (size_t)b * S) : (const void*)lse, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t dq_rs = make_rsrc(dq_acc + (size_t)bh * S * D, (uint32_t)S * D * 4u);

  // Register staging of one 64-query block: 16 B of Q and of dO per thread and step.
  constexpr int QR = 64 * 8 / NT;
  bf16x8 qst[QR], gst[QR];
  float lse_st = 0.f, delta_st = 0.f;
  int seg_st = 0;
  auto load_q = [&](int qq0) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int idx = tid + NT * r;
      const int qi = idx >> 3, c = idx & 7;
      qst[r] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                              q_rs, ((qq0 + qi) * (int)Q.ss + 8 * c) * 2, 0, 0));
      gst[r] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                              g_rs, ((qq0 + qi) * (int)dO.ss + 8 * c) * 2, 0, 0));
    }
    if (tid < kBwdM) {
      lse_st = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lse_rs, (qq0 + tid) * 4, 0, 0));
      delta_st = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(delta_rs, (qq0 + tid) * 4, 0, 0));
      if (kSeg) seg_st = (int)__builtin_amdgcn_raw_buffer_load_b32(seg_rs, (qq0 + tid) * 4, 0, 0);
    }
  };
  auto store_q = [&]() {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int idx = tid + NT * r;
      const int qi = idx >> 3, c = idx & 7;
      *(at64::lds_x8*)(Qs + at64::swz(qi, c)) = qst[r];
      *(at64::lds_x8*)(dOs + at64::swz(qi, c)) = gst[r];
    }
    if (tid < kBwdM) {
      // Scaled here, after (B), so the loads are not waited for at issue.
      lse_s[tid] = lse_st * GPTRIG_LOG2E;
      delta_s[tid] = delta_st * scale;  // dS = P * (scale*dP - scale*Delta)
      if (kSeg) seg_s[tid] = seg_st;
    }
  };

  const int qb_first = k0 / kBwdM;
  const int nqb = (S + kBwdM - 1) / kBwdM;
  load_q(qb_first * kBwdM);
  store_q();

  for (int qb = qb_first; qb < nqb; ++qb) {
    const int qq0 = qb * kBwdM;
    // (A) Q, dO, lse, delta of this block published.  Only LDS has to be
    // complete here: the previous block's dQ atomics stay in flight.
    GPTRIG_WAIT_LGKM0();
    wg_barrier();
    // Prefetch the next block into registers; it is written to LDS after (B),
    // once every wave is done with this block's Q / dO, ahead of the dQ
    // atomics (so that wait never drains them).
    // (The last block re-loads itself: the same code on every iteration.)
    load_q(qb + 1 < nqb ? qq0 + kBwdM : qq0);

    const bool wave_active = kw0 <= qq0 + kBwdM - 1 && kw0 < S;
    // One 32-query half of the block.  kMask: the causal / ragged / segment
    // mask is evaluated per element (diagonal and edge blocks only); the
    // interior blocks run a mask-free copy of the same code.
    auto qs_body = [&](int qs, auto mask_tag) {
      constexpr bool kMask = decltype(mask_tag)::value;
      bf16x8 qf[KC], gf[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        qf[kc] = at64::rowfrag(Qs, 32 * qs + l32, 2 * kc + hl);
        gf[kc] = at64::rowfrag(dOs, 32 * qs + l32, 2 * kc + hl);
      }
      f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        sacc = mfma32(qf[kc], at64::rowfrag(Ks, 32 * wave + l32, 2 * kc + hl), sacc);
        pacc = mfma32(gf[kc], at64::rowfrag(Vs, 32 * wave + l32, 2 * kc + hl), pacc);
      }
      bf16x8 pb[2], db8[2];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qr = 32 * qs + 8 * r + 4 * hl;
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&lse_s[qr]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&delta_s[qr]);
        bf16x4 ds4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int i = 4 * r + t;
          float p = fast_exp2(fmaf(sacc[i], scale_log2, -l4[t]));
          if (kMask) {
            const int q = qq0 + qr + t;
            bool vis = my_k <= q && q < S && k_ok;
            if (kSeg && vis) vis = seg_s[qr + t] == seg_k;
            p = vis ? p : 0.f;
          }
          const float ds = p * fmaf(pacc[i], scale, -d4[t]);
          pb[i >> 3][i & 7] = (bf16)p;
          const bf16 dsb = (bf16)ds;
          db8[i >> 3][i & 7] = dsb;
          ds4[t] = dsb;
        }
        // dS^T row = this lane's key, queries 32qs + 8r + 4hl .. +3.
        *(__attribute__((address_space(3))) bf16x4*)(dSt + at64::swz(32 * wave + l32, 4 * qs + r) + 4 * hl) = ds4;
      }
      bf16x8 gt[DB][2], qt[DB][2];
#pragma unroll
      for (int dbk = 0; dbk < DB; ++dbk)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          gt[dbk][c] = at64::trfrag<true>(dOs, 32 * dbk, 32 * qs + 16 * c, lane);
          qt[dbk][c] = at64::trfrag<true>(Qs, 32 * dbk, 32 * qs + 16 * c, lane);
        }
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int dbk = 0; dbk < DB; ++dbk) {
          dv_acc[dbk] = mfma32(gt[dbk][c], pb[c], dv_acc[dbk]);
          dk_acc[dbk] = mfma32(qt[dbk][c], db8[c], dk_acc[dbk]);
        }
    };
    if (!wave_active) {
#pragma unroll
      for (int c = 0; c < 8; ++c) *(__attribute__((address_space(3))) bf16x4*)(dSt + at64::swz(32 * wave + l32, c) + 4 * hl) = bf16x4{};
    } else if ((qq0 < kw0 + 31) || (qq0 + kBwdM > S) || (kw0 + 32 > S) || kSeg) {
      qs_body(0, std::true_type{});
      __builtin_amdgcn_sched_barrier(0);  // keep the two halves' live ranges apart
      qs_body(1, std::true_type{});
    } else {
      qs_body(0, std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
      qs_body(1, std::false_type{});
    }
    GPTRIG_WAIT_LGKM0();
    wg_barrier();  // (B) dS^T published; Q / dO / lse / delta of this block no longer read
    store_q();

    if (wave < 4) {  // dQ tile of this wave: queries 32*(wave/2).., d 32*(wave%2).. over all NK keys.
      const int qs = wave >> 1, dblk = wave & 1;
      // Two independent accumulation chains halve the dependent-MFMA latency.
      f32x16 dqh[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int kq = 0; kq < NK / 64; ++kq) {
        bf16x8 af[4], bfk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          af[j] = at64::trfrag<false>(dSt, 32 * qs, 16 * (4 * kq + j), lane);
          bfk[j] = at64::trfrag<false>(Ks, 32 * dblk, 16 * (4 * kq + j), lane);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) dqh[kq & 1] = mfma32(af[j], bfk[j], dqh[kq & 1]);
      }
      const f32x16 dq = dqh[0] + dqh[1];
      // Row q = qq0 + 32qs + 4hl + 8(i/4) + i%4 of this lane's column; rows at
      // or past S fall outside the buffer resource and are dropped.
      const int voff = ((qq0 + 32 * qs + 4 * hl) * D + 32 * dblk + l32) * 4;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(dq[i], dq_rs, voff + (8 * (i >> 2) + (i & 3)) * D * 4, 0, 0);
    }
    // The next block's dS^T writes come after the next (A), which every wave
    // reaches only after finishing this dQ step.
  }

  if (k_ok) {
    bf16* dvrow = dV.row(b, h, my_k);
    bf16* dkrow = dK.row(b, h, my_k);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bf16x4 v4, k4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v4[t] = (bf16)dv_acc[db][4 * r + t];
          k4[t] = (bf16)dk_acc[db][4 * r + t];
        }
        if (rcs) {  // RoPE VJP: d = 32db + 8r + 4hl + t, pairs (t, t+1) for t = 0, 2
          const int j0 = (32 * db + 8 * r + 4 * hl) / 2;
          const bf16x2 c2 = *reinterpret_cast<const bf16x2*>(&rope_s[0][(32 * wave + l32) * (D / 2) + j0]);
          const bf16x2 s2 = *reinterpret_cast<const bf16x2*>(&rope_s[1][(32 * wave + l32) * (D / 2) + j0]);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const bf16x2 rr = rope_pair((float)k4[2 * u], (float)k4[2 * u + 1], (float)c2[u], -(float)s2[u]);
            k4[2 * u] = rr[0];
            k4[2 * u + 1] = rr[1];
          }
        }
        *reinterpret_cast<bf16x4*>(dvrow + 32 * db + 8 * r + 4 * hl) = v4;
        *reinterpret_cast<bf16x4*>(dkrow + 32 * db + 8 * r + 4 * hl) = k4;
      }
  }
}

// ============================================================================
// Backward, head_dim 128
// ============================================================================
// A workgroup owns 128 keys as 4 waves x 32 keys, one wave per SIMD (the dV /
// dK accumulators of 32 keys x 128 d are 128 registers per wave).  Each wave
// keeps its keys' K and V operands in registers for the whole loop.  Q / dO /
// lse / Delta and dS^T are double-buffered, one barrier per query block: a
// wave computes this block's scores and dV / dK, stores the prefetched next
// block to LDS, then computes the previous block's dQ tile and adds it with
// fp32 atomics.  Every 128-wide matrix in LDS is kept as two 64-wide
// swizzled tiles (d 0..63, then d 64..127), so the head_dim-64 swizzle and
// its row and transposed reads serve it unchanged.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr int kBwd128Threads = 256;
constexpr int kBwd128Keys = 128;

// Element offset of 16-byte chunk c16 (0..15) of row `row` in a 128-wide
// matrix of `rows` rows stored as two 64-wide tiles.
__device__ __forceinline__ int at128(int rows, int row, int c16) {
  return (c16 >> 3) * rows * 64 + at64::swz(row, c16 & 7);
}

template <bool kSeg>
__global__ void __launch_bounds__(kBwd128Threads, 1)
    attn_bwd128_kernel(View Q, View K, View V, View dO, const float* __restrict__ lse,
                       const float* __restrict__ delta, const int32_t* __restrict__ seg, float* __restrict__ dq_acc,
                       MutView dK, MutView dV, int B, int H, int S, float scale, float scale_log2,
                       const bf16* __restrict__ rcs, const bf16* __restrict__ rsn) {
  constexpr int D = 128, KC = D / 16, DB = D / 32, NT = kBwd128Threads, NK = kBwd128Keys, M = kBwdM;
  __shared__ __attribute__((aligned(16))) bf16 q_smem[2 * M * D];
  __shared__ __attribute__((aligned(16))) bf16 g_smem[2 * M * D];
  __shared__ __attribute__((aligned(16))) bf16 k_smem[NK * D];
  __shared__ __attribute__((aligned(16))) bf16 ds_smem[2 * NK * M];
  __shared__ __attribute__((aligned(16))) float lse_s[2 * M], delta_s[2 * M];
  __shared__ int seg_s[2 * M];
  at64::lds_t* const Ks = gemm::lds_cast(k_smem);

  const int nkv = (S + NK - 1) / NK;
  int bh, kb;
  xcd_map(blockIdx.x, nkv, B * H, bh, kb);
  const int b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int k0 = kb * NK;
  const int kw0 = k0 + 32 * wave;
  const int my_k = kw0 + l32;

  // The workgroup's K tile (dQ operand) into LDS and this wave's K and V
  // operands (B operands of S = Q K^T and dP = dO V^T, k = d) into registers,
  // through buffer resources over the (b, h) slice (rows at or past S read
  // as zeros); every load is issued before the first wait.
  const __amdgpu_buffer_rsrc_t k_rs = make_rsrc(K.row(b, h, 0), (uint32_t)(S * K.ss * 2));
  const __amdgpu_buffer_rsrc_t v_rs = make_rsrc(V.row(b, h, 0), (uint32_t)(S * V.ss * 2));
  constexpr int KR = NK * (D / 8) / NT;
  bf16x8 kst[KR];
#pragma unroll
  for (int r = 0; r < KR; ++r) {
    const int idx = tid + NT * r;
    kst[r] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                            k_rs, ((k0 + (idx >> 4)) * (int)K.ss + 8 * (idx & 15)) * 2, 0, 0));
  }
  bf16x8 kfr[KC], vfr[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    kfr[kc] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                             k_rs, (my_k * (int)K.ss + 8 * (2 * kc + hl)) * 2, 0, 0));
    vfr[kc] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                             v_rs, (my_k * (int)V.ss + 8 * (2 * kc + hl)) * 2, 0, 0));
  }
  const int seg_k = (kSeg && my_k < S) ? seg[(size_t)b * S + my_k] : 0;
#pragma unroll
  for (int r = 0; r < KR; ++r) {
    const int idx = tid + NT * r;
    *(at64::lds_x8*)(Ks + at128(NK, idx >> 4, idx & 15)) = kst[r];
  }

  f32x16 dv_acc[DB], dk_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dv_acc[db] = f32x16{};
    dk_acc[db] = f32x16{};
  }
  const __amdgpu_buffer_rsrc_t q_rs = make_rsrc(Q.row(b, h, 0), (uint32_t)(S * Q.ss * 2));
  const __amdgpu_buffer_rsrc_t g_rs = make_rsrc(dO.row(b, h, 0), (uint32_t)(S * dO.ss * 2));
  const __amdgpu_buffer_rsrc_t lse_rs = make_rsrc(lse + (size_t)bh * S, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t delta_rs = make_rsrc(delta + (size_t)bh * S, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t seg_rs =
      make_rsrc(kSeg ? (const void*)(seg + (size_t)b * S) : (const void*)lse, (uint32_t)S * 4u);
  const __amdgpu_buffer_rsrc_t dq_rs = make_rsrc(dq_acc + (size_t)bh * S * D, (uint32_t)S * D * 4u);

  // Register staging of one query block: 4 x 16 B of Q and of dO per thread.
  constexpr int QR = M * (D / 8) / NT;
  bf16x8 qst[QR], gst[QR];
  float lse_st = 0.f, delta_st = 0.f;
  int seg_st = 0;
  auto load_q = [&](int qq0) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int idx = tid + NT * r;
      const int qi = idx >> 4, c = idx & 15;
      qst[r] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                              q_rs, ((qq0 + qi) * (int)Q.ss + 8 * c) * 2, 0, 0));
      gst[r] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                              g_rs, ((qq0 + qi) * (int)dO.ss + 8 * c) * 2, 0, 0));
    }
    if (tid < M) {
      lse_st = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lse_rs, (qq0 + tid) * 4, 0, 0));
      delta_st = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(delta_rs, (qq0 + tid) * 4, 0, 0));
      if (kSeg) seg_st = (int)__builtin_amdgcn_raw_buffer_load_b32(seg_rs, (qq0 + tid) * 4, 0, 0);
    }
  };
  auto store_q = [&](int buf) {
    at64::lds_t* const Qs = gemm::lds_cast(q_smem) + buf * M * D;
    at64::lds_t* const dOs = gemm::lds_cast(g_smem) + buf * M * D;
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int idx = tid + NT * r;
      *(at64::lds_x8*)(Qs + at128(M, idx >> 4, idx & 15)) = qst[r];
      *(at64::lds_x8*)(dOs + at128(M, idx >> 4, idx & 15)) = gst[r];
    }
    if (tid < M) {
      lse_s[buf * M + tid] = lse_st * GPTRIG_LOG2E;
      delta_s[buf * M + tid] = delta_st * scale;  // dS = P * (scale*dP - scale*Delta)
      if (kSeg) seg_s[buf * M + tid] = seg_st;
    }
  };

  // dQ of a query block for queries 32*(wave/2).. and d 64*(wave%2).. (two
  // 32-wide tiles) over all NK keys, from that block's dS^T buffer (a wave
  // whose keys cannot see the block leaves zeros there), in groups of 32
  // keys whose LDS reads are issued one group ahead of their MFMAs.
  auto dq_step = [&](int qq0, int buf) {
    const at64::lds_t* const dSt = gemm::lds_cast(ds_smem) + buf * NK * M;
    const at64::lds_t* const Kh = Ks + (wave & 1) * NK * 64;
    const int qs = wave >> 1;
    bf16x8 fa[2][2], fb[2][2][2];
    auto rd = [&](int g) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        fa[g & 1][u] = at64::trfrag<false>(dSt, 32 * qs, 16 * (2 * g + u), lane);
#pragma unroll
        for (int j = 0; j < 2; ++j) fb[g & 1][u][j] = at64::trfrag<false>(Kh, 32 * j, 16 * (2 * g + u), lane);
      }
    };
    f32x16 acc[2] = {f32x16{}, f32x16{}};
    rd(0);
#pragma unroll
    for (int g = 0; g < NK / 32; ++g) {
      if (g + 1 < NK / 32) rd(g + 1);
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[j] = mfma32(fa[g & 1][u], fb[g & 1][u][j], acc[j]);
    }
    // Row q = qq0 + 32qs + 4hl + 8(i/4) + i%4 of this lane's column; rows at
    // or past S fall outside the buffer resource and are dropped.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int voff = ((qq0 + 32 * qs + 4 * hl) * D + 64 * (wave & 1) + 32 * j + l32) * 4;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(acc[j][i], dq_rs, voff + (8 * (i >> 2) + (i & 3)) * D * 4,
                                                        0, 0);
    }
  };
  // A wave whose keys cannot see a block leaves zeros as its dS^T rows.
  auto zero_ds = [&](int buf) {
    at64::lds_t* const dSt = gemm::lds_cast(ds_smem) + buf * NK * M;
#pragma unroll
    for (int r = 0; r < 32 * M / 8 / 64; ++r)
      *(at64::lds_x8*)(dSt + 32 * M * wave + 8 * (lane + 64 * r)) = bf16x8{};
  };

  const int qb_first = k0 / M;
  const int nqb = (S + M - 1) / M;
  load_q(qb_first * M);
  store_q(0);

  auto begin = [&](int qb) {
    // Q / dO / lse / Delta of this block and the previous block's dS^T published.
    GPTRIG_WAIT_LGKM0();
    wg_barrier();
    load_q(qb + 1 < nqb ? (qb + 1) * M : qb * M);
  };
  auto nbuf = [&](int qb) { return ((qb - qb_first) & 1) ^ 1; };  // the buffer of block qb - 1 / qb + 1

  // Scores, dS and dV / dK of query block qb against this wave's 32 keys.
  auto body = [&](int qb, auto mask_tag) {
    constexpr bool kMask = decltype(mask_tag)::value;
    const int qq0 = qb * M, buf = (qb - qb_first) & 1;
    const at64::lds_t* const Qs = gemm::lds_cast(q_smem) + buf * M * D;
    const at64::lds_t* const dOs = gemm::lds_cast(g_smem) + buf * M * D;
    at64::lds_t* const dSt = gemm::lds_cast(ds_smem) + buf * NK * M;
    const float* const ls = lse_s + buf * M;
    const float* const dls = delta_s + buf * M;
    const int* const sgs = seg_s + buf * M;
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      bf16x8 qf[KC], gf[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        qf[kc] = *(const at64::lds_x8*)(Qs + at128(M, 32 * qs + l32, 2 * kc + hl));
        gf[kc] = *(const at64::lds_x8*)(dOs + at128(M, 32 * qs + l32, 2 * kc + hl));
      }
      f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        sacc = mfma32(qf[kc], kfr[kc], sacc);
        pacc = mfma32(gf[kc], vfr[kc], pacc);
      }
      bf16x8 pb[2], db8[2];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qr = 32 * qs + 8 * r + 4 * hl;
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(&ls[qr]);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dls[qr]);
        bf16x4 ds4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int i = 4 * r + t;
          float p = fast_exp2(fmaf(sacc[i], scale_log2, -l4[t]));
          if (kMask) {
            // Causal; with segment ids also the document.  Queries and keys
            // at or past S need no mask: their Q / K / dO / V rows, lse and
            // Delta read as zeros, so they add nothing to dV, dK or dQ.
            const int q = qq0 + qr + t;
            bool vis = my_k <= q;
            if (kSeg && vis) vis = sgs[qr + t] == seg_k;
            p = vis ? p : 0.f;
          }
          const float ds = p * fmaf(pacc[i], scale, -d4[t]);
          pb[i >> 3][i & 7] = (bf16)p;
          const bf16 dsb = (bf16)ds;
          db8[i >> 3][i & 7] = dsb;
          ds4[t] = dsb;
        }
        // dS^T row = this lane's key, queries 32qs + 8r + 4hl .. +3.
        *(__attribute__((address_space(3))) bf16x4*)(dSt + at64::swz(32 * wave + l32, 4 * qs + r) + 4 * hl) = ds4;
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int half = (db >> 1) * M * 64;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const bf16x8 gt = at64::trfrag<true>(dOs + half, 32 * (db & 1), 32 * qs + 16 * c, lane);
          const bf16x8 qt = at64::trfrag<true>(Qs + half, 32 * (db & 1), 32 * qs + 16 * c, lane);
          dv_acc[db] = mfma32(gt, pb[c], dv_acc[db]);
          dk_acc[db] = mfma32(qt, db8[c], dk_acc[db]);
        }
      }
    }
  };

  // Per wave: the first block (no dQ before it), the blocks before this
  // wave's keys (no scores), the diagonal block (causal mask), the blocks
  // after it (mask-free unless segment ids are given).  Every wave runs
  // nqb - qb_first blocks, one barrier each, so the barriers match; no dQ is
  // conditional inside a phase, so the waits for the prefetched block count
  // the atomics issued after it instead of draining them.
  const int my_first = min(kw0 / M, nqb);
  begin(qb_first);
  if (my_first == qb_first)
    body(qb_first, std::true_type{});
  else
    zero_ds(0);
  store_q(1);
  int qb = qb_first + 1;
  for (; qb < my_first; ++qb) {
    begin(qb);
    zero_ds(nbuf(qb) ^ 1);
    dq_step((qb - 1) * M, nbuf(qb));
    store_q(nbuf(qb));
  }
  if (qb == my_first && qb < nqb) {
    begin(qb);
    body(qb, std::true_type{});
    store_q(nbuf(qb));
    dq_step((qb - 1) * M, nbuf(qb));
    ++qb;
  }
  for (; qb < nqb; ++qb) {
    begin(qb);
    body(qb, std::integral_constant<bool, kSeg>{});
    store_q(nbuf(qb));
    dq_step((qb - 1) * M, nbuf(qb));
  }

  // dV and dK rows of this wave's keys (lane: key my_k, d = 32db + 8r + 4hl
  // .. +3), with the RoPE VJP of dK when tables are given.  Stores and table
  // reads go through buffer resources (keys at or past S dropped / read as
  // zeros); all table reads are issued before the first use.
  const __amdgpu_buffer_rsrc_t dv_rs = make_rsrc(dV.row(b, h, 0), (uint32_t)(S * dV.ss * 2));
  const __amdgpu_buffer_rsrc_t dk_rs = make_rsrc(dK.row(b, h, 0), (uint32_t)(S * dK.ss * 2));
  uint32_t rc[DB][4], rsv[DB][4];
  if (rcs) {
    const __amdgpu_buffer_rsrc_t rc_rs = make_rsrc(rcs, (uint32_t)(S * (D / 2) * 2));
    const __amdgpu_buffer_rsrc_t rs_rs = make_rsrc(rsn, (uint32_t)(S * (D / 2) * 2));
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int off = (my_k * (D / 2) + (32 * db + 8 * r + 4 * hl) / 2) * 2;
        rc[db][r] = __builtin_amdgcn_raw_buffer_load_b32(rc_rs, off, 0, 0);
        rsv[db][r] = __builtin_amdgcn_raw_buffer_load_b32(rs_rs, off, 0, 0);
      }
  }
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bf16x4 v4, k4;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v4[t] = (bf16)dv_acc[db][4 * r + t];
        k4[t] = (bf16)dk_acc[db][4 * r + t];
      }
      if (rcs) {  // RoPE VJP: pairs (t, t+1) for t = 0, 2
        const bf16x2 c2 = __builtin_bit_cast(bf16x2, rc[db][r]);
        const bf16x2 s2 = __builtin_bit_cast(bf16x2, rsv[db][r]);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bf16x2 rr = rope_pair((float)k4[2 * u], (float)k4[2 * u + 1], (float)c2[u], -(float)s2[u]);
          k4[2 * u] = rr[0];
          k4[2 * u + 1] = rr[1];
        }
      }
      const int d0 = 32 * db + 8 * r + 4 * hl;
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v4), dv_rs, (my_k * (int)dV.ss + d0) * 2, 0,
                                            0);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, k4), dk_rs, (my_k * (int)dK.ss + d0) * 2, 0,
                                            0);
    }
  // The last block's dQ, after the dK / dV stores so no store waits for its atomics.
  GPTRIG_WAIT_LGKM0();
  wg_barrier();
  dq_step((nqb - 1) * M, (nqb - 1 - qb_first) & 1);
}

bool strides_ok(const int64_t* st, int n) {
  // Row starts must stay 16-byte aligned for the vector loads.
  for (int i = 0; i < 3 * n; ++i)
    if (st[i] < 0 || (st[i] & 7)) return false;
  return true;
}

void default_strides(int64_t* st, int n, int H, int S, int D) {
  for (int i = 0; i < n; ++i) {
    st[3 * i + 0] = (int64_t)H * S * D;
    st[3 * i + 1] = (int64_t)S * D;
    st[3 * i + 2] = D;
  }
}

}  // namespace

extern "C" {

int gptrig_attn_fwd(const void* q, const void* k, const void* v, const int32_t* segment_ids, void* o, float* lse,
                    int batch, int heads, int seq, int head_dim, const int64_t* strides, float softmax_scale,
                    void* stream) {
  if (!q || !k || !v || !o || !lse) return GPTRIG_E_NULL;
  if (batch <= 0 || heads <= 0 || seq <= 0 || head_dim <= 0) return GPTRIG_E_SHAPE;
  if (head_dim != 64 && head_dim != 128) return GPTRIG_E_UNSUPPORTED;
  if (!(softmax_scale > 0.f)) return GPTRIG_E_SHAPE;
  int64_t st[12];
  if (strides) {
    for (int i = 0; i < 12; ++i) st[i] = strides[i];
  } else {
    default_strides(st, 4, heads, seq, head_dim);
  }
  if (!strides_ok(st, 4)) return GPTRIG_E_SHAPE;
  View Q{(const bf16*)q, st[0], st[1], st[2]}, K{(const bf16*)k, st[3], st[4], st[5]},
      V{(const bf16*)v, st[6], st[7], st[8]};
  MutView O{(bf16*)o, st[9], st[10], st[11]};
  const int nq = (seq + kBlockM - 1) / kBlockM;
  const long long grid = (long long)batch * heads * nq;
  const float sl2 = softmax_scale * GPTRIG_LOG2E;
  hipStream_t s = (hipStream_t)stream;
  // The kernels copy one (b, h) slice of K / V through 32-bit buffer offsets.
  if ((long long)seq * (K.ss > V.ss ? K.ss : V.ss) * 2 >= (1ll << 31)) return GPTRIG_E_SHAPE;
  if (head_dim == 64) {
    if (segment_ids)
      attn_fwd64_kernel<true><<<(unsigned)grid, 256, 0, s>>>(Q, K, V, O, lse, segment_ids, batch, heads, seq, sl2);
    else
      attn_fwd64_kernel<false><<<(unsigned)grid, 256, 0, s>>>(Q, K, V, O, lse, nullptr, batch, heads, seq, sl2);
  } else {
    if (segment_ids)
      attn_fwd128_kernel<true><<<(unsigned)grid, 256, 0, s>>>(Q, K, V, O, lse, segment_ids, batch, heads, seq, sl2);
    else
      attn_fwd128_kernel<false><<<(unsigned)grid, 256, 0, s>>>(Q, K, V, O, lse, nullptr, batch, heads, seq, sl2);
  }
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

size_t gptrig_attn_bwd_workspace_bytes(int batch, int heads, int seq, int head_dim) {
  const size_t rows = (size_t)batch * heads * seq;
  const size_t delta = (rows * sizeof(float) + 255) & ~(size_t)255;
  return delta + rows * head_dim * sizeof(float);
}

}  // extern "C"

namespace {

// The backward launches; rcs / rsn (nullable) add the RoPE VJP to dq and dk.
int attn_bwd_impl(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                  const int32_t* segment_ids, void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                  int batch, int heads, int seq, int head_dim, const int64_t* strides, float softmax_scale,
                  const bf16* rcs, const bf16* rsn, void* stream) {
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv || !workspace) return GPTRIG_E_NULL;
  if (batch <= 0 || heads <= 0 || seq <= 0 || head_dim <= 0) return GPTRIG_E_SHAPE;
  if (head_dim != 64 && head_dim != 128) return GPTRIG_E_UNSUPPORTED;
  if (!(softmax_scale > 0.f)) return GPTRIG_E_SHAPE;
  if (workspace_bytes < gptrig_attn_bwd_workspace_bytes(batch, heads, seq, head_dim)) return GPTRIG_E_WORKSPACE;
  if ((uintptr_t)workspace & 15) return GPTRIG_E_SHAPE;
  int64_t st[24];
  if (strides) {
    for (int i = 0; i < 24; ++i) st[i] = strides[i];
  } else {
    default_strides(st, 8, heads, seq, head_dim);
  }
  if (!strides_ok(st, 8)) return GPTRIG_E_SHAPE;
  View Q{(const bf16*)q, st[0], st[1], st[2]}, K{(const bf16*)k, st[3], st[4], st[5]},
      V{(const bf16*)v, st[6], st[7], st[8]}, O{(const bf16*)o, st[9], st[10], st[11]},
      dO{(const bf16*)dout, st[12], st[13], st[14]};
  MutView dQ{(bf16*)dq, st[15], st[16], st[17]}, dK{(bf16*)dk, st[18], st[19], st[20]},
      dV{(bf16*)dv, st[21], st[22], st[23]};
  const size_t rows = (size_t)batch * heads * seq;
  float* delta = (float*)workspace;
  float* dq_acc = (float*)((char*)workspace + ((rows * sizeof(float) + 255) & ~(size_t)255));
  hipStream_t s = (hipStream_t)stream;
  const float sl2 = softmax_scale * GPTRIG_LOG2E;
  if (head_dim == 64) {
    // The kernel addresses one (b, h) slice of Q / dO / dq_acc through 32-bit
    // buffer offsets.
    const long long span = (long long)seq * (Q.ss > dO.ss ? Q.ss : dO.ss) * 2;
    if (span >= (1ll << 31) || (long long)seq * 64 * 4 >= (1ll << 31)) return GPTRIG_E_SHAPE;
    attn_bwd_pre_kernel<64><<<ceil_div((long long)rows * 8, 256), 256, 0, s>>>(O, dO, delta, dq_acc, batch, heads,
                                                                                seq);
    GPTRIG_CHECK_LAUNCH();
    const unsigned grid64 = (unsigned)((long long)batch * heads * ceil_div(seq, kBwd64Keys));
    if (segment_ids)
      attn_bwd64_kernel<true><<<grid64, kBwd64Threads, 0, s>>>(Q, K, V, dO, lse, delta, segment_ids, dq_acc, dK, dV,
                                                               batch, heads, seq, softmax_scale, sl2, rcs, rsn);
    else
      attn_bwd64_kernel<false><<<grid64, kBwd64Threads, 0, s>>>(Q, K, V, dO, lse, delta, nullptr, dq_acc, dK, dV,
                                                                batch, heads, seq, softmax_scale, sl2, rcs, rsn);
    GPTRIG_CHECK_LAUNCH();
    attn_dq_convert_kernel<64><<<ceil_div((long long)rows * 8, 256), 256, 0, s>>>(dq_acc, dQ, batch, heads, seq,
                                                                                   rcs, rsn);
  } else {
    const long long span = (long long)seq * (Q.ss > dO.ss ? Q.ss : dO.ss) * 2;
    const long long kspan = (long long)seq * (K.ss > V.ss ? K.ss : V.ss) * 2;
    const long long ospan = (long long)seq * (dK.ss > dV.ss ? dK.ss : dV.ss) * 2;
    if (span >= (1ll << 31) || kspan >= (1ll << 31) || ospan >= (1ll << 31) || (long long)seq * 128 * 4 >= (1ll << 31))
      return GPTRIG_E_SHAPE;
    attn_bwd_pre_kernel<128><<<ceil_div((long long)rows * 16, 256), 256, 0, s>>>(O, dO, delta, dq_acc, batch, heads,
                                                                                 seq);
    GPTRIG_CHECK_LAUNCH();
    const unsigned grid128 = (unsigned)((long long)batch * heads * ceil_div(seq, kBwd128Keys));
    if (segment_ids)
      attn_bwd128_kernel<true><<<grid128, kBwd128Threads, 0, s>>>(Q, K, V, dO, lse, delta, segment_ids, dq_acc, dK,
                                                                  dV, batch, heads, seq, softmax_scale, sl2, rcs, rsn);
    else
      attn_bwd128_kernel<false><<<grid128, kBwd128Threads, 0, s>>>(Q, K, V, dO, lse, delta, nullptr, dq_acc, dK, dV,
                                                                   batch, heads, seq, softmax_scale, sl2, rcs, rsn);
    GPTRIG_CHECK_LAUNCH();
    attn_dq_convert_kernel<128><<<ceil_div((long long)rows * 16, 256), 256, 0, s>>>(dq_acc, dQ, batch, heads, seq,
                                                                                    rcs, rsn);
  }
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // namespace

extern "C" {

int gptrig_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                    const int32_t* segment_ids, void* dq, void* dk, void* dv, void* workspace,
                    size_t workspace_bytes, int batch, int heads, int seq, int head_dim, const int64_t* strides,
                    float softmax_scale, void* stream) {
  return attn_bwd_impl(q, k, v, o, dout, lse, segment_ids, dq, dk, dv, workspace, workspace_bytes, batch, heads, seq,
                       head_dim, strides, softmax_scale, nullptr, nullptr, stream);
}

int gptrig_attn_bwd_rope(const void* q, const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, const int32_t* segment_ids, void* dq, void* dk, void* dv, void* workspace,
                         size_t workspace_bytes, int batch, int heads, int seq, int head_dim, const int64_t* strides,
                         float softmax_scale, const void* rope_cos, const void* rope_sin, void* stream) {
  if (!rope_cos || !rope_sin) return GPTRIG_E_NULL;
  if (((uintptr_t)rope_cos | (uintptr_t)rope_sin) & 7) return GPTRIG_E_SHAPE;
  return attn_bwd_impl(q, k, v, o, dout, lse, segment_ids, dq, dk, dv, workspace, workspace_bytes, batch, heads, seq,
                       head_dim, strides, softmax_scale, (const bf16*)rope_cos, (const bf16*)rope_sin, stream);
}

}  // extern "C"
