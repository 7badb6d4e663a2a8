// bf16 MFMA GEMM core for gfx950: C[m][n] = sum_k A(m,k) B(k,n), fp32 accumulate.
//
// Workgroup tile 256 x 256 x 64, 512 threads = 8 waves laid out 2 (M) x 4 (N),
// each wave owning a 128 x 64 sub-tile as 4 x 2 blocks of v_mfma_f32_32x32x16_bf16.
// LDS is double buffered (2 operands x 2 stages, 144 KB).
//
// Each operand is K-major (A[m*ld + k], B[n*ld + k]) or MN-major
// (A[k*ld + m], B[k*ld + n]).  Both are copied to LDS in their natural layout
// with 16-byte stores.  K-major fragments are one 16-byte LDS read per lane;
// MN-major fragments use ds_read_b64_tr_b16, which hands each lane of a
// 16-lane group the column of a 4 x 16 block: lane c supplies the address of
// row k0 + c/4, columns m0 + 4(c%4) .. +3, and lane i receives rows k0..k0+3 of
// column m0 + i.  Two such reads give the 8 k-values of one MFMA operand.
#pragma once

#include "common.h"

namespace gemm {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int THREADS = 512;
constexpr int KLD = BK + 8;         // K-major LDS row stride (elements), 144 B rows
constexpr int MLD = 256 + 32;       // MN-major LDS row stride: 576 B rows, 144 dwords == 16 (mod 64 banks)
constexpr int SLAB = 256 * KLD;     // elements per operand per stage (>= BK * MLD)
static_assert(BK * MLD <= SLAB, "MN-major slab must fit");
constexpr int LDS_BYTES = 4 * SLAB * 2;
constexpr int kGroupM = 8;

typedef short v4i16 __attribute__((ext_vector_type(4)));
// Address-space-qualified views: LDS (3) so fragment traffic is ds_read/ds_write,
// global (1) so operand loads are global_load rather than flat.
typedef __attribute__((address_space(3))) bf16 lds_t;
typedef __attribute__((address_space(3))) bf16x8 lds_x8;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef const __attribute__((address_space(1))) bf16x8 gbl_x8;

// Element (row r, column c) of the stored matrix is p[row(r) * ld + c] with
// row(r) = idx ? idx[r] : r: idx gathers rows (K-major: M/N rows; MN-major:
// k rows), which is how the routed expert GEMMs read token rows in bucket
// order without a gathered copy.
struct Operand {
  const bf16* p;
  int64_t ld;
  const int32_t* idx = nullptr;
};

__device__ __forceinline__ lds_t* lds_cast(bf16* p) { return (lds_t*)p; }

__device__ __forceinline__ bf16x4 read_tr(const lds_t* lds) {
  v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds));
  return __builtin_bit_cast(bf16x4, r);
}

// Global -> registers: 4 x 16 bytes per thread per 256 x 64 slab.
template <bool KMAJOR>
__device__ __forceinline__ void load_slab(bf16x8 (&st)[4], Operand op, int mn0, int k0, int MN, int K, int tid) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int idx = tid + THREADS * r;
    if (KMAJOR) {
      const int row = idx >> 3, kc = (idx & 7) * 8;
      const int m = mn0 + row, k = k0 + kc;
      if (m < MN && k < K) {
        const int64_t pr = op.idx ? op.idx[m] : m;
        st[r] = *(gbl_x8*)(op.p + pr * op.ld + k);
      } else {
        st[r] = bf16x8{};
      }
    } else {
      const int kk = idx >> 5, mc = (idx & 31) * 8;
      const int m = mn0 + mc, k = k0 + kk;
      if (m < MN && k < K) {
        const int64_t pk = op.idx ? op.idx[k] : k;
        st[r] = *(gbl_x8*)(op.p + pk * op.ld + m);
      } else {
        st[r] = bf16x8{};
      }
    }
  }
}

template <bool KMAJOR>
__device__ __forceinline__ void store_slab(lds_t* lds, const bf16x8 (&st)[4], int tid) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int idx = tid + THREADS * r;
    if (KMAJOR) {
      const int row = idx >> 3, kc = (idx & 7) * 8;
      *(lds_x8*)(lds + row * KLD + kc) = st[r];
    } else {
      const int kk = idx >> 5, mc = (idx & 31) * 8;
      *(lds_x8*)(lds + kk * MLD + mc) = st[r];
    }
  }
}

// MFMA operand (8 k-values) for rows r0 .. r0+31 at k-chunk kc of a slab.
template <bool KMAJOR>
__device__ __forceinline__ bf16x8 frag(const lds_t* lds, int r0, int kc, int lane) {
  const int hl = lane >> 5;
  if (KMAJOR) {
    return *(const lds_x8*)(lds + (r0 + (lane & 31)) * KLD + 16 * kc + 8 * hl);
  } else {
    const int c = lane & 15;
    const int m = r0 + 16 * ((lane >> 4) & 1) + 4 * (c & 3);
    const int k = 16 * kc + 8 * hl + (c >> 2);
    bf16x4 lo = read_tr(lds + k * MLD + m);
    bf16x4 hi = read_tr(lds + (k + 4) * MLD + m);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Give XCD x a contiguous range of logical tile ids so that the tiles sharing
// A/B slabs run on the same L2.
__device__ __forceinline__ int xcd_swizzle(int pid, int total) {
  const int q = total >> 3, r = total & 7, x = pid & 7;
  return x * q + min(x, r) + (pid >> 3);
}

// Grouped tile order: kGroupM M-tiles share each N sweep so their B slabs stay in L2.
__device__ __forceinline__ void tile_coords(int pid, int M, int N, int& tm, int& tn) {
  const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
  pid = xcd_swizzle(pid, mt * nt);
  const int in_group = kGroupM * nt;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsize = min(mt - first_m, kGroupM);
  tm = first_m + (pid % in_group) % gsize;
  tn = (pid % in_group) / gsize;
}

// Column sums of an MN-major B slab: thread t adds rows 8(t/64) .. +7 of
// columns 4(t%64) .. +3 (one 8-byte LDS read per row) into sum.
__device__ __forceinline__ void colsum_slab(f32x4& sum, const lds_t* lb, int tid) {
  const int n4 = (tid & 63) * 4, k0 = (tid >> 6) * 8;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const bf16x4 v = *(const __attribute__((address_space(3))) bf16x4*)(lb + (k0 + k) * MLD + n4);
    sum[0] += (float)v[0];
    sum[1] += (float)v[1];
    sum[2] += (float)v[2];
    sum[3] += (float)v[3];
  }
}

// acc[mb][nb][i] = C[tm0 + wm0 + 32mb + 8(i/4) + 4(lane/32) + i%4][tn0 + wn0 + 32nb + lane%32]
// with wm0 = 128*(wave&1), wn0 = 64*(wave>>1); K range [k_begin, k_end).
// With kColSum (MN-major B only) and colsum_on, colsum also accumulates the
// column sums of B over the K range (see colsum_slab for the thread mapping).
template <bool AK, bool BKM, bool kColSum = false>
__device__ __forceinline__ void mainloop(f32x16 (&acc)[4][2], Operand A, Operand B, int M, int N, int k_begin,
                                         int k_end, int tm0, int tn0, bf16* lds, f32x4* colsum = nullptr,
                                         bool colsum_on = false) {
  static_assert(!kColSum || !BKM, "column sums need an MN-major B operand");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = 128 * (wave & 1), wn0 = 64 * (wave >> 1);
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};
  const int nk = (k_end - k_begin + BK - 1) / BK;
  if (nk <= 0) return;
  lds_t* const lbase = lds_cast(lds);
  bf16x8 sa[4], sb[4];
  load_slab<AK>(sa, A, tm0, k_begin, M, k_end, tid);
  load_slab<BKM>(sb, B, tn0, k_begin, N, k_end, tid);
  store_slab<AK>(lbase, sa, tid);
  store_slab<BKM>(lbase + 2 * SLAB, sb, tid);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const lds_t* la = lbase + buf * SLAB;
    const lds_t* lb = lbase + (2 + buf) * SLAB;
    if (kt + 1 < nk) {
      load_slab<AK>(sa, A, tm0, k_begin + (kt + 1) * BK, M, k_end, tid);
      load_slab<BKM>(sb, B, tn0, k_begin + (kt + 1) * BK, N, k_end, tid);
    }
#pragma unroll
    for (int kc = 0; kc < BK / 16; ++kc) {
      bf16x8 fa[4], fb[2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) fa[mb] = frag<AK>(la, wm0 + 32 * mb, kc, lane);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) fb[nb] = frag<BKM>(lb, wn0 + 32 * nb, kc, lane);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(fa[mb], fb[nb], acc[mb][nb]);
    }
    if (kColSum && colsum_on) colsum_slab(*colsum, lb, tid);
    if (kt + 1 < nk) {
      store_slab<AK>(lbase + (buf ^ 1) * SLAB, sa, tid);
      store_slab<BKM>(lbase + (2 + (buf ^ 1)) * SLAB, sb, tid);
    }
    __syncthreads();
  }
}

// ---- host side: launch shaping ----

inline int device_cus() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cached[dev] = c;
  }
  return cached[dev];
}

// K-split count for a GEMM of `tiles` output tiles over k_iters BK-steps.
// One 256x256 workgroup fills a CU (its LDS use allows no second), so the grid
// runs in ceil(tiles*split/CUs) rounds of k_iters/split steps each, plus one
// fp32 atomic epilogue per round (about 3% of a full-K mainloop).  The split
// minimising that estimate keeps the last round from running a CU-sized
// grid a quarter full, which a fixed split does for skinny outputs.
inline int choose_split(unsigned tiles, int k_iters) {
  const int cus = device_cus();
  const int max_split = k_iters / 4 > 1 ? k_iters / 4 : 1;
  double best = 1e30;
  int best_split = 1;
  for (int s = 1; s <= max_split && s <= 256; ++s) {
    const double rounds = (double)ceil_div((int64_t)tiles * s, (int64_t)cus);
    const double cost = rounds * (1.0 / s + 0.03);
    if (cost < best * 0.999) {
      best = cost;
      best_split = s;
    }
  }
  return best_split;
}

}  // namespace gemm
