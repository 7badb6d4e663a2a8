// Top-k expert routing (recipes/reference_moe/train.py:1259-1273).
//
// route_topk: one thread per token.  softmax over the fp32 router logits,
//   jax.lax.top_k selection (largest value first; on equal values the lower
//   expert index first), softmax over the chosen logits.
// route_sort: one 1024-thread workgroup builds the dropless bucket layout:
//   counts[e], and order = stable argsort(chosen.reshape(-1)) by counting sort
//   (per-expert bases from an exclusive scan of counts, stable ranks from
//   wave ballots in slot order), rows = order / top_k.
#include "common.h"

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

__global__ void __launch_bounds__(1024) route_sort_kernel(const int32_t* __restrict__ chosen, int n_slots, int E,
                                                          int k, int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ order, int32_t* __restrict__ rows) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int wave_cnt[16][kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < E) cnt[tid] = 0;
  __syncthreads();
  for (int s = tid; s < n_slots; s += blockDim.x) atomicAdd(&cnt[chosen[s]], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      base[e] = acc;
      acc += cnt[e];
      counts[e] = cnt[e];
    }
  }
  __syncthreads();
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int tile = 0; tile < n_slots; tile += blockDim.x) {
    const int s = tile + tid;
    const int my_e = s < n_slots ? chosen[s] : -1;
    int rank = 0;
    for (int e = 0; e < E; ++e) {
      const uint64_t m = __ballot(my_e == e);
      if (my_e == e) rank = __popcll(m & lt_mask);
      if (lane == 0) wave_cnt[wave][e] = __popcll(m);
    }
    __syncthreads();
    if (my_e >= 0) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += wave_cnt[w][my_e];
      const int pos = base[my_e] + before + rank;
      order[pos] = s;
      rows[pos] = s / k;
    }
    __syncthreads();
    if (tid < E) {
      int tot = 0;
      for (int w = 0; w < 16; ++w) tot += wave_cnt[w][tid];
      base[tid] += tot;
    }
    __syncthreads();
  }
}

}  // namespace

extern "C" {

size_t gptrig_moe_route_workspace_bytes(int tokens, int experts, int top_k) {
  (void)tokens;
  (void)experts;
  (void)top_k;
  return 0;
}

int gptrig_moe_route(const float* logits, float* probs, int32_t* chosen, float* gate, int32_t* counts,
                     int32_t* order, int32_t* rows, void* workspace, size_t workspace_bytes, int tokens, int experts,
                     int top_k, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (!logits || !chosen || !gate || !counts || !order || !rows) return GPTRIG_E_NULL;
  if (tokens <= 0 || experts <= 0 || top_k <= 0) return GPTRIG_E_SHAPE;
  if (experts > kMaxExperts || top_k > experts) return GPTRIG_E_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  route_topk_kernel<<<ceil_div(tokens, 128), 128, 0, s>>>(logits, probs, chosen, gate, tokens, experts, top_k);
  GPTRIG_CHECK_LAUNCH();
  route_sort_kernel<<<1, 1024, 0, s>>>(chosen, tokens * top_k, experts, top_k, counts, order, rows);
  GPTRIG_CHECK_LAUNCH();
  return GPTRIG_OK;
}

}  // extern "C"
