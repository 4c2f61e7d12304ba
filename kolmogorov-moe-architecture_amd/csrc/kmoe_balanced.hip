// Capacity-balanced top-k: Router._balanced_topk_assignment (moe_arch/model/moe.py:353-421),
// used by Router.forward when moe_balanced_routing is set (moe.py:443-451).
//
// k rounds over all tokens at once, one launch per round (the capacity test of a
// round needs the whole previous round's counts).  cap = max(T*k/E, 1).  In round r
// an expert is full when the picks of rounds < r reached cap; each token takes its
// best expert (fp32 logit descending, equal logits -> lowest index) among those it
// has not picked and that are not full, else (all full) its best expert not picked
// yet (moe.py:402-407).  The round's picks are counted per block in LDS and added
// to the round's global histogram with integer atomics (order-independent totals).
// Weights are the picks' softmax probabilities, normalised by their sum + 1e-9 in
// the last round (moe.py:411,420).
#include "kmoe_common.h"

namespace {

constexpr int BT_THREADS = 256;  // one token per thread

__global__ __launch_bounds__(BT_THREADS) void balanced_round_kernel(const float* __restrict__ logits, int64_t T,
                                                                   int E, int k, int round, int cap,
                                                                   int32_t* __restrict__ hist,
                                                                   int64_t* __restrict__ idx, float* __restrict__ w) {
  __shared__ int full_l[KMOE_MAX_EXPERTS];
  __shared__ int cnt_l[KMOE_MAX_EXPERTS];
  const int tid = threadIdx.x;
  if (tid < E) {
    int c = 0;
    for (int r = 0; r < round; ++r) c += hist[r * E + tid];
    full_l[tid] = c >= cap;
    cnt_l[tid] = 0;
  }
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * BT_THREADS + tid;
  if (t < T) {
    const float* lg = logits + t * E;
    uint64_t taken = 0;
    for (int r = 0; r < round; ++r) taken |= 1ull << (int)idx[t * k + r];
    int best = -1, alt = -1;
    float best_l = 0.0f, alt_l = 0.0f, mx = -INFINITY;
    for (int e = 0; e < E; ++e) {
      const float v = lg[e];
      mx = fmaxf(mx, v);
      if ((taken >> e) & 1ull) continue;
      if (alt < 0 || v > alt_l) {
        alt = e;
        alt_l = v;
      }
      if (!full_l[e] && (best < 0 || v > best_l)) {
        best = e;
        best_l = v;
      }
    }
    if (best < 0) best = alt;
    float den = 0.0f;
    for (int e = 0; e < E; ++e) den += __expf(lg[e] - mx);
    const float p = __expf(lg[best] - mx) / den;
    idx[t * k + round] = best;
    if (round + 1 < k) {
      w[t * k + round] = p;  // normalised in the last round
    } else {
      float s = 0.0f;
      for (int r = 0; r < round; ++r) s += w[t * k + r];
      s += p;
      const float inv = 1.0f / (s + 1e-9f);
      for (int r = 0; r < round; ++r) w[t * k + r] *= inv;
      w[t * k + round] = p * inv;
    }
    atomicAdd(&cnt_l[best], 1);
  }
  __syncthreads();
  if (tid < E && cnt_l[tid] > 0) atomicAdd(&hist[round * E + tid], cnt_l[tid]);
}

__global__ void zero_i32_kernel(int32_t* __restrict__ p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

}  // namespace

extern "C" size_t kmoe_balanced_workspace_bytes(int E, int k) {
  return (size_t)(E > 0 ? E : 0) * (size_t)(k > 0 ? k : 0) * sizeof(int32_t);
}

extern "C" int kmoe_balanced_topk(const float* logits, int64_t T, int E, int k, int64_t* idx, float* w,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  KMOE_REQUIRE(logits && idx && w, KMOE_ERR_NULL, "kmoe_balanced_topk: null buffer");
  KMOE_REQUIRE(T >= 0 && T * (int64_t)k < ((int64_t)1 << 31), KMOE_ERR_SHAPE, "kmoe_balanced_topk: T*k must fit in int32");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_balanced_topk: E=%d out of range", E);
  KMOE_REQUIRE(k >= 1 && k <= 8 && k <= E, KMOE_ERR_SHAPE, "kmoe_balanced_topk: k=%d not in [1, min(8,E)]", k);
  KMOE_REQUIRE(workspace && workspace_bytes >= kmoe_balanced_workspace_bytes(E, k), KMOE_ERR_WORKSPACE,
               "kmoe_balanced_topk: workspace %zu < %zu bytes", workspace_bytes, kmoe_balanced_workspace_bytes(E, k));
  if (T == 0) return KMOE_OK;
  hipStream_t s = kmoe::as_stream(stream);
  int32_t* hist = static_cast<int32_t*>(workspace);
  const int64_t tk = T * (int64_t)k / E;
  const int cap = (int)(tk > 1 ? tk : 1);
  hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(256), 0, s, hist, E * k);
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T, BT_THREADS));
  for (int r = 0; r < k; ++r)
    hipLaunchKernelGGL(balanced_round_kernel, grid, dim3(BT_THREADS), 0, s, logits, T, E, k, r, cap, hist, idx, w);
  return kmoe::check_launch("kmoe_balanced_topk");
}
