// Dispatch: stable counting sort of the T*k token->expert assignments, optional
// capacity drop, and the gather of token rows into expert-contiguous order.
// Replaces the argsort/bincount/cumsum/gather/pad block of GroupedExperts.forward
// (moe_arch/model/moe.py:238-272); the capacity drop is this build's rule for
// config 3 (keep the first `capacity` assignments of each expert in assignment
// order, drop the rest).
//
// Launches, no host sync:
//   1. hist:    per-block (DTB tokens) expert histograms (skipped by
//               kmoe_dispatch_counted: the router wrote them)
//   2. scan:    per-expert exclusive scan over blocks -> block bases, counts,
//               kept counts and expert offsets (up to FUSED_SCAN_MAX_BLOCKS blocks
//               each permute block computes its own share of this instead)
//   3. permute: per-block stable ranks via wave ballots -> slot tables
//   4. rows (when asked for): one wave per token reads its row once and writes its
//               kept permuted rows (bf16 copy, or e4m3 with the per-token scale)
#include <mutex>

#include "kmoe_common.h"

namespace {

constexpr int DTB = 64;       // tokens per dispatch block
constexpr int DTHREADS = 256;

__device__ __forceinline__ int load_expert(const int64_t* idx, int64_t a, int E) {
  int64_t e = idx[a];
  return (e >= 0 && e < E) ? (int)e : -1;  // out-of-range ids are dropped
}

__global__ __launch_bounds__(DTHREADS) void hist_kernel(const int64_t* __restrict__ idx, int64_t T, int k, int E,
                                                        int32_t* __restrict__ block_counts) {
  __shared__ int cnt[KMOE_MAX_EXPERTS];
  const int tid = threadIdx.x;
  if (tid < E) cnt[tid] = 0;
  __syncthreads();
  const int64_t a0 = (int64_t)blockIdx.x * DTB * k;
  const int64_t a1 = min<int64_t>(a0 + (int64_t)DTB * k, T * k);
  for (int64_t a = a0 + tid; a < a1; a += DTHREADS) {
    int e = load_expert(idx, a, E);
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid < E) block_counts[(int64_t)blockIdx.x * E + tid] = cnt[tid];
}

// Single workgroup of 16 waves: wave w scans experts w, w+16, ... over the blocks
// (64 blocks per shuffle scan), then thread 0 lays out the expert offsets.
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* __restrict__ block_counts, int64_t nblk, int E,
                                                    int64_t capacity, int32_t* __restrict__ block_base,
                                                    int32_t* __restrict__ counts, int32_t* __restrict__ offsets) {
  __shared__ int total[KMOE_MAX_EXPERTS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
  for (int e = wave; e < E; e += nwave) {
    int running = 0;
    for (int64_t b0 = 0; b0 < nblk; b0 += 64) {
      const int64_t b = b0 + lane;
      const int v = b < nblk ? block_counts[b * E + e] : 0;
      int s = v;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(s, o, 64);
        if (lane >= o) s += u;
      }
      if (b < nblk) block_base[b * E + e] = running + s - v;
      running += __shfl(s, 63, 64);
    }
    if (lane == 0) total[e] = running;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0;
    for (int e = 0; e < E; ++e) {
      const int c = total[e];
      counts[e] = c;
      offsets[e] = off;
      off += (capacity > 0 && c > capacity) ? (int)capacity : c;
    }
    offsets[E] = off;
  }
}

// Tables of a block of DTB tokens (the rows are copied by scatter_rows_kernel).
// FUSED_SCAN: the block computes its own per-expert base (sum of the counts of the
// blocks before it), the totals and the expert offsets from all block counts (block
// 0 also writes counts and offsets), instead of reading them from the scan kernel:
// one launch less, for up to FUSED_SCAN_MAX_BLOCKS blocks.
// With aux_out (FUSED_SCAN only) the launch has one block more, block nblk: it sums the
// block counts like the others (the routed count of each expert), then reduces the
// router's aux partials and writes the auxiliary losses (aux_reduce_cols / aux_finish:
// the same sums in the same order as kmoe_aux_loss) instead of a launch of its own.
// The histograms may be finer than the DTB-token blocks (FUSED_SCAN only): nhb rows of
// DTB / hper tokens each (the router's 32-token workgroups give hper = 2), so block b
// starts after histogram row b * hper; the aux partials have the same nhb rows.
constexpr int FUSED_SCAN_MAX_BLOCKS = 1024;
template <bool FUSED_SCAN>
__global__ __launch_bounds__(DTHREADS) void permute_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, int64_t T, int d,
    const int64_t* __restrict__ idx, const void* __restrict__ wsrc, int w_dtype, int k, int E, int64_t capacity,
    const int32_t* __restrict__ block_counts, int64_t nblk, int64_t nhb, int hper,
    const int32_t* __restrict__ block_base, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ row_token, int32_t* __restrict__ slot_row, float* __restrict__ slot_w,
    const float* __restrict__ aux_partials, float w_lb, float w_z, float* __restrict__ aux_out) {
  __shared__ int wave_cnt[DTHREADS / 64][KMOE_MAX_EXPERTS];
  __shared__ int running[KMOE_MAX_EXPERTS];
  __shared__ int base_l[KMOE_MAX_EXPERTS];
  __shared__ int off_l[KMOE_MAX_EXPERTS + 1];
  __shared__ int tot_l[KMOE_MAX_EXPERTS];           // aux block: routed count per expert
  __shared__ float aux_col[KMOE_MAX_EXPERTS + 1];  // aux block: partial column sums
  const bool aux_block = FUSED_SCAN && aux_out && (int64_t)blockIdx.x == nblk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * DTB;
  const int64_t a0 = t0 * k;
  const int64_t a1 = min<int64_t>(a0 + (int64_t)DTB * k, T * k);
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  if (tid < E) running[tid] = 0;
  auto load_w = [&](int64_t a) -> float {
    return w_dtype == KMOE_DTYPE_F32 ? static_cast<const float*>(wsrc)[a]
                                     : bf16_to_f32(static_cast<const uint16_t*>(wsrc)[a]);
  };
  // the first chunk's expert ids and weights are loaded before the scan, so their round
  // trips overlap the block-count loads
  bool valid = a0 + tid < a1;
  int e = valid ? load_expert(idx, a0 + tid, E) : -1;
  float wv = valid ? load_w(a0 + tid) : 0.0f;
  if constexpr (FUSED_SCAN) {
    // thread (j, e) of an ep x (DTHREADS/ep) grid sums blocks j, j + DTHREADS/ep, ...
    __shared__ int red_pre[DTHREADS], red_tot[DTHREADS];
    int ep = 1;
    while (ep < E) ep <<= 1;
    const int ex = tid & (ep - 1), j = tid / ep, ng = DTHREADS / ep;
    int pre = 0, tot = 0;
    if (ex < E) {
      // 16 loads in flight per batch (a loop of dependent round trips took most of the
      // kernel's time)
      constexpr int NB = 16;
      const int64_t first = (int64_t)blockIdx.x * hper;  // this block's first histogram row
      for (int64_t b0 = j; b0 < nhb; b0 += (int64_t)NB * ng) {
        int v[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const int64_t b = b0 + (int64_t)u * ng;
          v[u] = b < nhb ? block_counts[b * E + ex] : 0;
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          tot += v[u];
          if (b0 + (int64_t)u * ng < first) pre += v[u];
        }
      }
    }
    red_pre[tid] = pre;
    red_tot[tid] = tot;
    __syncthreads();
    if (wave == 0) {
      // lane e: sums over the groups, then the exclusive scan of the kept counts
      int p = 0, c = 0;
      if (lane < E) {
        for (int jj = 0; jj < ng; ++jj) {
          p += red_pre[jj * ep + lane];
          c += red_tot[jj * ep + lane];
        }
      }
      const int kept = (capacity > 0 && c > capacity) ? (int)capacity : c;
      int incl = kept;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o, 64);
        if (lane >= o) incl += u;
      }
      if (lane < E) {
        base_l[lane] = p;
        off_l[lane] = incl - kept;
        tot_l[lane] = c;
        if (blockIdx.x == 0) {
          counts[lane] = c;
          offsets[lane] = incl - kept;
        }
      }
      const int all = __shfl(incl, E - 1, 64);
      if (lane == 0) {
        off_l[E] = all;
        if (blockIdx.x == 0) offsets[E] = all;
      }
    }
  } else {
    if (tid < E) {
      base_l[tid] = block_base[(int64_t)blockIdx.x * E + tid];
      off_l[tid] = offsets[tid];
    }
  }
  __syncthreads();
  if (aux_block) {
    aux_reduce_cols(aux_partials, nhb, E, wave, DTHREADS / 64, lane, aux_col);
    __syncthreads();
    if (tid == 0) aux_finish(aux_col, tot_l, T, E, k, w_lb, w_z, aux_out);
    return;
  }

  // ---- ranks, in assignment order (chunks of 256 assignments)
  for (int64_t c0 = a0; c0 < a1; c0 += DTHREADS) {
    const int64_t a = c0 + tid;
    int rank_w = 0;
    for (int ee = 0; ee < E; ++ee) {
      const uint64_t m = __ballot(e == ee);
      if (e == ee) rank_w = __popcll(m & lt_mask);
      if (lane == 0) wave_cnt[wave][ee] = __popcll(m);
    }
    __syncthreads();
    if (valid) {
      int row = -1;
      if (e >= 0) {
        int r = running[e] + rank_w;
        for (int w = 0; w < wave; ++w) r += wave_cnt[w][e];
        const int64_t g = (int64_t)base_l[e] + r;
        if (capacity <= 0 || g < capacity) {
          row = off_l[e] + (int)g;
          row_token[row] = (int32_t)(a / k);
        }
      }
      slot_row[a] = row;
      slot_w[a] = wv;
    }
    // the next chunk's ids and weights
    valid = a + DTHREADS < a1;
    e = valid ? load_expert(idx, a + DTHREADS, E) : -1;
    wv = valid ? load_w(a + DTHREADS) : 0.0f;
    __syncthreads();
    if (tid < E) {
      int s = 0;
      for (int w = 0; w < DTHREADS / 64; ++w) s += wave_cnt[w][tid];
      running[tid] += s;
    }
    __syncthreads();
  }

}

// bf16 rows of the materialising dispatch: one wave per token reads the token's row
// once (ROW_REGS 16-byte vectors per lane at a time, all in flight together) and
// writes it to each of its kept permuted rows (slot_row of its k assignments).  A
// separate launch of T/4 workgroups keeps far more bytes in flight than a copy inside
// the table kernel's 64-token blocks.
__global__ __launch_bounds__(256) void scatter_rows_kernel(const uint16_t* __restrict__ x,
                                                           const int32_t* __restrict__ row_index, int64_t T, int d,
                                                           int k, const int32_t* __restrict__ slot_row,
                                                           uint16_t* __restrict__ xperm) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  int rows[8];
  bool any = false;
  for (int j = 0; j < k; ++j) {
    rows[j] = slot_row[t * k + j];
    any |= rows[j] >= 0;
  }
  if (!any) return;  // every assignment of the token was dropped
  const int nvec = d / 8;
  const int64_t xr = row_index ? (int64_t)row_index[t] : t;
  const i32x4_t* src = reinterpret_cast<const i32x4_t*>(x + xr * (int64_t)d);
  for (int v0 = 0; v0 < nvec; v0 += 64 * ROW_REGS) {
    i32x4_t r[ROW_REGS];
#pragma unroll
    for (int i = 0; i < ROW_REGS; ++i) {
      const int v = v0 + lane + 64 * i;
      if (v < nvec) r[i] = src[v];
    }
    for (int j = 0; j < k; ++j) {
      if (rows[j] < 0) continue;
      i32x4_t* dst = reinterpret_cast<i32x4_t*>(xperm + (int64_t)rows[j] * d);
#pragma unroll
      for (int i = 0; i < ROW_REGS; ++i) {
        const int v = v0 + lane + 64 * i;
        // non-temporal: the permuted rows are read back only by the backward's weight
        // gradient, long after this; x itself stays cached for the gate/up GEMM
        if (v < nvec) __builtin_nontemporal_store(r[i], dst + v);
      }
    }
  }
}

// fp8 rows of the dispatch: one wave per token quantises the token's row once
// (register-resident, per-token scale amax/448) and writes it to the token's kept
// permuted rows (slot_row of its k assignments), with their scales.
__global__ __launch_bounds__(256) void quant_scatter_kernel(const uint16_t* __restrict__ x,
                                                            const int32_t* __restrict__ row_index, int64_t T,
                                                            int d, int k, const int32_t* __restrict__ slot_row,
                                                            uint8_t* __restrict__ xperm,
                                                            float* __restrict__ xperm_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  int rows[8];
  bool any = false;
  for (int j = 0; j < k; ++j) {
    rows[j] = slot_row[t * k + j];
    any |= rows[j] >= 0;
  }
  if (!any) return;  // every assignment of the token was dropped
  const int nvec = d / 8;
  const int64_t xr = row_index ? (int64_t)row_index[t] : t;
  RowRegs r;
  const float amax = load_row_amax(reinterpret_cast<const i32x4_t*>(x + xr * (int64_t)d), nvec, lane, r);
  const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
  uint32_t q[2 * ROW_REGS];
#pragma unroll
  for (int i = 0; i < ROW_REGS; ++i)
    if (lane + 64 * i < nvec) quant_vec_e4m3(r.v[i], inv, q[2 * i], q[2 * i + 1]);
  for (int j = 0; j < k; ++j) {
    if (rows[j] < 0) continue;
    uint32_t* dst = reinterpret_cast<uint32_t*>(xperm + (int64_t)rows[j] * d);
#pragma unroll
    for (int i = 0; i < ROW_REGS; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) *reinterpret_cast<uint2*>(dst + 2 * v) = make_uint2(q[2 * i], q[2 * i + 1]);
    }
    if (lane == 0) xperm_scale[rows[j]] = amax / 448.0f;
  }
}

template <bool FP8>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ x,
                                                          const int32_t* __restrict__ row_token, int64_t n_rows,
                                                          const int32_t* __restrict__ n_rows_dev, int d,
                                                          void* __restrict__ out, float* __restrict__ out_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int64_t nr = n_rows;
  if (n_rows_dev) nr = min<int64_t>(nr, (int64_t)*n_rows_dev);
  if (r >= nr) return;
  const int nvec = d / 8;
  const int32_t tok = row_token[r];
  if (!FP8) {
    i32x4_t* dst = reinterpret_cast<i32x4_t*>(static_cast<uint16_t*>(out) + r * d);
    if (tok < 0) {
      const i32x4_t z = {0, 0, 0, 0};
      for (int v = lane; v < nvec; v += 64) dst[v] = z;
      return;
    }
    const i32x4_t* src = reinterpret_cast<const i32x4_t*>(x + (int64_t)tok * d);
    for (int v = lane; v < nvec; v += 64) dst[v] = src[v];
  } else {
    uint32_t* dst = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(out) + r * d);
    if (tok < 0) {
      for (int v = lane; v < nvec; v += 64) {
        dst[2 * v] = 0u;
        dst[2 * v + 1] = 0u;
      }
      if (lane == 0) out_scale[r] = 0.0f;
      return;
    }
    const i32x4_t* src = reinterpret_cast<const i32x4_t*>(x + (int64_t)tok * d);
    RowRegs rr;  // d <= 64 * 8 * ROW_REGS (checked on the host)
    const float amax = load_row_amax(src, nvec, lane, rr);
    const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
#pragma unroll
    for (int i = 0; i < ROW_REGS; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) {
        uint32_t lo, hi;
        quant_vec_e4m3(rr.v[i], inv, lo, hi);
        *reinterpret_cast<uint2*>(dst + 2 * v) = make_uint2(lo, hi);
      }
    }
    if (lane == 0) out_scale[r] = amax / 448.0f;
  }
}

}  // namespace

extern "C" size_t kmoe_dispatch_workspace_bytes(int64_t T, int k, int E) {
  (void)k;
  const int64_t nblk = kmoe::ceil_div<int64_t>(T, DTB);
  return (size_t)(2 * nblk * E) * sizeof(int32_t) + 256;
}

namespace {

// Argument checks shared by kmoe_dispatch and kmoe_dispatch_noalloc.
int check_dispatch_args(const char* who, const void* x, int64_t T, int d, const int64_t* topk_idx,
                        const void* topk_w, int w_dtype, int k, int E, int32_t* counts, int32_t* offsets,
                        int32_t* row_token, int32_t* slot_row, float* slot_w, void* xperm, int xperm_dtype,
                        float* xperm_scale) {
  KMOE_REQUIRE(x && topk_idx && topk_w && counts && offsets && row_token && slot_row && slot_w &&
                   (xperm || xperm_dtype == KMOE_DTYPE_BF16),
               KMOE_ERR_NULL, "%s: null buffer", who);
  KMOE_REQUIRE(T >= 0 && T * (int64_t)k < ((int64_t)1 << 31), KMOE_ERR_SHAPE, "%s: T*k must fit in int32", who);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "%s: d=%d must be a positive multiple of 64", who, d);
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "%s: E=%d out of range", who, E);
  KMOE_REQUIRE(k >= 1 && k <= 8 && k <= E, KMOE_ERR_SHAPE, "%s: k=%d not in [1, min(8,E)]", who, k);
  KMOE_REQUIRE(w_dtype == KMOE_DTYPE_BF16 || w_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "%s: topk_w dtype must be bf16 or f32", who);
  KMOE_REQUIRE(xperm_dtype == KMOE_DTYPE_BF16 || xperm_dtype == KMOE_DTYPE_FP8_E4M3, KMOE_ERR_DTYPE,
               "%s: xperm dtype must be bf16 or fp8_e4m3", who);
  KMOE_REQUIRE(xperm_dtype != KMOE_DTYPE_FP8_E4M3 || xperm_scale, KMOE_ERR_NULL, "%s: fp8 output needs xperm_scale",
               who);
  KMOE_REQUIRE(xperm_dtype != KMOE_DTYPE_FP8_E4M3 || d <= 64 * 8 * ROW_REGS, KMOE_ERR_UNSUPPORTED,
               "%s: fp8 rows need d <= %d (d=%d)", who, 64 * 8 * ROW_REGS, d);
  return KMOE_OK;
}

// The launches of a dispatch whose per-block histograms and bases live in `workspace`
// (at least kmoe_dispatch_workspace_bytes(T, k, E) bytes).  Every workspace entry a
// launch reads is written by an earlier launch of the same call (hist_kernel writes all
// nblk*E counts, the scan writes all bases), so nothing needs to start at zero.
int dispatch_launch(const void* x, const int32_t* row_index, int64_t T, int d, const int64_t* topk_idx,
                    const void* topk_w, int w_dtype, int k, int E, int64_t capacity, int32_t* counts,
                    int32_t* offsets, int32_t* row_token, int32_t* slot_row, float* slot_w, void* xperm,
                    int xperm_dtype, float* xperm_scale, void* workspace, hipStream_t s,
                    const int32_t* given_counts = nullptr, const float* aux_partials = nullptr, float w_lb = 0.0f,
                    float w_z = 0.0f, float* aux_out = nullptr) {
  const int64_t nblk = kmoe::ceil_div<int64_t>(T, DTB);
  int32_t* ws_counts = static_cast<int32_t*>(workspace);
  int32_t* block_base = ws_counts + nblk * E;
  // the per-block histograms: given (kmoe_router_hist wrote them, one row per router
  // workgroup of kmoe::router_block_tokens(T) tokens) or counted here per DTB tokens
  const int32_t* block_counts = given_counts ? given_counts : ws_counts;
  const int hb = given_counts ? kmoe::router_block_tokens(T) : DTB;
  const int64_t nhb = kmoe::ceil_div<int64_t>(T, hb);
  const int hper = DTB / hb;
  if (T == 0) {
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, s, block_counts, (int64_t)0, E, capacity, block_base,
                       counts, offsets);
    return kmoe::check_launch("kmoe_dispatch(scan)");
  }
  // the auxiliary losses ride on the permute launch when it sums the block counts itself
  const bool aux_fused = aux_out && nblk <= FUSED_SCAN_MAX_BLOCKS;
  if (!given_counts)
    hipLaunchKernelGGL(hist_kernel, dim3((unsigned)nblk), dim3(DTHREADS), 0, s, topk_idx, T, k, E, ws_counts);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const bool fp8 = xperm_dtype == KMOE_DTYPE_FP8_E4M3;
  if (nblk <= FUSED_SCAN_MAX_BLOCKS) {
    hipLaunchKernelGGL(permute_kernel<true>, dim3((unsigned)(nblk + (aux_fused ? 1 : 0))), dim3(DTHREADS), 0, s, xp,
                       row_index, T, d, topk_idx, topk_w, w_dtype, k, E, capacity, block_counts, nblk, nhb, hper,
                       block_base, counts, offsets, row_token, slot_row, slot_w, aux_partials, w_lb, w_z,
                       aux_fused ? aux_out : nullptr);
  } else {
    // the scan path reads one histogram row per DTB-token block
    KMOE_REQUIRE(hper == 1, KMOE_ERR_UNSUPPORTED, "kmoe_dispatch: %d-token histograms over %lld tokens", hb,
                 (long long)T);
    hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, s, block_counts, nblk, E, capacity, block_base, counts,
                       offsets);
    hipLaunchKernelGGL(permute_kernel<false>, dim3((unsigned)nblk), dim3(DTHREADS), 0, s, xp, row_index, T, d,
                       topk_idx, topk_w, w_dtype, k, E, capacity, block_counts, nblk, nblk, 1, block_base, counts,
                       offsets, row_token, slot_row, slot_w, nullptr, 0.0f, 0.0f, nullptr);
  }
  if (aux_out && !aux_fused) {
    const int rc = kmoe_aux_loss(aux_partials, T, E, counts, k, w_lb, w_z, aux_out, s);
    if (rc) return rc;
  }
  const dim3 rows_grid((unsigned)kmoe::ceil_div<int64_t>(T, 4));
  if (fp8)
    hipLaunchKernelGGL(quant_scatter_kernel, rows_grid, dim3(256), 0, s, xp, row_index, T, d, k, slot_row,
                       static_cast<uint8_t*>(xperm), xperm_scale);
  else if (xperm)
    hipLaunchKernelGGL(scatter_rows_kernel, rows_grid, dim3(256), 0, s, xp, row_index, T, d, k, slot_row,
                       static_cast<uint16_t*>(xperm));
  return kmoe::check_launch("kmoe_dispatch");
}

// ---- allocation-free dispatch: its workspace is this file-scope device array.  Host
// code never passes `scratch` itself to a kernel (on the host the name is a stand-in,
// not a device address); it passes the address hipGetSymbolAddress returns for the
// current device, looked up once per device on the first call there.
static __device__ __align__(256) uint8_t scratch[KMOE_DISPATCH_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  KMOE_REQUIRE(e == hipSuccess, KMOE_ERR_LAUNCH, "kmoe_dispatch_noalloc: hipGetDevice failed: %s",
               hipGetErrorString(e));
  KMOE_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, KMOE_ERR_UNSUPPORTED,
               "kmoe_dispatch_noalloc: device %d beyond the %d supported", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    KMOE_REQUIRE(e == hipSuccess && p != nullptr, KMOE_ERR_LAUNCH,
                 "kmoe_dispatch_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                 hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KMOE_OK;
}

}  // namespace

extern "C" int kmoe_dispatch(const void* x, const int32_t* row_index, int64_t T, int d, const int64_t* topk_idx,
                             const void* topk_w, int w_dtype, int k, int E, int64_t capacity, int32_t* counts,
                             int32_t* offsets, int32_t* row_token, int32_t* slot_row, float* slot_w, void* xperm,
                             int xperm_dtype, float* xperm_scale, void* workspace, size_t workspace_bytes,
                             void* stream) {
  int rc = check_dispatch_args("kmoe_dispatch", x, T, d, topk_idx, topk_w, w_dtype, k, E, counts, offsets,
                               row_token, slot_row, slot_w, xperm, xperm_dtype, xperm_scale);
  if (rc) return rc;
  const size_t need = kmoe_dispatch_workspace_bytes(T, k, E);
  KMOE_REQUIRE(workspace && workspace_bytes >= need, KMOE_ERR_WORKSPACE,
               "kmoe_dispatch: workspace %zu < %zu bytes", workspace_bytes, need);
  return dispatch_launch(x, row_index, T, d, topk_idx, topk_w, w_dtype, k, E, capacity, counts, offsets, row_token,
                         slot_row, slot_w, xperm, xperm_dtype, xperm_scale, workspace, kmoe::as_stream(stream));
}

extern "C" int kmoe_dispatch_counted(const void* x, const int32_t* row_index, int64_t T, int d,
                                     const int64_t* topk_idx, const void* topk_w, int w_dtype, int k, int E,
                                     int64_t capacity, const int32_t* block_counts, int32_t* counts, int32_t* offsets,
                                     int32_t* row_token, int32_t* slot_row, float* slot_w, void* xperm,
                                     int xperm_dtype, float* xperm_scale, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  int rc = check_dispatch_args("kmoe_dispatch_counted", x, T, d, topk_idx, topk_w, w_dtype, k, E, counts, offsets,
                               row_token, slot_row, slot_w, xperm, xperm_dtype, xperm_scale);
  if (rc) return rc;
  KMOE_REQUIRE(block_counts, KMOE_ERR_NULL, "kmoe_dispatch_counted: null block_counts");
  const size_t need = kmoe_dispatch_workspace_bytes(T, k, E);
  KMOE_REQUIRE(workspace && workspace_bytes >= need, KMOE_ERR_WORKSPACE,
               "kmoe_dispatch_counted: workspace %zu < %zu bytes", workspace_bytes, need);
  return dispatch_launch(x, row_index, T, d, topk_idx, topk_w, w_dtype, k, E, capacity, counts, offsets, row_token,
                         slot_row, slot_w, xperm, xperm_dtype, xperm_scale, workspace, kmoe::as_stream(stream),
                         block_counts);
}

extern "C" int kmoe_dispatch_counted_aux(const void* x, const int32_t* row_index, int64_t T, int d,
                                         const int64_t* topk_idx, const void* topk_w, int w_dtype, int k, int E,
                                         int64_t capacity, const int32_t* block_counts, int32_t* counts,
                                         int32_t* offsets, int32_t* row_token, int32_t* slot_row, float* slot_w,
                                         void* xperm, int xperm_dtype, float* xperm_scale, void* workspace,
                                         size_t workspace_bytes, const float* partials, float w_lb, float w_z,
                                         float* aux_out, void* stream) {
  int rc = check_dispatch_args("kmoe_dispatch_counted_aux", x, T, d, topk_idx, topk_w, w_dtype, k, E, counts,
                               offsets, row_token, slot_row, slot_w, xperm, xperm_dtype, xperm_scale);
  if (rc) return rc;
  KMOE_REQUIRE(block_counts && partials && aux_out, KMOE_ERR_NULL,
               "kmoe_dispatch_counted_aux: null block_counts / partials / aux_out");
  KMOE_REQUIRE(T > 0, KMOE_ERR_SHAPE, "kmoe_dispatch_counted_aux: T must be > 0 (the losses average over tokens)");
  const size_t need = kmoe_dispatch_workspace_bytes(T, k, E);
  KMOE_REQUIRE(workspace && workspace_bytes >= need, KMOE_ERR_WORKSPACE,
               "kmoe_dispatch_counted_aux: workspace %zu < %zu bytes", workspace_bytes, need);
  return dispatch_launch(x, row_index, T, d, topk_idx, topk_w, w_dtype, k, E, capacity, counts, offsets, row_token,
                         slot_row, slot_w, xperm, xperm_dtype, xperm_scale, workspace, kmoe::as_stream(stream),
                         block_counts, partials, w_lb, w_z, aux_out);
}

extern "C" int kmoe_dispatch_noalloc(const void* x, const int32_t* row_index, int64_t T, int d,
                                     const int64_t* topk_idx, const void* topk_w, int w_dtype, int k, int E,
                                     int64_t capacity, int32_t* counts, int32_t* offsets, int32_t* row_token,
                                     int32_t* slot_row, float* slot_w, void* xperm, int xperm_dtype,
                                     float* xperm_scale, void* stream) {
  int rc = check_dispatch_args("kmoe_dispatch_noalloc", x, T, d, topk_idx, topk_w, w_dtype, k, E, counts, offsets,
                               row_token, slot_row, slot_w, xperm, xperm_dtype, xperm_scale);
  if (rc) return rc;
  const size_t need = kmoe_dispatch_workspace_bytes(T, k, E);
  KMOE_REQUIRE(need <= (size_t)KMOE_DISPATCH_SCRATCH_BYTES, KMOE_ERR_WORKSPACE,
               "kmoe_dispatch_noalloc: T=%lld, E=%d needs %zu bytes of scratch, more than the %zu it has "
               "(use kmoe_dispatch with a workspace)",
               (long long)T, E, need, (size_t)KMOE_DISPATCH_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return dispatch_launch(x, row_index, T, d, topk_idx, topk_w, w_dtype, k, E, capacity, counts, offsets, row_token,
                         slot_row, slot_w, xperm, xperm_dtype, xperm_scale, ws, kmoe::as_stream(stream));
}

extern "C" int kmoe_gather_rows(const void* x, const int32_t* row_token, int64_t n_rows, const int32_t* n_rows_dev,
                                int d, void* out, int out_dtype, float* out_scale, void* stream) {
  KMOE_REQUIRE(x && row_token && out, KMOE_ERR_NULL, "kmoe_gather_rows: null buffer");
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "kmoe_gather_rows: d=%d must be a positive multiple of 64", d);
  KMOE_REQUIRE(n_rows >= 0, KMOE_ERR_SHAPE, "kmoe_gather_rows: n_rows < 0");
  KMOE_REQUIRE(out_dtype == KMOE_DTYPE_BF16 || out_dtype == KMOE_DTYPE_FP8_E4M3, KMOE_ERR_DTYPE,
               "kmoe_gather_rows: out dtype must be bf16 or fp8_e4m3");
  KMOE_REQUIRE(out_dtype != KMOE_DTYPE_FP8_E4M3 || out_scale, KMOE_ERR_NULL, "kmoe_gather_rows: fp8 needs out_scale");
  KMOE_REQUIRE(out_dtype != KMOE_DTYPE_FP8_E4M3 || d <= 64 * 8 * ROW_REGS, KMOE_ERR_UNSUPPORTED,
               "kmoe_gather_rows: fp8 rows need d <= %d (d=%d)", 64 * 8 * ROW_REGS, d);
  if (n_rows == 0) return KMOE_OK;
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(n_rows, 4));
  hipStream_t s = kmoe::as_stream(stream);
  if (out_dtype == KMOE_DTYPE_BF16)
    hipLaunchKernelGGL(gather_rows_kernel<false>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x), row_token,
                       n_rows, n_rows_dev, d, out, out_scale);
  else
    hipLaunchKernelGGL(gather_rows_kernel<true>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x), row_token,
                       n_rows, n_rows_dev, d, out, out_scale);
  return kmoe::check_launch("kmoe_gather_rows");
}
