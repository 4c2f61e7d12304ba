// Router: logits = SiLU(x . w_in^T) . w_out^T (+ bias), softmax, top-k, aux partials.
// Follows Router.forward (moe_arch/model/moe.py:423-462) and the loss inputs of
// MoELayer._compute_load_balance_loss / _compute_router_z_loss (moe.py:872-939).
//
// Layout: one workgroup = 4 waves = 64 tokens.  The d -> 128 layer runs on
// v_mfma_f32_32x32x16_bf16 (each wave: 32 tokens x 64 hidden units) over a K
// pipeline of as many stages as fit in LDS (K-steps of 128 or 256 bytes per row):
// x rows and w_in rows go global -> LDS directly (global_load_lds), so all but one
// stage are in flight while one is computed.  The hidden activations go through LDS
// (fp32) to the 128 -> E layer, which runs in fp32 on v_mfma_f32_16x16x4_f32 (each
// wave: 16 tokens x all experts); softmax/top-k then run four lanes per token (each
// with a quarter of the experts' logits in registers, merged by DPP moves inside the
// quad), the logits leave through a coalesced all-thread copy and each aux partial is
// one thread's fixed-order column sum.
#include "kmoe_common.h"

namespace {

constexpr int RT_TOK = 64;        // tokens per workgroup (32 on small grids: kmoe::router_block_tokens)
constexpr int RT_THREADS = 256;   // 4 waves: 2 (token halves) x 2 (hidden halves); 32-token tiles: 4 hidden quarters
constexpr int RT_HID = KMOE_ROUTER_HIDDEN;
// padded LDS row strides (floats) of the hidden tile and of w_out: 2 mod 32, so the 32
// lanes (row i, k) of a 16x16x4 MFMA operand read (banks 2i + k) are conflict free
constexpr int HSTR = RT_HID + 2;
constexpr int WOS = RT_HID + 2;
// One K-step covers RKB bytes of every row (RKB = 128 or 256: 64 or 128 bf16); TOK
// tokens per workgroup (64, or 32 on small grids: kmoe::router_block_tokens).
template <int RKB, int TOK = RT_TOK>
struct RtGeom {
  static constexpr int XT = TOK * RKB;         // x tile of one K-step (TOK rows)
  static constexpr int WT = RT_HID * RKB;      // w_in tile of one K-step (128 rows)
  static constexpr int STAGE = XT + WT;
  static constexpr int RPB = 1024 / RKB;       // rows per 1 KiB load block
  static constexpr int CPR = RKB / 16;         // 16-byte chunks per row
  static constexpr int XBLK = TOK / RPB / 4;   // x load blocks per wave per K-step
  static constexpr int WBLK = RT_HID / RPB / 4;  // w_in load blocks per wave per K-step
  static constexpr int LOADS = XBLK + WBLK;    // direct-to-LDS instructions per wave per K-step
  // Byte offset of 16-byte chunk `chunk` of row `row`: the XOR spreads the 16 lanes
  // of each LDS read pass (16 consecutive rows, one chunk) over distinct banks.
  __device__ static __forceinline__ int swz(int row, int chunk) {
    return row * RKB + ((chunk ^ (RKB == 128 ? ((row >> 1) & 7) : (row & 15))) << 4);
  }
};
// K pipeline depth: as many stages as fit beside w_out (NE rows, at least 16, of WOS
// fp32), the block's expert counts and the RMS scales
template <int NE, int RKB, int TOK = RT_TOK>
constexpr int rt_stages() {
  return (160 * 1024 - (NE < 16 ? 16 : NE) * WOS * 4 - NE * 4 - RT_TOK * 4) / RtGeom<RKB, TOK>::STAGE;
}

// RMS: the router input is RMSNorm(x) (embeddings.py:167-195) with the norm weight
// already folded into w_in's columns; the kernel sums x^2 over the K loop from the
// x fragments it reads anyway, scales each token's hidden pre-activation by
// r = 1/sqrt(mean(x^2) + eps) (the scale commutes with the d -> 128 product) and
// writes r to rscale for the expert GEMM.
// TOK = 32 (when all 32-token workgroups fit the device at once): each wave computes
// all 32 tokens x a quarter of the hidden units, and the epilogue's layer 2, softmax,
// top-k and per-block outputs run on the first 32 token slots.
template <int NE, int RKB, bool RMS = false, int TOK = RT_TOK>
__global__ __launch_bounds__(RT_THREADS) void router_kernel(const uint16_t* __restrict__ x,
                                                            const int32_t* __restrict__ row_index, int64_t T, int d,
                                                            const uint16_t* __restrict__ w_in,
                                                            const uint16_t* __restrict__ w_out, int E,
                                                            const float* __restrict__ bias, int k,
                                                            float* __restrict__ logits, int64_t* __restrict__ topk_idx,
                                                            float* __restrict__ topk_w, float* __restrict__ partials,
                                                            float* __restrict__ hidden_pre, float eps,
                                                            float* __restrict__ rscale,
                                                            int32_t* __restrict__ block_counts) {
  using G = RtGeom<RKB, TOK>;
  constexpr int RT_STAGES = rt_stages<NE, RKB, TOK>();
  constexpr int NH = TOK == 64 ? 2 : 1;  // 32-wide hidden blocks per wave
  static_assert(TOK == 64 || TOK == 32, "token tile");
  constexpr int RT_STAGE = G::STAGE;
  static_assert(RT_STAGES >= 2, "K pipeline");
  static_assert(RT_STAGES * RT_STAGE >= (RT_TOK * HSTR + 2 * RT_TOK * (NE + 4) + RT_TOK) * 4,
                "the epilogue's hidden / logit / probability tiles reuse the stages");
  constexpr int NEP = NE < 16 ? 16 : NE;  // experts padded to whole 16-wide MFMA blocks
  constexpr int LGS = NE + 4;             // logits / probabilities row stride (floats), 16-byte aligned rows
  __shared__ __attribute__((aligned(1024))) uint8_t smem[RT_STAGES * RT_STAGE];
  __shared__ __attribute__((aligned(16))) float wo[NEP * WOS];  // w_out as fp32 (rows >= E: 0)
  __shared__ float rs_l[RMS ? RT_TOK : 1];                      // per-token RMSNorm scale
  __shared__ int cnt_l[NE];                                     // the block's per-expert routed counts
  // after the K loop smem holds: hs[64][HSTR], lg[64][LGS], pe[64][LGS], lse2[64]
  float* hs = reinterpret_cast<float*>(smem);
  float* lg = hs + RT_TOK * HSTR;  // 64 * 130 floats = 33280 bytes: lg rows stay 16-byte aligned
  float* pe = lg + RT_TOK * LGS;
  float* lse2 = pe + RT_TOK * LGS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  // wave (wm, wn): tokens wm*32 .. +31, hidden units wn*32*NH .. +32*NH-1
  const int wm = TOK == 64 ? (wave & 1) : 0, wn = TOK == 64 ? (wave >> 1) : wave;
  const int64_t tok0 = (int64_t)blockIdx.x * TOK;

  // ---- per-lane sources of the direct-to-LDS loads (block q fills tile rows
  // [RPB q, RPB q + RPB), lane l lands at byte 16*l of the block: row RPB q + l/CPR,
  // physical chunk l%CPR, holding the logical chunk that swz() maps there)
  const int rsub = lane / G::CPR, pc = lane % G::CPR;
  auto chunk_of = [&](int tr) { return (G::swz(tr, pc) - tr * RKB); };
  // fixed sizes (the largest geometry): a template-dependent local array size keeps
  // hipcc from emitting the kernel's host launch stub
  static_assert(G::XBLK <= 4 && G::WBLK <= 8, "load blocks per wave");
  const uint8_t* xsrc[4];
  uint32_t wsrc[8];
#pragma unroll
  for (int q = 0; q < G::XBLK; ++q) {
    const int tr = (wave * G::XBLK + q) * G::RPB + rsub;
    int64_t t = tok0 + tr;
    t = t < T ? t : T - 1;
    const int64_t xr = row_index ? (int64_t)row_index[t] : t;
    xsrc[q] = reinterpret_cast<const uint8_t*>(x) + xr * (int64_t)d * 2 + chunk_of(tr);
  }
#pragma unroll
  for (int q = 0; q < G::WBLK; ++q) {
    const int tr = (wave * G::WBLK + q) * G::RPB + rsub;
    wsrc[q] = (uint32_t)tr * (uint32_t)d * 2u + (uint32_t)chunk_of(tr);
  }
  const uint8_t* wbase = reinterpret_cast<const uint8_t*>(w_in);
  // Workgroups walk K from different starting steps (the 64-token block index mod the
  // step count): with every workgroup at the same K offset of 4 KiB-strided rows at
  // once, the loads concentrate on a few memory channels (measured: 22% slower
  // cold-cache).  The sum order over K then depends on the token's 64-token block,
  // deterministically and the same for both tile sizes.
  const int nk_all = d * 2 / RKB;
  const int k_rot = (int)((uint64_t)(tok0 / RT_TOK) % (uint64_t)nk_all);
  auto issue = [&](int kt) {
    uint8_t* st = smem + (kt % RT_STAGES) * RT_STAGE;
    const int kr = kt + k_rot;
    const int kb = (kr < nk_all ? kr : kr - nk_all) * RKB;
#pragma unroll
    for (int q = 0; q < G::XBLK; ++q)
      dma16_to_lds(xsrc[q] + kb, (KMOE_LDS void*)(st + (wave * G::XBLK + q) * 1024));
#pragma unroll
    for (int q = 0; q < G::WBLK; ++q)
      dma16_to_lds(wbase + wsrc[q] + kb, (KMOE_LDS void*)(st + G::XT + (wave * G::WBLK + q) * 1024));
  };

  // ---- layer 1 on MFMA: wave (wm, wn) computes 32 tokens x 32*NH hidden; the next
  // substep's fragments are read before the current substep's MFMAs
  f32x16_t acc[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  const int nk = d * 2 / RKB;
  float ss = 0.0f;  // RMS: this lane's part of sum(x^2) of token wm*32 + lr
  for (int s = 0; s < RT_STAGES - 1 && s < nk; ++s) issue(s);
  // w_out (needed only by layer 2) goes out behind the first K-steps, one 16-byte load
  // per thread and vector (rows past E read as zero), and reaches LDS after the K loop:
  // loaded before the K-steps its round trip delayed every x load, and as 2-byte loads
  // in a loop it cost 8 dependent round trips (~3.5 us) before the first K-step
  constexpr int WOV = NEP * RT_HID / 8;  // 16-byte vectors of the padded w_out
  constexpr int WOQ = (WOV + RT_THREADS - 1) / RT_THREADS;
  const bool wo_vec = (reinterpret_cast<uintptr_t>(w_out) & 15) == 0;
  i32x4_t wov[WOQ];
  if (wo_vec) {
#pragma unroll
    for (int q = 0; q < WOQ; ++q) {
      const int v = tid + q * RT_THREADS;
      wov[q] = (v < WOV && v / (RT_HID / 8) < E) ? reinterpret_cast<const i32x4_t*>(w_out)[v]
                                                   : i32x4_t{0, 0, 0, 0};
    }
  } else {
    for (int i = tid; i < NEP * RT_HID; i += RT_THREADS) {
      const int e = i / RT_HID, j = i % RT_HID;
      wo[e * WOS + j] = e < E ? bf16_to_f32(w_out[i]) : 0.0f;
    }
  }
  if (tid < NE) cnt_l[tid] = 0;
  constexpr int NSUB = RKB / 32;  // MFMA K-substeps per K-step
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + RT_STAGES - 2 < nk)
      wait_vmcnt<(RT_STAGES - 2) * G::LOADS>();
    else
      wait_vmcnt<0>();
    barrier_nofence();
    if (kt + RT_STAGES - 1 < nk) issue(kt + RT_STAGES - 1);
    const uint8_t* xt = smem + (kt % RT_STAGES) * RT_STAGE;
    const uint8_t* wt = xt + G::XT;
    bf16x8_t a[2], b0[2], b1[2];
    auto rdf = [&](int i, int buf) {
      const int ch = 2 * i + lh;
      a[buf] = *reinterpret_cast<const bf16x8_t*>(xt + G::swz(wm * 32 + lr, ch));
      b0[buf] = *reinterpret_cast<const bf16x8_t*>(wt + G::swz(wn * 32 * NH + lr, ch));
      if constexpr (NH == 2) b1[buf] = *reinterpret_cast<const bf16x8_t*>(wt + G::swz(wn * 64 + 32 + lr, ch));
    };
    rdf(0, 0);
#pragma unroll
    for (int i = 0; i < NSUB; ++i) {
      if (i + 1 < NSUB) rdf(i + 1, (i + 1) & 1);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i & 1], b0[i & 1], acc[0], 0, 0, 0);
      if constexpr (NH == 2) acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i & 1], b1[i & 1], acc[1], 0, 0, 0);
      if constexpr (RMS) {
        // the waves of a token half (all four with 32-token tiles) read the same x
        // fragments: one of them sums
        if (wn == 0) {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const float v = (float)a[i & 1][c];
            ss = fmaf(v, v, ss);
          }
        }
      }
    }
  }
  if constexpr (RMS) {
    // lanes lr and lr + 32 hold the two K halves (chunk parity) of token wm*32 + lr
    ss += __shfl_xor(ss, 32, 64);
    if (wn == 0 && lh == 0) {
      const float r = 1.0f / sqrtf(ss / (float)d + eps);
      rs_l[wm * 32 + lr] = r;
      if (tok0 + wm * 32 + lr < T) rscale[tok0 + wm * 32 + lr] = r;
    }
  }
  if (wo_vec) {
#pragma unroll
    for (int q = 0; q < WOQ; ++q) {
      const int v = tid + q * RT_THREADS;
      if (v < WOV) {
        float* dst = wo + (v / (RT_HID / 8)) * WOS + (v % (RT_HID / 8)) * 8;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t pr = (uint32_t)wov[q][c];
          dst[2 * c] = __uint_as_float(pr << 16);
          dst[2 * c + 1] = __uint_as_float(pr & 0xffff0000u);
        }
      }
    }
  }
  __syncthreads();  // stage buffers are reused below

  // SiLU, then to LDS: acc[j][r] is hidden wn*32*NH+j*32+lr of token wm*32+8*(r/4)+4*lh+r%4
  // (training: the pre-activation is also kept for the backward)
#pragma unroll
  for (int j = 0; j < NH; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = wm * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
      const int hcol = wn * 32 * NH + j * 32 + lr;
      const float pre = RMS ? acc[j][r] * rs_l[m] : acc[j][r];
      hs[m * HSTR + hcol] = silu_fast_f32(pre);
      if (hidden_pre && tok0 + m < T) hidden_pre[(tok0 + m) * RT_HID + hcol] = pre;
    }
  __syncthreads();

  // ---- layer 2 on v_mfma_f32_16x16x4_f32 (fp32 operands): wave w computes tokens
  // [16w, 16w + 16) x every 16-expert block; operand lane l holds row l%16 at k = l/16,
  // result register r of lane l is (token 4(l/16) + r, expert l%16)
  if (wave * 16 < TOK) {
    constexpr int NEB = NEP / 16;
    const int i16 = lane & 15, k4 = lane >> 4;
    f32x4_t l2[NEB];
#pragma unroll
    for (int eb = 0; eb < NEB; ++eb) l2[eb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const float* ha = hs + (wave * 16 + i16) * HSTR + k4;
    const float* wb = wo + i16 * WOS + k4;
#pragma unroll 8
    for (int st = 0; st < RT_HID / 4; ++st) {
      const float av = ha[4 * st];
#pragma unroll
      for (int eb = 0; eb < NEB; ++eb)
        l2[eb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wb[eb * 16 * WOS + 4 * st], l2[eb], 0, 0, 0);
    }
#pragma unroll
    for (int eb = 0; eb < NEB; ++eb) {
      const int e = eb * 16 + i16;
      if (e < NE) {
        const float be = (e < E && bias) ? bias[e] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) lg[(wave * 16 + 4 * k4 + r) * LGS + e] = e < E ? l2[eb][r] + be : 0.0f;
      }
    }
  }
  __syncthreads();

  // ---- softmax, top-k, outputs: four lanes per token (lane part p holds the logits of
  // experts p + 4q in registers), merged with shuffles inside each group of four
  const int64_t ntok = T - tok0 < TOK ? T - tok0 : TOK;
  {
    constexpr int NQ = NE / 4;
    const int tl = tid >> 2, part = tid & 3;
    const int64_t t = tok0 + tl;
    float L[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) L[q] = lg[tl * LGS + part + 4 * q];
    float* P = pe + tl * LGS;
    if (tl < TOK && t < T) {  // the same for the four lanes of a token
      float mx = -INFINITY;
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        if (part + 4 * q < E) mx = fmaxf(mx, L[q]);
      mx = fmaxf(mx, quad_xor<1>(mx));
      mx = fmaxf(mx, quad_xor<2>(mx));
      float ex[NQ], s = 0.0f;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        ex[q] = part + 4 * q < E ? __expf(L[q] - mx) : 0.0f;
        s += ex[q];
      }
      s += quad_xor<1>(s);
      s += quad_xor<2>(s);
      const float inv_s = 1.0f / s;
#pragma unroll
      for (int q = 0; q < NQ; ++q) P[part + 4 * q] = ex[q] * inv_s;
      if (part == 0) {
        const float lse = mx + __logf(s);
        lse2[tl] = lse * lse;
      }
      if (k > 0) {
        // k rounds: each lane's best untaken expert (strict '>' over ascending q keeps
        // the lower index), then the best of the four (higher logit, or the lower index
        // on equal logits); NaN ranks below every number
        uint32_t taken = 0;
        int sel[8];
        float sev[8];
        float ssum = 0.0f;
        for (int j = 0; j < k; ++j) {
          int bi = -1;
          float bv = -INFINITY;
#pragma unroll
          for (int q = 0; q < NQ; ++q) {
            const float v = L[q] != L[q] ? -INFINITY : L[q];
            if (part + 4 * q < E && !((taken >> q) & 1u) && (bi < 0 || v > bv)) {
              bi = part + 4 * q;
              bv = v;
            }
          }
          auto merge = [&](int oi, float ov) {
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
              bi = oi;
              bv = ov;
            }
          };
          merge(quad_xor<1>(bi), quad_xor<1>(bv));
          merge(quad_xor<2>(bi), quad_xor<2>(bv));
          if ((bi & 3) == part) taken |= 1u << (bi >> 2);
          sel[j] = bi;
          sev[j] = __expf(bv - mx);
          ssum += sev[j];
        }
        if (part == 0) {
          const float inv = 1.0f / ssum;
          for (int j = 0; j < k; ++j) {
            topk_idx[t * k + j] = sel[j];
            topk_w[t * k + j] = sev[j] * inv;
            // the block's per-expert routed counts (the dispatch's histogram of the
            // block's TOK tokens)
            if (block_counts) atomicAdd(&cnt_l[sel[j]], 1);
          }
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < NQ; ++q) P[part + 4 * q] = 0.0f;
      if (part == 0) lse2[tl] = 0.0f;
    }
  }
  __syncthreads();
  if (block_counts && k > 0 && tid < E) block_counts[(int64_t)blockIdx.x * E + tid] = cnt_l[tid];

  // ---- logits out: the block's ntok x E floats are contiguous; coalesced copy
  for (int i = tid; i < ntok * E; i += RT_THREADS) logits[tok0 * E + i] = lg[(i / E) * LGS + i % E];

  // ---- per-block aux partials: column c of the block's TOK tokens (c < E: the
  // probabilities, c == E: lse^2) summed by thread c in a fixed order (four running
  // sums over tokens m = 4i + u, then added u = 0..3)
  if (partials && tid <= E) {
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int m = 0; m < TOK; m += 4)
#pragma unroll
      for (int u = 0; u < 4; ++u) sum[u] += tid < E ? pe[(m + u) * LGS + tid] : lse2[m + u];
    partials[(int64_t)blockIdx.x * (E + 1) + tid] = (sum[0] + sum[1]) + (sum[2] + sum[3]);
  }
}

// One workgroup, 4 waves: the column sums (aux_reduce_cols), then thread 0 forms the
// losses (aux_finish).
__global__ __launch_bounds__(256) void aux_loss_kernel(const float* __restrict__ partials, int64_t nblk, int64_t T,
                                                       int E, const int32_t* __restrict__ counts, int k, float w_lb,
                                                       float w_z, float* __restrict__ out) {
  __shared__ float col[KMOE_MAX_EXPERTS + 1];
  aux_reduce_cols(partials, nblk, E, threadIdx.x >> 6, 4, threadIdx.x & 63, col);
  __syncthreads();
  if (threadIdx.x == 0) aux_finish(col, counts, T, E, k, w_lb, w_z, out);
}

}  // namespace

namespace kmoe {
int router_block_tokens(int64_t T) { return T <= 32 * (int64_t)cu_count() ? 32 : RT_TOK; }
}  // namespace kmoe

extern "C" int kmoe_router_block_tokens(int64_t T) { return kmoe::router_block_tokens(T < 0 ? 0 : T); }

extern "C" int64_t kmoe_router_partials_len(int64_t T, int E) {
  return kmoe::ceil_div<int64_t>(T, kmoe::router_block_tokens(T)) * (int64_t)(E + 1);
}

namespace {
int router_launch(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in, const void* w_out,
                  int E, const float* logit_bias, int k, float* logits, int64_t* topk_idx, float* topk_w,
                  float* partials, float* hidden_pre, float eps, float* rscale, int32_t* block_counts,
                  void* stream) {
  KMOE_REQUIRE(x && w_in && w_out && logits, KMOE_ERR_NULL, "kmoe_router: null x/w_in/w_out/logits");
  KMOE_REQUIRE(T >= 0 && T <= (int64_t)1 << 31, KMOE_ERR_SHAPE, "kmoe_router: T=%lld out of range",
               (long long)T);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "kmoe_router: d=%d must be a positive multiple of 64", d);
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_router: E=%d not in [1,%d]", E,
               KMOE_MAX_EXPERTS);
  KMOE_REQUIRE(k >= 0 && k <= E && k <= 8, KMOE_ERR_SHAPE, "kmoe_router: k=%d not in [0, min(8, E=%d)]", k, E);
  KMOE_REQUIRE(k == 0 || (topk_idx && topk_w), KMOE_ERR_NULL, "kmoe_router: k>0 needs topk_idx and topk_w");
  if (T == 0) return KMOE_OK;
  // 32-token tiles when they all fit the device at once (64-token tiles would leave
  // CUs idle); the aux partials and block histograms are then per 32 tokens
  const int tok = kmoe::router_block_tokens(T);
  const bool tok32 = tok == 32;
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T, tok));
  hipStream_t s = kmoe::as_stream(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wi = static_cast<const uint16_t*>(w_in);
  const uint16_t* wo = static_cast<const uint16_t*>(w_out);
  // wide K-steps (256 bytes of every row, half the barriers) when d allows and at
  // least three stages fit; 128-byte steps otherwise
#define KMOE_ROUTER_LAUNCH3(NE_, RKB_, RMS_)                                                                    \
  do {                                                                                                           \
    if (tok32)                                                                                                   \
      hipLaunchKernelGGL((router_kernel<NE_, RKB_, RMS_, 32>), grid, dim3(RT_THREADS), 0, s, xp, row_index, T, d, \
                         wi, wo, E, logit_bias, k, logits, topk_idx, topk_w, partials, hidden_pre, eps, rscale,   \
                         block_counts);                                                                          \
    else                                                                                                         \
      hipLaunchKernelGGL((router_kernel<NE_, RKB_, RMS_, RT_TOK>), grid, dim3(RT_THREADS), 0, s, xp, row_index, T, \
                         d, wi, wo, E, logit_bias, k, logits, topk_idx, topk_w, partials, hidden_pre, eps, rscale, \
                         block_counts);                                                                          \
  } while (0)
#define KMOE_ROUTER_LAUNCH2(NE_, RMS_)                       \
  do {                                                       \
    if (d % 128 == 0 && rt_stages<NE_, 256>() >= 3)          \
      KMOE_ROUTER_LAUNCH3(NE_, 256, RMS_);                   \
    else                                                     \
      KMOE_ROUTER_LAUNCH3(NE_, 128, RMS_);                   \
  } while (0)
#define KMOE_ROUTER_LAUNCH(NE_)             \
  do {                                      \
    if (rscale)                             \
      KMOE_ROUTER_LAUNCH2(NE_, true);       \
    else                                    \
      KMOE_ROUTER_LAUNCH2(NE_, false);      \
  } while (0)
  if (E <= 8)
    KMOE_ROUTER_LAUNCH(8);
  else if (E <= 16)
    KMOE_ROUTER_LAUNCH(16);
  else if (E <= 32)
    KMOE_ROUTER_LAUNCH(32);
  else
    KMOE_ROUTER_LAUNCH(64);
#undef KMOE_ROUTER_LAUNCH
#undef KMOE_ROUTER_LAUNCH2
#undef KMOE_ROUTER_LAUNCH3
  return kmoe::check_launch("kmoe_router");
}
}  // namespace

extern "C" int kmoe_router_train(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                                 const void* w_out, int E, const float* logit_bias, int k, float* logits,
                                 int64_t* topk_idx, float* topk_w, float* partials, float* hidden_pre, void* stream) {
  return router_launch(x, row_index, T, d, w_in, w_out, E, logit_bias, k, logits, topk_idx, topk_w, partials,
                       hidden_pre, 0.0f, nullptr, nullptr, stream);
}

extern "C" int kmoe_router_hist(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                                const void* w_out, int E, const float* logit_bias, int k, float* logits,
                                int64_t* topk_idx, float* topk_w, float* partials, float* hidden_pre,
                                int32_t* block_counts, void* stream) {
  KMOE_REQUIRE(block_counts && k >= 1, KMOE_ERR_NULL, "kmoe_router_hist: needs block_counts and k >= 1");
  return router_launch(x, row_index, T, d, w_in, w_out, E, logit_bias, k, logits, topk_idx, topk_w, partials,
                       hidden_pre, 0.0f, nullptr, block_counts, stream);
}

extern "C" int kmoe_router_rms(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in_g,
                               const void* w_out, int E, const float* logit_bias, int k, float* logits,
                               int64_t* topk_idx, float* topk_w, float* partials, float eps, float* rscale,
                               void* stream) {
  KMOE_REQUIRE(rscale, KMOE_ERR_NULL, "kmoe_router_rms: null rscale");
  KMOE_REQUIRE(eps >= 0.0f, KMOE_ERR_SHAPE, "kmoe_router_rms: eps must be >= 0");
  return router_launch(x, row_index, T, d, w_in_g, w_out, E, logit_bias, k, logits, topk_idx, topk_w, partials,
                       nullptr, eps, rscale, nullptr, stream);
}

extern "C" int kmoe_router(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                           const void* w_out, int E, const float* logit_bias, int k, float* logits,
                           int64_t* topk_idx, float* topk_w, float* partials, void* stream) {
  return kmoe_router_train(x, row_index, T, d, w_in, w_out, E, logit_bias, k, logits, topk_idx, topk_w, partials,
                           nullptr, stream);
}

// MoD auxiliary router loss (mod.py:141-171) from its logits l (T): weight * the mean
// over t of BCE-with-logits(l_t, y_t), y_t = 1 for the kept rows rows[0, n_keep) and 0
// elsewhere, i.e. weight / T * (sum_t softplus(l_t) - sum_j l[rows[j]]).  One
// workgroup; fixed-order sums (per-thread strided, a wave butterfly, the wave sums in
// order).  Each thread issues U independent loads per round, and softplus takes the
// hardware log of 1 + e (e = exp(-|l|); where 1 + e rounds to 1 the dropped log1p(e)
// is below 6e-8): with single dependent loads and libm's log1pf the one workgroup
// took 11 us for 8192 logits.
__global__ __launch_bounds__(1024) void mod_aux_bce_kernel(const float* __restrict__ l, int64_t T,
                                                           const int32_t* __restrict__ rows, int64_t n_keep,
                                                           float weight, float* __restrict__ out) {
  constexpr int U = 8;
  __shared__ float red[16];
  const int tid = threadIdx.x;
  float acc = 0.0f;
  for (int64_t t0 = tid; t0 < T; t0 += 1024 * U) {
    float v[U];
#pragma unroll
    for (int q = 0; q < U; ++q) v[q] = t0 + 1024 * q < T ? l[t0 + 1024 * q] : 0.0f;
#pragma unroll
    for (int q = 0; q < U; ++q)
      if (t0 + 1024 * q < T) acc += fmaxf(v[q], 0.0f) + __logf(1.0f + __expf(-fabsf(v[q])));  // softplus
  }
  for (int64_t j0 = tid; j0 < n_keep; j0 += 1024 * U) {
    int32_t r[U];
#pragma unroll
    for (int q = 0; q < U; ++q) r[q] = j0 + 1024 * q < n_keep ? rows[j0 + 1024 * q] : -1;
    float v[U];
#pragma unroll
    for (int q = 0; q < U; ++q) v[q] = r[q] >= 0 ? l[r[q]] : 0.0f;
#pragma unroll
    for (int q = 0; q < U; ++q) acc -= v[q];
  }
  // wave sums (xor butterfly), then the 16 wave sums in order
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    float sum = 0.0f;
    for (int w = 0; w < 16; ++w) sum += red[w];
    out[0] = sum * (weight / (float)T);
  }
}

extern "C" int kmoe_mod_aux_bce(const float* logits, int64_t T, const int32_t* rows, int64_t n_keep, float weight,
                                float* out, void* stream) {
  KMOE_REQUIRE(logits && rows && out, KMOE_ERR_NULL, "kmoe_mod_aux_bce: null buffer");
  KMOE_REQUIRE(T > 0 && n_keep >= 0 && n_keep <= T, KMOE_ERR_SHAPE, "kmoe_mod_aux_bce: T=%lld n_keep=%lld",
               (long long)T, (long long)n_keep);
  hipLaunchKernelGGL(mod_aux_bce_kernel, dim3(1), dim3(1024), 0, kmoe::as_stream(stream), logits, T, rows, n_keep,
                     weight, out);
  return kmoe::check_launch("kmoe_mod_aux_bce");
}

extern "C" int kmoe_aux_loss(const float* partials, int64_t T, int E, const int32_t* counts, int k, float w_lb,
                             float w_z, float* out, void* stream) {
  KMOE_REQUIRE(partials && out, KMOE_ERR_NULL, "kmoe_aux_loss: null partials/out");
  KMOE_REQUIRE(T > 0, KMOE_ERR_SHAPE, "kmoe_aux_loss: T must be > 0");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_aux_loss: E=%d out of range", E);
  KMOE_REQUIRE(!counts || k >= 1, KMOE_ERR_SHAPE, "kmoe_aux_loss: k must be >= 1 with counts");
  const int64_t nblk = kmoe::ceil_div<int64_t>(T, kmoe::router_block_tokens(T));
  hipLaunchKernelGGL(aux_loss_kernel, dim3(1), dim3(256), 0, kmoe::as_stream(stream), partials, nblk, T, E,
                     counts, k, w_lb, w_z, out);
  return kmoe::check_launch("kmoe_aux_loss");
}
