// Router: logits = SiLU(x . w_in^T) . w_out^T (+ bias), softmax, top-k, aux partials.
// Follows Router.forward (moe_arch/model/moe.py:423-462) and the loss inputs of
// MoELayer._compute_load_balance_loss / _compute_router_z_loss (moe.py:872-939).
//
// Layout: one workgroup = 2 waves = 64 tokens.  Each wave owns 32 tokens and all
// 128 hidden units: 4 accumulator blocks of v_mfma_f32_32x32x16_bf16.  Operands are
// read straight from global memory (x rows and w_in rows are both K-contiguous);
// within every 64-wide K block lane half h holds elements [32h, 32h+32) of its row,
// a consistent K permutation for A and B that lets each lane issue 64-byte loads.
// The hidden activations go through LDS (fp32) for the 128->E layer, which runs on
// the vector ALUs in fp32; softmax/top-k then run one token per lane.
#include "kmoe_common.h"

namespace {

constexpr int RT_TOK = 64;       // tokens per workgroup
constexpr int RT_HID = KMOE_ROUTER_HIDDEN;
constexpr int HSTR = RT_HID + 1;  // padded LDS row stride (floats) of the hidden tile

template <int NE>
__global__ __launch_bounds__(128) void router_kernel(const uint16_t* __restrict__ x,
                                                     const int32_t* __restrict__ row_index, int64_t T,
                                                     int d, const uint16_t* __restrict__ w_in,
                                                     const uint16_t* __restrict__ w_out, int E,
                                                     const float* __restrict__ bias, int k,
                                                     float* __restrict__ logits, int64_t* __restrict__ topk_idx,
                                                     float* __restrict__ topk_w, float* __restrict__ partials) {
  __shared__ float hs[2][32 * HSTR];     // SiLU(hidden) per wave, fp32
  __shared__ float wo[NE * RT_HID];      // w_out as fp32
  __shared__ float lg[2][32][NE + 1];    // logits per wave
  __shared__ float pe[RT_TOK][NE + 1];   // softmax probabilities (aux partials)
  __shared__ float lse2[RT_TOK];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lr = lane & 31;
  const int lh = lane >> 5;
  const int64_t tok0 = (int64_t)blockIdx.x * RT_TOK + wave * 32;

  for (int i = tid; i < NE * RT_HID; i += blockDim.x) {
    int e = i / RT_HID;
    wo[i] = e < E ? bf16_to_f32(w_out[i]) : 0.0f;
  }

  // ---- layer 1 on MFMA: 32 tokens x 128 hidden, K = d
  int64_t t_a = tok0 + lr;
  if (t_a >= T) t_a = T - 1;
  const int64_t xrow = row_index ? (int64_t)row_index[t_a] : t_a;
  const uint16_t* ap = x + xrow * (int64_t)d + 32 * lh;
  const uint16_t* bp[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) bp[nb] = w_in + (int64_t)(nb * 32 + lr) * d + 32 * lh;

  f32x16_t acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;

  for (int k0 = 0; k0 < d; k0 += 64) {
    bf16x8_t a[4], b[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const bf16x8_t*>(ap + k0 + 8 * i);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i) b[nb][i] = *reinterpret_cast<const bf16x8_t*>(bp[nb] + k0 + 8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[nb][i], acc[nb], 0, 0, 0);
  }

  // SiLU, then to LDS: acc[nb][r] holds hidden nb*32+lr of token 8*(r/4)+4*lh+(r%4)
  float* h = hs[wave];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      int m = 8 * (r >> 2) + 4 * lh + (r & 3);
      h[m * HSTR + nb * 32 + lr] = silu_f32(acc[nb][r]);
    }
  __syncthreads();

  // ---- layer 2 (fp32 FMA): lane (lr, lh) computes experts e = 2q + lh of token lr
  {
    float l2[NE / 2];
#pragma unroll
    for (int q = 0; q < NE / 2; ++q) l2[q] = 0.0f;
    const float* hrow = h + lr * HSTR;
#pragma unroll 4
    for (int j = 0; j < RT_HID; j += 4) {
      float h0 = hrow[j], h1 = hrow[j + 1], h2 = hrow[j + 2], h3 = hrow[j + 3];
#pragma unroll
      for (int q = 0; q < NE / 2; ++q) {
        const f32x4_t wv = *reinterpret_cast<const f32x4_t*>(&wo[(2 * q + lh) * RT_HID + j]);
        l2[q] = fmaf(h0, wv[0], l2[q]);
        l2[q] = fmaf(h1, wv[1], l2[q]);
        l2[q] = fmaf(h2, wv[2], l2[q]);
        l2[q] = fmaf(h3, wv[3], l2[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < NE / 2; ++q) {
      int e = 2 * q + lh;
      if (e < E) lg[wave][lr][e] = l2[q] + (bias ? bias[e] : 0.0f);
    }
  }
  __syncthreads();

  // ---- softmax, top-k, outputs: one token per lane (lanes 0..31 of each wave)
  if (lh == 0) {
    const int64_t t = tok0 + lr;
    const float* L = lg[wave][lr];
    const int tl = wave * 32 + lr;
    if (t < T) {
      float mx = L[0];
      for (int e = 1; e < E; ++e) mx = fmaxf(mx, L[e]);
      float s = 0.0f;
      for (int e = 0; e < E; ++e) s += __expf(L[e] - mx);
      const float inv_s = 1.0f / s;
      const float lse = mx + __logf(s);
      float* lout = logits + t * E;
      for (int e = 0; e < E; ++e) {
        lout[e] = L[e];
        pe[tl][e] = __expf(L[e] - mx) * inv_s;
      }
      lse2[tl] = lse * lse;
      if (k > 0) {
        // Two identical selection passes (sum of the selected exps, then the
        // outputs) keep everything in registers.
        float ssum = 0.0f;
        float inv = 0.0f;
        for (int pass = 0; pass < 2; ++pass) {
          uint64_t taken = 0;
          for (int j = 0; j < k; ++j) {
            int bi = -1;
            float bv = 0.0f;
            for (int e = 0; e < E; ++e) {
              if ((taken >> e) & 1ull) continue;
              if (bi < 0 || L[e] > bv) {  // strict: equal logits keep the lower index
                bi = e;
                bv = L[e];
              }
            }
            taken |= 1ull << bi;
            const float ev = __expf(bv - mx);
            if (pass == 0) {
              ssum += ev;
            } else {
              topk_idx[t * k + j] = bi;
              topk_w[t * k + j] = ev * inv;
            }
          }
          inv = 1.0f / ssum;
        }
      }
    } else {
      for (int e = 0; e < E; ++e) pe[tl][e] = 0.0f;
      lse2[tl] = 0.0f;
    }
  }
  __syncthreads();

  // ---- per-block aux partials, summed over tokens in a fixed order
  if (partials) {
    float* pb = partials + (int64_t)blockIdx.x * (E + 1);
    if (tid < E) {
      float s = 0.0f;
      for (int i = 0; i < RT_TOK; ++i) s += pe[i][tid];
      pb[tid] = s;
    } else if (tid == E) {
      float s = 0.0f;
      for (int i = 0; i < RT_TOK; ++i) s += lse2[i];
      pb[E] = s;
    }
  }
}

__global__ void aux_loss_kernel(const float* __restrict__ partials, int64_t nblk, int64_t T, int E,
                                const int32_t* __restrict__ counts, int k, float w_lb, float w_z,
                                float* __restrict__ out) {
  __shared__ float col[KMOE_MAX_EXPERTS + 1];
  const int tid = threadIdx.x;
  if (tid <= E) {
    float s = 0.0f;
    for (int64_t b = 0; b < nblk; ++b) s += partials[b * (E + 1) + tid];
    col[tid] = s;
  }
  __syncthreads();
  if (tid == 0) {
    const float invT = 1.0f / (float)T;
    float lb = 0.0f;
    if (counts) {
      const float inv_assign = 1.0f / ((float)T * (float)k);
      for (int e = 0; e < E; ++e) lb += ((float)counts[e] * inv_assign) * (col[e] * invT);
      lb *= (float)E;
    }
    const float z = col[E] * invT;
    out[0] = w_lb * lb + w_z * z;
    out[1] = lb;
    out[2] = z;
  }
}

}  // namespace

extern "C" int64_t kmoe_router_partials_len(int64_t T, int E) {
  return kmoe::ceil_div<int64_t>(T, RT_TOK) * (int64_t)(E + 1);
}

extern "C" int kmoe_router(const void* x, const int32_t* row_index, int64_t T, int d, const void* w_in,
                           const void* w_out, int E, const float* logit_bias, int k, float* logits,
                           int64_t* topk_idx, float* topk_w, float* partials, void* stream) {
  KMOE_REQUIRE(x && w_in && w_out && logits, KMOE_ERR_NULL, "kmoe_router: null x/w_in/w_out/logits");
  KMOE_REQUIRE(T >= 0 && T <= (int64_t)1 << 31, KMOE_ERR_SHAPE, "kmoe_router: T=%lld out of range",
               (long long)T);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "kmoe_router: d=%d must be a positive multiple of 64", d);
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_router: E=%d not in [1,%d]", E,
               KMOE_MAX_EXPERTS);
  KMOE_REQUIRE(k >= 0 && k <= E, KMOE_ERR_SHAPE, "kmoe_router: k=%d not in [0,E=%d]", k, E);
  KMOE_REQUIRE(k == 0 || (topk_idx && topk_w), KMOE_ERR_NULL, "kmoe_router: k>0 needs topk_idx and topk_w");
  if (T == 0) return KMOE_OK;
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T, RT_TOK));
  hipStream_t s = kmoe::as_stream(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wi = static_cast<const uint16_t*>(w_in);
  const uint16_t* wo = static_cast<const uint16_t*>(w_out);
#define KMOE_ROUTER_LAUNCH(NE_)                                                                          \
  hipLaunchKernelGGL(router_kernel<NE_>, grid, dim3(128), 0, s, xp, row_index, T, d, wi, wo, E, logit_bias, k, \
                     logits, topk_idx, topk_w, partials)
  if (E <= 8)
    KMOE_ROUTER_LAUNCH(8);
  else if (E <= 16)
    KMOE_ROUTER_LAUNCH(16);
  else if (E <= 32)
    KMOE_ROUTER_LAUNCH(32);
  else
    KMOE_ROUTER_LAUNCH(64);
#undef KMOE_ROUTER_LAUNCH
  return kmoe::check_launch("kmoe_router");
}

extern "C" int kmoe_aux_loss(const float* partials, int64_t T, int E, const int32_t* counts, int k, float w_lb,
                             float w_z, float* out, void* stream) {
  KMOE_REQUIRE(partials && out, KMOE_ERR_NULL, "kmoe_aux_loss: null partials/out");
  KMOE_REQUIRE(T > 0, KMOE_ERR_SHAPE, "kmoe_aux_loss: T must be > 0");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_aux_loss: E=%d out of range", E);
  KMOE_REQUIRE(!counts || k >= 1, KMOE_ERR_SHAPE, "kmoe_aux_loss: k must be >= 1 with counts");
  const int64_t nblk = kmoe::ceil_div<int64_t>(T, RT_TOK);
  hipLaunchKernelGGL(aux_loss_kernel, dim3(1), dim3(128), 0, kmoe::as_stream(stream), partials, nblk, T, E,
                     counts, k, w_lb, w_z, out);
  return kmoe::check_launch("kmoe_aux_loss");
}
