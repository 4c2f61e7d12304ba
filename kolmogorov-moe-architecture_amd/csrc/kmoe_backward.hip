// Backward pass of the token-choice MoE layer: the memory-bound kernels around the
// grouped GEMMs (which run in kmoe_gemm.hip).  Gradients of the reference forward
//   logits = SiLU(x w_in^T) w_out^T,  p = softmax(logits),  (v, i) = topk(p, k),
//   w = v / sum(v)                                             (moe.py:423-462)
//   y[t] = sum_j w[t,j] * FFN_{i[t,j]}(x[t]),  FFN(x) = (silu(x w1) * (x w2)) w3
//                                                              (moe.py:213-294, ffn.py:17-64)
//   aux = w_lb * E * sum_e f_e P_e + w_z * mean_t lse_t^2      (moe.py:840-939)
// with f_e = counts[e] / (T k) a constant (one-hot of the selections) and
// P_e = mean_t p[t,e].
#include "kmoe_common.h"

namespace {

// dyperm[r] = scale[t] * w[t,j] * dy[row(t)] (bf16) for the kept slot r = slot_row[t,j];
// dw[t,j] = scale[t] * (dy[row(t)] . yperm[r]) and dscale[t] = sum_j w[t,j] (dy[row(t)] .
// yperm[r]) (fp32, lane-ordered fma then a fixed shuffle tree: bit-reproducible; a
// dropped slot gives dw 0 and adds nothing).  row(t) = row_index[t] (or t), scale 1 and
// dscale skipped when NULL.  One wave per token.
__global__ __launch_bounds__(256) void combine_bwd_kernel(const uint16_t* __restrict__ dy,
                                                          const uint16_t* __restrict__ yperm,
                                                          const int32_t* __restrict__ slot_row,
                                                          const float* __restrict__ slot_w, int k, int d, int64_t T,
                                                          const int32_t* __restrict__ row_index,
                                                          const float* __restrict__ scale,
                                                          uint16_t* __restrict__ dyperm, float* __restrict__ dw,
                                                          float* __restrict__ dscale) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nvec = d / 8;
  const int64_t trow = row_index ? (int64_t)row_index[t] : t;
  const float sc = scale ? scale[t] : 1.0f;
  const i32x4_t* dyr = reinterpret_cast<const i32x4_t*>(dy + trow * d);
  float ds = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int r = slot_row[t * k + j];
    const float wj = slot_w[t * k + j];
    if (r < 0) {
      if (lane == 0) dw[t * k + j] = 0.0f;
      continue;
    }
    const float w = sc * wj;
    const i32x4_t* yr = reinterpret_cast<const i32x4_t*>(yperm + (int64_t)r * d);
    i32x4_t* out = reinterpret_cast<i32x4_t*>(dyperm + (int64_t)r * d);
    float dot = 0.0f;
    for (int v = lane; v < nvec; v += 64) {
      const i32x4_t a = dyr[v], b = yr[v];
      i32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a0 = __uint_as_float(((uint32_t)a[q]) << 16), a1 = __uint_as_float(((uint32_t)a[q]) & 0xffff0000u);
        const float b0 = __uint_as_float(((uint32_t)b[q]) << 16), b1 = __uint_as_float(((uint32_t)b[q]) & 0xffff0000u);
        dot = fmaf(a0, b0, dot);
        dot = fmaf(a1, b1, dot);
        o[q] = (int)((uint32_t)f32_to_bf16(w * a0) | ((uint32_t)f32_to_bf16(w * a1) << 16));
      }
      out[v] = o;
    }
    dot = wave_sum(dot);
    if (lane == 0) dw[t * k + j] = sc * dot;
    ds = fmaf(wj, dot, ds);
  }
  if (dscale && lane == 0) dscale[t] = ds;
}

// SwiGLU backward on the packed column order (per 128-column block: 128 gate then 128
// up columns): for h = silu(g) * u,
//   dg = dh * u * s * (1 + g (1 - s)),  du = dh * silu(g),  s = sigmoid(g).
// dh (rows, Fp), gu / dgu (rows, 2 Fp); rows < n_rows_dev[0] when given.
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint16_t* __restrict__ dh,
                                                         const uint16_t* __restrict__ gu, int64_t rows,
                                                         const int32_t* __restrict__ n_rows_dev, int Fp,
                                                         uint16_t* __restrict__ dgu) {
  int64_t nr = rows;
  if (n_rows_dev) nr = min<int64_t>(nr, (int64_t)*n_rows_dev);
  const int cpr = Fp / 8;  // 8-column chunks of a dh row
  const int64_t total = nr * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cpr;
    const int f = (int)(i - r * cpr) * 8;
    const int gc = (f >> 7) * 256 + (f & 127);  // gate column of f in the packed order
    const i32x4_t hv = *reinterpret_cast<const i32x4_t*>(dh + r * Fp + f);
    const i32x4_t gv = *reinterpret_cast<const i32x4_t*>(gu + r * 2 * Fp + gc);
    const i32x4_t uv = *reinterpret_cast<const i32x4_t*>(gu + r * 2 * Fp + gc + 128);
    i32x4_t dgo, duo;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t og = 0, ou = 0;
#pragma unroll
      for (int hlf = 0; hlf < 2; ++hlf) {
        const int sh = hlf * 16;
        const float hh = bf16_to_f32((uint16_t)((uint32_t)hv[q] >> sh));
        const float g = bf16_to_f32((uint16_t)((uint32_t)gv[q] >> sh));
        const float u = bf16_to_f32((uint16_t)((uint32_t)uv[q] >> sh));
        const float s = 1.0f / (1.0f + __expf(-g));
        const float dg = hh * u * s * (1.0f + g * (1.0f - s));
        const float du = hh * g * s;
        og |= (uint32_t)f32_to_bf16(dg) << sh;
        ou |= (uint32_t)f32_to_bf16(du) << sh;
      }
      dgo[q] = (int)og;
      duo[q] = (int)ou;
    }
    *reinterpret_cast<i32x4_t*>(dgu + r * 2 * Fp + gc) = dgo;
    *reinterpret_cast<i32x4_t*>(dgu + r * 2 * Fp + gc + 128) = duo;
  }
}

// Non-gated experts (silu(x . w1) . w2, moe.py:187-191,281-283) on rows of F_pad
// columns, rows < n_rows_dev[0] when given:
//   forward:  h = silu(p)                            (p: the pre-activation x . w1)
//   backward: dp = dh * s * (1 + p (1 - s)),  s = sigmoid(p)
template <bool BWD>
__global__ __launch_bounds__(256) void silu_rows_kernel(const uint16_t* __restrict__ dh, const uint16_t* __restrict__ p,
                                                        int64_t rows, const int32_t* __restrict__ n_rows_dev, int Fp,
                                                        uint16_t* __restrict__ out) {
  int64_t nr = rows;
  if (n_rows_dev) nr = min<int64_t>(nr, (int64_t)*n_rows_dev);
  const int64_t total = nr * (Fp / 8);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const i32x4_t pv = reinterpret_cast<const i32x4_t*>(p)[i];
    i32x4_t hv = {0, 0, 0, 0};
    if constexpr (BWD) hv = reinterpret_cast<const i32x4_t*>(dh)[i];
    i32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t w = 0;
#pragma unroll
      for (int hlf = 0; hlf < 2; ++hlf) {
        const int sh = hlf * 16;
        const float g = bf16_to_f32((uint16_t)((uint32_t)pv[q] >> sh));
        const float sg = 1.0f / (1.0f + __expf(-g));
        float v;
        if constexpr (BWD)
          v = bf16_to_f32((uint16_t)((uint32_t)hv[q] >> sh)) * sg * (1.0f + g * (1.0f - sg));
        else
          v = g * sg;
        w |= (uint32_t)f32_to_bf16(v) << sh;
      }
      o[q] = (int)w;
    }
    reinterpret_cast<i32x4_t*>(out)[i] = o;
  }
}

// Router logit gradient, one thread per token (E <= 64):
//   top-k renormalisation (w_j = p_j / sum_sel p = softmax over the selected logits):
//     dl[i_j] += w_j (dw_j - sum_l w_l dw_l)
//   aux (scaled by the upstream gradient g of the aux loss):
//     dl += g * (w_lb E / T * p (f - p.f) + w_z 2/T * lse * p),  f_e = counts[e] / (T k)
template <int NE>
__global__ __launch_bounds__(256) void router_dlogits_kernel(const float* __restrict__ logits, int64_t T, int E,
                                                             const int64_t* __restrict__ topk_idx,
                                                             const float* __restrict__ topk_w,
                                                             const float* __restrict__ dw, int k,
                                                             const int32_t* __restrict__ counts,
                                                             const float* __restrict__ grad_aux, float w_lb,
                                                             float w_z, float* __restrict__ dl) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  float L[NE], g[NE];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    L[e] = e < E ? logits[t * E + e] : -INFINITY;
    mx = fmaxf(mx, L[e]);
    g[e] = 0.0f;
  }
  const float ga = grad_aux ? grad_aux[0] : 0.0f;
  if (ga != 0.0f) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      L[e] = e < E ? __expf(L[e] - mx) : 0.0f;
      s += L[e];
    }
    const float inv = 1.0f / s, lse = mx + __logf(s);
    const float invTk = 1.0f / ((float)T * (float)k);
    float pf = 0.0f;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      L[e] *= inv;  // p
      if (counts && e < E) pf += L[e] * ((float)counts[e] * invTk);
    }
    const float clb = w_lb * (float)E / (float)T, cz = w_z * 2.0f / (float)T * lse;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      if (e < E) {
        const float fe = counts ? (float)counts[e] * invTk : 0.0f;
        g[e] = ga * (clb * L[e] * (fe - pf) + cz * L[e]);
      }
    }
  }
  float c = 0.0f;
  for (int j = 0; j < k; ++j) c += topk_w[t * k + j] * dw[t * k + j];
  for (int j = 0; j < k; ++j) {
    const int e = (int)topk_idx[t * k + j];
    const float v = topk_w[t * k + j] * (dw[t * k + j] - c);
#pragma unroll
    for (int q = 0; q < NE; ++q)
      if (q == e) g[q] += v;
  }
#pragma unroll
  for (int e = 0; e < NE; ++e)
    if (e < E) dl[t * E + e] = g[e];
}

// Expert-choice logit gradient (ExpertChoiceRouter.forward, moe.py:513-528): per
// sequence b and expert e, p_s = softmax over the S tokens of logits[b, :, e]; the C
// selected tokens (src_row[t, e] >= 0) carry w_s = p_s / (P + 1e-9), P = sum_sel p.
// With g_s = dL/dw_s (dw[t, e]):  dL/dp_s = (g_s - G) / (P + 1e-9) for selected s (0
// otherwise), G = sum_sel g w;  dl_s += p_s (dL/dp_s - Q),  Q = sum_sel p dL/dp.  One
// 1024-thread workgroup per (b, e), fixed-order block reductions (bit-reproducible).
constexpr int ECD_THREADS = 1024;
__device__ __forceinline__ float ecd_block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float tot = 0.0f;
  for (int w = 0; w < ECD_THREADS / 64; ++w) tot += red[w];
  return tot;
}
__device__ __forceinline__ float ecd_block_max(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = -INFINITY;
  for (int w = 0; w < ECD_THREADS / 64; ++w) m = fmaxf(m, red[w]);
  return m;
}
__global__ __launch_bounds__(ECD_THREADS) void ec_dlogits_kernel(const float* __restrict__ logits, int S, int E,
                                                                 const int32_t* __restrict__ src_row,
                                                                 const float* __restrict__ src_w,
                                                                 const float* __restrict__ dw, float* __restrict__ dl) {
  __shared__ float red[ECD_THREADS / 64];
  const int b = blockIdx.x / E, e = blockIdx.x % E;
  const int64_t t0 = (int64_t)b * S;
  float mx = -INFINITY;
  for (int s = threadIdx.x; s < S; s += ECD_THREADS) mx = fmaxf(mx, logits[(t0 + s) * E + e]);
  mx = ecd_block_max(mx, red);
  float se = 0.0f, pe = 0.0f, gw = 0.0f;
  for (int s = threadIdx.x; s < S; s += ECD_THREADS) {
    const int64_t i = (t0 + s) * E + e;
    const float ex = __expf(logits[i] - mx);
    se += ex;
    if (src_row[i] >= 0) {
      pe += ex;
      gw += dw[i] * src_w[i];
    }
  }
  se = ecd_block_sum(se, red);
  pe = ecd_block_sum(pe, red);
  const float G = ecd_block_sum(gw, red);
  const float inv = 1.0f / se;
  const float invZ = 1.0f / (pe * inv + 1e-9f);
  float q = 0.0f;
  for (int s = threadIdx.x; s < S; s += ECD_THREADS) {
    const int64_t i = (t0 + s) * E + e;
    if (src_row[i] >= 0) q += __expf(logits[i] - mx) * inv * (dw[i] - G) * invZ;
  }
  const float Q = ecd_block_sum(q, red);
  for (int s = threadIdx.x; s < S; s += ECD_THREADS) {
    const int64_t i = (t0 + s) * E + e;
    const float p = __expf(logits[i] - mx) * inv;
    const float dp = src_row[i] >= 0 ? (dw[i] - G) * invZ : 0.0f;
    dl[i] += p * (dp - Q);
  }
}

// Router MLP backward over a block of 64 tokens (256 threads, 4 per token):
//   s = silu(a), ds = dl w_out, da = ds * silu'(a)      -> da (T, 128) bf16
//   partial[b][e][j] = sum_{t in block} dl[t,e] s[t,j]  -> reduced by router_reduce_kernel
// a (T, 128) f32 is the saved pre-activation of the d -> 128 layer.
constexpr int RB_TOK = 64;
constexpr int RH = KMOE_ROUTER_HIDDEN;
template <int NE>
__global__ __launch_bounds__(256) void router_mlp_bwd_kernel(const float* __restrict__ dl,
                                                             const float* __restrict__ a, int64_t T, int E,
                                                             const uint16_t* __restrict__ w_out,
                                                             uint16_t* __restrict__ da,
                                                             float* __restrict__ partial) {
  __shared__ float wo[NE][RH];
  __shared__ float s_l[RB_TOK][RH + 1];
  __shared__ float dl_l[RB_TOK][NE];
  const int tid = threadIdx.x;
  const int64_t t0 = (int64_t)blockIdx.x * RB_TOK;
  for (int i = tid; i < NE * RH; i += 256) wo[i / RH][i % RH] = i / RH < E ? bf16_to_f32(w_out[i]) : 0.0f;
  for (int i = tid; i < RB_TOK * NE; i += 256) {
    const int tl = i / NE, e = i % NE;
    dl_l[tl][e] = (t0 + tl < T && e < E) ? dl[(t0 + tl) * E + e] : 0.0f;
  }
  __syncthreads();
  const int tl = tid >> 2, part = tid & 3;
  const int64_t t = t0 + tl;
  for (int jj = 0; jj < RH / 4; ++jj) {
    const int j = part + 4 * jj;
    const float av = t < T ? a[t * RH + j] : 0.0f;
    const float sg = 1.0f / (1.0f + __expf(-av));
    const float s = av * sg;
    float ds = 0.0f;
#pragma unroll
    for (int e = 0; e < NE; ++e) ds = fmaf(dl_l[tl][e], wo[e][j], ds);
    s_l[tl][j] = t < T ? s : 0.0f;
    if (t < T) da[t * RH + j] = f32_to_bf16(ds * sg * (1.0f + av * (1.0f - sg)));
  }
  __syncthreads();
  // partial dW_out of the block: thread handles (e, j) pairs tid, tid + 256, ...
  for (int i = tid; i < NE * RH; i += 256) {
    const int e = i / RH, j = i % RH;
    float acc = 0.0f;
    for (int q = 0; q < RB_TOK; ++q) acc = fmaf(dl_l[q][e], s_l[q][j], acc);
    if (e < E) partial[(int64_t)blockIdx.x * E * RH + e * RH + j] = acc;
  }
}

// out[i] = sum_b partial[b][i] (bf16 or f32 out).
// 64 outputs per workgroup (lane = output, coalesced across the wave), RWAVES waves
// each summing every RWAVES-th partial in order, then the RWAVES sums in wave order:
// a fixed order, so the result is bit-reproducible.  (One thread per output summing all
// partials serially left the 256-partial router reduction latency-bound: 8 workgroups.)
constexpr int RWAVES = 16;
__global__ __launch_bounds__(64 * RWAVES) void reduce_partials_kernel(const float* __restrict__ partial, int64_t nblk,
                                                                      int64_t n, void* __restrict__ out, bool out_f32) {
  __shared__ float red[RWAVES][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (i < n) {
#pragma unroll 4
    for (int64_t b = w; b < nblk; b += RWAVES) s += partial[b * n + i];
  }
  red[w][lane] = s;
  __syncthreads();
  if (w != 0 || i >= n) return;
  float t = 0.0f;
#pragma unroll
  for (int q = 0; q < RWAVES; ++q) t += red[q][lane];
  if (out_f32)
    static_cast<float*>(out)[i] = t;
  else
    static_cast<uint16_t*>(out)[i] = f32_to_bf16(t);
}

// Mixture-of-Depths router backward.  sel_w = softmax over each sequence's kept
// logits (mod.py:107-112), so for the gradient dsel of the weights
//   dlog[i] = p_i (dsel_i - sum_l p_l dsel_l)
// (one workgroup per sequence; the sum in a fixed order).  dlog is written with a
// stride, so that it can land in a column of a caller's table.
constexpr int MODB_THREADS = 1024;
__global__ __launch_bounds__(MODB_THREADS) void mod_dlog_kernel(const float* __restrict__ sel_w,
                                                                const float* __restrict__ dsel, int64_t keep,
                                                                float* __restrict__ dlog, int64_t stride) {
  __shared__ float red[MODB_THREADS / 64];
  const int64_t base = (int64_t)blockIdx.x * keep;
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < keep; i += MODB_THREADS) s = fmaf(sel_w[base + i], dsel[base + i], s);
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int q = 0; q < MODB_THREADS / 64; ++q) tot += red[q];
  for (int64_t i = threadIdx.x; i < keep; i += MODB_THREADS) {
    const float p = sel_w[base + i];
    dlog[(base + i) * stride] = p * (dsel[base + i] - tot);
  }
}

// partial[seg][c] = sum over the rows t of segment seg of dlog[t] x[t][c]: the MoD
// router weight's gradient (logits = x . w_mod).  4 waves per workgroup, wave w taking
// every 4th row of the segment, 512 columns per workgroup (8 per lane); the waves'
// sums are added in wave order through LDS.
__global__ __launch_bounds__(256) void mod_wgrad_kernel(const uint16_t* __restrict__ x, int d, int64_t T,
                                                        const float* __restrict__ dlog, int64_t stride,
                                                        int64_t seg_rows, float* __restrict__ partial) {
  __shared__ float red[4][512];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c0 = (int)blockIdx.y * 512 + lane * 8;
  const int64_t t0 = (int64_t)blockIdx.x * seg_rows;
  const int64_t t1 = t0 + seg_rows < T ? t0 + seg_rows : T;
  float acc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
  if (c0 < d) {
    for (int64_t t = t0 + w; t < t1; t += 4) {
      const float gl = dlog[t * stride];
      const i32x4_t a = *reinterpret_cast<const i32x4_t*>(x + t * d + c0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[2 * q] = fmaf(gl, __uint_as_float(((uint32_t)a[q]) << 16), acc[2 * q]);
        acc[2 * q + 1] = fmaf(gl, __uint_as_float(((uint32_t)a[q]) & 0xffff0000u), acc[2 * q + 1]);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) red[w][lane * 8 + q] = acc[q];
  __syncthreads();
  for (int c = threadIdx.x; c < 512; c += 256) {
    const int col = (int)blockIdx.y * 512 + c;
    if (col < d) partial[(int64_t)blockIdx.x * d + col] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
  }
}

int64_t mod_seg_rows(int64_t n) {
  // at most 256 segments, each a multiple of 4 rows
  int64_t rows = kmoe::ceil_div<int64_t>(n, 256);
  rows = kmoe::ceil_div<int64_t>(rows, 4) * 4;
  return rows < 4 ? 4 : rows;
}

// w_in (128, d) -> packed rows of w_in^T: (round_up(d, 256), 128 + 64) bf16, row i =
// w_in[:, i] (the B operand of dx_router = da . w_in), zero padded.
__global__ __launch_bounds__(256) void pack_w_in_t_kernel(const void* __restrict__ w_in, bool in_f32, int d,
                                                          uint16_t* __restrict__ out, int64_t rows, int ld) {
  const int64_t n = rows * ld;
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < n; o += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = o / ld;
    const int j = (int)(o - i * ld);
    uint16_t v = 0;
    if (i < d && j < RH) {
      const int64_t src = (int64_t)j * d + i;
      v = in_f32 ? f32_to_bf16(static_cast<const float*>(w_in)[src]) : static_cast<const uint16_t*>(w_in)[src];
    }
    out[o] = v;
  }
}

unsigned grid_for(int64_t n, int per_block) {
  const int64_t b = kmoe::ceil_div<int64_t>(n, per_block);
  return (unsigned)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

// ---------------------------------------------------------------- fp8 straight-through operands
// The fp8 experts' backward lets the gradients through the e4m3 quantisations unchanged
// and multiplies by the operands the fp8 GEMMs actually took: the dequantised rows and
// weights, bf16.

// out[r, :] = bf16(e4m3(q[r, :]) * scale[r]) for rows r < min(rows, *n_rows_dev) (the
// other rows are not written).  One wave per row at a time, 8 codes per lane and step
// (an 8-byte load, a 16-byte store).
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ q,
                                                           const float* __restrict__ scale, int64_t rows,
                                                           const int32_t* __restrict__ n_rows_dev, int cols,
                                                           uint16_t* __restrict__ out) {
  int64_t nr = rows;
  if (n_rows_dev) nr = min<int64_t>(nr, (int64_t)*n_rows_dev);
  const int lane = threadIdx.x & 63;
  const int nvec = cols / 8;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < nr; r += (int64_t)gridDim.x * 4) {
    const float s = scale[r];
    const uint2* src = reinterpret_cast<const uint2*>(q + r * cols);
    uint4* dst = reinterpret_cast<uint4*>(out + r * cols);
    for (int v = lane; v < nvec; v += 64) {
      const uint2 c = src[v];
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = (i < 2 ? c.x : c.y) >> ((i & 1) * 16);
        const float a = e4m3_to_f32(w & 0xffu) * s, b = e4m3_to_f32((w >> 8) & 0xffu) * s;
        o[i] = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
      }
      dst[v] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// out (E, K, N) bf16 = w (E, K, N) fake-quantised per column n of each expert, as the
// fp8 weight packing quantises it: scale = amax / 448 over the column's K values, code =
// e4m3(w * (448 / amax)) (saturating, nearest even), out = bf16(code * scale); a zero
// column stays zero.  Workgroup: 64 columns of one expert, the 4 waves splitting K.
template <bool F32>
__global__ __launch_bounds__(256) void fake_quant_cols_kernel(const void* __restrict__ w, int K, int N,
                                                              uint16_t* __restrict__ out) {
  __shared__ float red[4][64];
  const int c = threadIdx.x & 63, kw = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + c;
  const int64_t base = (int64_t)blockIdx.y * K * N;
  auto ld = [&](int64_t i) -> float {
    return F32 ? static_cast<const float*>(w)[i] : bf16_to_f32(static_cast<const uint16_t*>(w)[i]);
  };
  float amax = 0.0f;
  if (n < N)
    for (int k = kw; k < K; k += 4) amax = fmaxf(amax, fabsf(ld(base + (int64_t)k * N + n)));
  red[kw][c] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0][c], red[1][c]), fmaxf(red[2][c], red[3][c]));
  if (n >= N) return;
  const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
  const float sc = amax / 448.0f;
  for (int k = kw; k < K; k += 4) {
    const int64_t i = base + (int64_t)k * N + n;
    out[i] = f32_to_bf16(e4m3_to_f32(f32_to_e4m3(ld(i) * inv)) * sc);
  }
}

}  // namespace

extern "C" int kmoe_combine_bwd(const void* dy, const void* yperm, const int32_t* slot_row, const float* slot_w, int k,
                                int d, int64_t T, void* dyperm, float* dw, void* stream) {
  KMOE_REQUIRE(dy && yperm && slot_row && slot_w && dyperm && dw, KMOE_ERR_NULL, "kmoe_combine_bwd: null buffer");
  KMOE_REQUIRE(k >= 1 && k <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_combine_bwd: k=%d", k);
  KMOE_REQUIRE(d > 0 && d % 8 == 0, KMOE_ERR_SHAPE, "kmoe_combine_bwd: d=%d must be a multiple of 8", d);
  KMOE_REQUIRE(T >= 0, KMOE_ERR_SHAPE, "kmoe_combine_bwd: T < 0");
  if (T == 0) return KMOE_OK;
  hipLaunchKernelGGL(combine_bwd_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(T, 4)), dim3(256), 0,
                     kmoe::as_stream(stream), static_cast<const uint16_t*>(dy), static_cast<const uint16_t*>(yperm),
                     slot_row, slot_w, k, d, T, nullptr, nullptr, static_cast<uint16_t*>(dyperm), dw, nullptr);
  return kmoe::check_launch("kmoe_combine_bwd");
}

extern "C" int kmoe_combine_bwd_rows(const void* dy, const void* yperm, const int32_t* slot_row, const float* slot_w,
                                     int k, int d, int64_t T, const int32_t* row_index, const float* scale,
                                     void* dyperm, float* dw, float* dscale, void* stream) {
  KMOE_REQUIRE(dy && yperm && slot_row && slot_w && dyperm && dw, KMOE_ERR_NULL,
               "kmoe_combine_bwd_rows: null buffer");
  KMOE_REQUIRE(k >= 1 && k <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_combine_bwd_rows: k=%d", k);
  KMOE_REQUIRE(d > 0 && d % 8 == 0, KMOE_ERR_SHAPE, "kmoe_combine_bwd_rows: d=%d must be a multiple of 8", d);
  KMOE_REQUIRE(T >= 0, KMOE_ERR_SHAPE, "kmoe_combine_bwd_rows: T < 0");
  if (T == 0) return KMOE_OK;
  hipLaunchKernelGGL(combine_bwd_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(T, 4)), dim3(256), 0,
                     kmoe::as_stream(stream), static_cast<const uint16_t*>(dy), static_cast<const uint16_t*>(yperm),
                     slot_row, slot_w, k, d, T, row_index, scale, static_cast<uint16_t*>(dyperm), dw, dscale);
  return kmoe::check_launch("kmoe_combine_bwd_rows");
}

extern "C" int kmoe_swiglu_bwd(const void* dh, const void* gu, int64_t rows, const int32_t* n_rows_dev, int F,
                               void* dgu, void* stream) {
  KMOE_REQUIRE(dh && gu && dgu, KMOE_ERR_NULL, "kmoe_swiglu_bwd: null buffer");
  KMOE_REQUIRE(rows >= 0 && F > 0, KMOE_ERR_SHAPE, "kmoe_swiglu_bwd: bad shape");
  if (rows == 0) return KMOE_OK;
  const int Fp = (F + 127) / 128 * 128;
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(grid_for(rows * (Fp / 8), 256)), dim3(256), 0, kmoe::as_stream(stream),
                     static_cast<const uint16_t*>(dh), static_cast<const uint16_t*>(gu), rows, n_rows_dev, Fp,
                     static_cast<uint16_t*>(dgu));
  return kmoe::check_launch("kmoe_swiglu_bwd");
}

extern "C" int kmoe_silu_rows(const void* p, int64_t rows, const int32_t* n_rows_dev, int F, void* h, void* stream) {
  KMOE_REQUIRE(p && h, KMOE_ERR_NULL, "kmoe_silu_rows: null buffer");
  KMOE_REQUIRE(rows >= 0 && F > 0, KMOE_ERR_SHAPE, "kmoe_silu_rows: bad shape");
  if (rows == 0) return KMOE_OK;
  const int Fp = (F + 127) / 128 * 128;
  hipLaunchKernelGGL(silu_rows_kernel<false>, dim3(grid_for(rows * (Fp / 8), 256)), dim3(256), 0,
                     kmoe::as_stream(stream), nullptr, static_cast<const uint16_t*>(p), rows, n_rows_dev, Fp,
                     static_cast<uint16_t*>(h));
  return kmoe::check_launch("kmoe_silu_rows");
}

extern "C" int kmoe_silu_bwd(const void* dh, const void* p, int64_t rows, const int32_t* n_rows_dev, int F, void* dp,
                             void* stream) {
  KMOE_REQUIRE(dh && p && dp, KMOE_ERR_NULL, "kmoe_silu_bwd: null buffer");
  KMOE_REQUIRE(rows >= 0 && F > 0, KMOE_ERR_SHAPE, "kmoe_silu_bwd: bad shape");
  if (rows == 0) return KMOE_OK;
  const int Fp = (F + 127) / 128 * 128;
  hipLaunchKernelGGL(silu_rows_kernel<true>, dim3(grid_for(rows * (Fp / 8), 256)), dim3(256), 0,
                     kmoe::as_stream(stream), static_cast<const uint16_t*>(dh), static_cast<const uint16_t*>(p), rows,
                     n_rows_dev, Fp, static_cast<uint16_t*>(dp));
  return kmoe::check_launch("kmoe_silu_bwd");
}

extern "C" int kmoe_router_dlogits(const float* logits, int64_t T, int E, const int64_t* topk_idx, const float* topk_w,
                                   const float* dw, int k, const int32_t* counts, const float* grad_aux, float w_lb,
                                   float w_z, float* dlogits, void* stream) {
  KMOE_REQUIRE(logits && dlogits && (k == 0 || (topk_idx && topk_w && dw)), KMOE_ERR_NULL,
               "kmoe_router_dlogits: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS && k >= 0 && k <= E, KMOE_ERR_SHAPE, "kmoe_router_dlogits: E=%d k=%d",
               E, k);
  if (T == 0) return KMOE_OK;
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T, 256));
  hipStream_t s = kmoe::as_stream(stream);
#define KMOE_DL(NE_) \
  hipLaunchKernelGGL(router_dlogits_kernel<NE_>, grid, dim3(256), 0, s, logits, T, E, topk_idx, topk_w, dw, k, counts, \
                     grad_aux, w_lb, w_z, dlogits)
  if (E <= 8)
    KMOE_DL(8);
  else if (E <= 16)
    KMOE_DL(16);
  else if (E <= 32)
    KMOE_DL(32);
  else
    KMOE_DL(64);
#undef KMOE_DL
  return kmoe::check_launch("kmoe_router_dlogits");
}

extern "C" int kmoe_ec_dlogits(const float* logits, int B, int S, int E, const int32_t* src_row, const float* src_w,
                               const float* dw, float* dlogits, void* stream) {
  KMOE_REQUIRE(logits && src_row && src_w && dw && dlogits, KMOE_ERR_NULL, "kmoe_ec_dlogits: null buffer");
  KMOE_REQUIRE(B >= 1 && S >= 1 && E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_ec_dlogits: B=%d S=%d E=%d",
               B, S, E);
  hipLaunchKernelGGL(ec_dlogits_kernel, dim3((unsigned)(B * E)), dim3(ECD_THREADS), 0, kmoe::as_stream(stream), logits,
                     S, E, src_row, src_w, dw, dlogits);
  return kmoe::check_launch("kmoe_ec_dlogits");
}

extern "C" size_t kmoe_router_bwd_workspace_bytes(int64_t T, int E) {
  return (size_t)kmoe::ceil_div<int64_t>(T, RB_TOK) * (size_t)E * RH * sizeof(float);
}

extern "C" int kmoe_router_mlp_bwd(const float* dlogits, const float* hidden_pre, int64_t T, int E, const void* w_out,
                                   void* da, void* dw_out, int dw_dtype, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  KMOE_REQUIRE(dlogits && hidden_pre && w_out && da && dw_out && workspace, KMOE_ERR_NULL,
               "kmoe_router_mlp_bwd: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_router_mlp_bwd: E=%d", E);
  KMOE_REQUIRE(dw_dtype == KMOE_DTYPE_BF16 || dw_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "kmoe_router_mlp_bwd: dw_out dtype");
  KMOE_REQUIRE(workspace_bytes >= kmoe_router_bwd_workspace_bytes(T, E), KMOE_ERR_WORKSPACE,
               "kmoe_router_mlp_bwd: workspace %zu < %zu", workspace_bytes, kmoe_router_bwd_workspace_bytes(T, E));
  if (T == 0) return KMOE_OK;
  const int64_t nblk = kmoe::ceil_div<int64_t>(T, RB_TOK);
  hipStream_t s = kmoe::as_stream(stream);
  float* part = static_cast<float*>(workspace);
#define KMOE_MB(NE_)                                                                                        \
  hipLaunchKernelGGL(router_mlp_bwd_kernel<NE_>, dim3((unsigned)nblk), dim3(256), 0, s, dlogits, hidden_pre, T, E, \
                     static_cast<const uint16_t*>(w_out), static_cast<uint16_t*>(da), part)
  if (E <= 8)
    KMOE_MB(8);
  else if (E <= 16)
    KMOE_MB(16);
  else if (E <= 32)
    KMOE_MB(32);
  else
    KMOE_MB(64);
#undef KMOE_MB
  const int64_t n = (int64_t)E * RH;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(n, 64)), dim3(64 * RWAVES), 0, s,
                     part, nblk, n, dw_out, dw_dtype == KMOE_DTYPE_F32);
  return kmoe::check_launch("kmoe_router_mlp_bwd");
}

extern "C" size_t kmoe_packed_w_in_t_bytes(int d) { return (size_t)((d + 255) / 256 * 256) * (RH + 64) * 2; }

extern "C" int kmoe_pack_w_in_t(const void* w_in, int w_dtype, int d, void* out, void* stream) {
  KMOE_REQUIRE(w_in && out, KMOE_ERR_NULL, "kmoe_pack_w_in_t: null buffer");
  KMOE_REQUIRE(d > 0, KMOE_ERR_SHAPE, "kmoe_pack_w_in_t: d=%d", d);
  KMOE_REQUIRE(w_dtype == KMOE_DTYPE_BF16 || w_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE, "kmoe_pack_w_in_t: dtype");
  const int64_t rows = (d + 255) / 256 * 256;
  hipLaunchKernelGGL(pack_w_in_t_kernel, dim3(grid_for(rows * (RH + 64), 256)), dim3(256), 0, kmoe::as_stream(stream),
                     w_in, w_dtype == KMOE_DTYPE_F32, d, static_cast<uint16_t*>(out), rows, RH + 64);
  return kmoe::check_launch("kmoe_pack_w_in_t");
}


extern "C" int kmoe_reduce_f32(const float* partial, int64_t n_parts, int64_t n, void* out, int out_dtype,
                               void* stream) {
  KMOE_REQUIRE(partial && out, KMOE_ERR_NULL, "kmoe_reduce_f32: null buffer");
  KMOE_REQUIRE(n_parts >= 1 && n >= 0, KMOE_ERR_SHAPE, "kmoe_reduce_f32: bad shape");
  KMOE_REQUIRE(out_dtype == KMOE_DTYPE_BF16 || out_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE, "kmoe_reduce_f32: dtype");
  if (n == 0) return KMOE_OK;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(n, 64)), dim3(64 * RWAVES), 0,
                     kmoe::as_stream(stream), partial, n_parts, n, out, out_dtype == KMOE_DTYPE_F32);
  return kmoe::check_launch("kmoe_reduce_f32");
}

extern "C" size_t kmoe_mod_bwd_workspace_bytes(int64_t n_rows, int d) {
  if (n_rows <= 0 || d <= 0) return 0;
  return (size_t)kmoe::ceil_div<int64_t>(n_rows, mod_seg_rows(n_rows)) * (size_t)d * sizeof(float);
}

extern "C" int kmoe_mod_bwd(const float* sel_w, const float* dsel, int B, int64_t keep, const void* x_sel, int d,
                            float* dlog, int64_t dlog_stride, void* dw_mod, int dw_dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  KMOE_REQUIRE(sel_w && dsel && dlog, KMOE_ERR_NULL, "kmoe_mod_bwd: null buffer");
  KMOE_REQUIRE(B >= 1 && keep >= 1 && dlog_stride >= 1, KMOE_ERR_SHAPE, "kmoe_mod_bwd: bad B/keep/stride");
  hipStream_t s = kmoe::as_stream(stream);
  hipLaunchKernelGGL(mod_dlog_kernel, dim3((unsigned)B), dim3(MODB_THREADS), 0, s, sel_w, dsel, keep, dlog,
                     dlog_stride);
  int rc = kmoe::check_launch("kmoe_mod_bwd");
  if (rc != KMOE_OK || !dw_mod) return rc;
  KMOE_REQUIRE(x_sel, KMOE_ERR_NULL, "kmoe_mod_bwd: null x_sel with a weight gradient");
  KMOE_REQUIRE(d > 0 && d % 8 == 0, KMOE_ERR_SHAPE, "kmoe_mod_bwd: d=%d must be a multiple of 8", d);
  KMOE_REQUIRE(dw_dtype == KMOE_DTYPE_BF16 || dw_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE, "kmoe_mod_bwd: dtype");
  const int64_t n = (int64_t)B * keep;
  const size_t need = kmoe_mod_bwd_workspace_bytes(n, d);
  KMOE_REQUIRE(workspace && workspace_bytes >= need, KMOE_ERR_WORKSPACE, "kmoe_mod_bwd: workspace %zu < %zu bytes",
               workspace_bytes, need);
  const int64_t seg = mod_seg_rows(n);
  const int64_t nseg = kmoe::ceil_div<int64_t>(n, seg);
  float* partial = static_cast<float*>(workspace);
  hipLaunchKernelGGL(mod_wgrad_kernel, dim3((unsigned)nseg, (unsigned)kmoe::ceil_div(d, 512)), dim3(256), 0, s,
                     static_cast<const uint16_t*>(x_sel), d, n, dlog, dlog_stride, seg, partial);
  rc = kmoe::check_launch("kmoe_mod_bwd");
  if (rc != KMOE_OK) return rc;
  return kmoe_reduce_f32(partial, nseg, d, dw_mod, dw_dtype, stream);
}

extern "C" int kmoe_dequant_rows_fp8(const uint8_t* q, const float* scale, int64_t rows, const int32_t* n_rows_dev,
                                     int cols, void* out, void* stream) {
  KMOE_REQUIRE(q && scale && out, KMOE_ERR_NULL, "kmoe_dequant_rows_fp8: null buffer");
  KMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, KMOE_ERR_SHAPE,
               "kmoe_dequant_rows_fp8: rows=%lld cols=%d (cols must be a positive multiple of 8)", (long long)rows,
               cols);
  if (rows == 0) return KMOE_OK;
  int64_t blocks = kmoe::ceil_div<int64_t>(rows, 4);
  const int64_t cap = (int64_t)kmoe::cu_count() * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, kmoe::as_stream(stream), q, scale,
                     rows, n_rows_dev, cols, static_cast<uint16_t*>(out));
  return kmoe::check_launch("kmoe_dequant_rows_fp8");
}

extern "C" int kmoe_fake_quant_e4m3_cols(const void* w, int w_dtype, int E, int K, int N, void* out, void* stream) {
  KMOE_REQUIRE(w && out, KMOE_ERR_NULL, "kmoe_fake_quant_e4m3_cols: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= 65535 && K >= 1 && N >= 1, KMOE_ERR_SHAPE, "kmoe_fake_quant_e4m3_cols: E=%d K=%d N=%d",
               E, K, N);
  KMOE_REQUIRE(w_dtype == KMOE_DTYPE_BF16 || w_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "kmoe_fake_quant_e4m3_cols: weights must be bf16 or f32");
  const dim3 grid((unsigned)kmoe::ceil_div(N, 64), (unsigned)E);
  hipStream_t s = kmoe::as_stream(stream);
  uint16_t* o = static_cast<uint16_t*>(out);
  if (w_dtype == KMOE_DTYPE_F32)
    hipLaunchKernelGGL(fake_quant_cols_kernel<true>, grid, dim3(256), 0, s, w, K, N, o);
  else
    hipLaunchKernelGGL(fake_quant_cols_kernel<false>, grid, dim3(256), 0, s, w, K, N, o);
  return kmoe::check_launch("kmoe_fake_quant_e4m3_cols");
}
