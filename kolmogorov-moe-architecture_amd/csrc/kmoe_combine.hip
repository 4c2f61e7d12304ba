// Combine: y[o] = scale[s] * sum_j w[s,j] * yperm[src[s,j]],  s = out_map ? out_map[o] : o.
// Replaces the gather / weight / index_add_ tail of GroupedExperts.forward
// (moe_arch/model/moe.py:285-292), the expert-choice scatter-add
// (_pytorch_scatter_add_experts, moe.py:132-158) and, with out_map/scale, the
// MoD weighted scatter back to full sequence length (layers.py:175-185).
//
// One wave per output row, 16-byte vector loads of each source row, fp32
// accumulation in a fixed source order: no atomics, bit-reproducible.
//
// With a residual (y's dtype, (T_out, d)): y[o] = residual[o] + the sum above, added
// in fp32 before the one rounding to y's dtype; rows without a source set
// (out_map[o] < 0) get residual[o].  This is the residual add of the block's FFN half
// (hidden_states = residual + ffn_output, layers.py:187) folded into the combine.
// With a keep mask ((T_out, d) bytes, 0 or 1) the sum is the residual dropout's output:
// y[o] = residual[o] + keep[o] * keep_scale * (the sum above), keep_scale = 1/(1-p)
// (layers.py:190, residual + residual_dropout(ffn_output)), still one rounding.
#include "kmoe_common.h"

namespace {

constexpr int CROWS = 4;  // rows (waves) per workgroup

template <bool OUT_F32, bool RES = false, bool MASK = false>
__global__ __launch_bounds__(64 * CROWS) void combine_kernel(const uint16_t* __restrict__ yperm, int d,
                                                             const int32_t* __restrict__ src_row,
                                                             const float* __restrict__ src_w, int fan,
                                                             const int32_t* __restrict__ out_map,
                                                             const float* __restrict__ scale, int64_t T_out,
                                                             void* __restrict__ y,
                                                             const void* __restrict__ residual,
                                                             const uint8_t* __restrict__ keep, float keep_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t o = (int64_t)blockIdx.x * CROWS + (threadIdx.x >> 6);
  if (o >= T_out) return;
  const int64_t s = out_map ? (int64_t)out_map[o] : o;
  const int nvec = d / 8;
  if (s < 0) {
    if (RES) {
      // 16 bytes per vector of 8 bf16, 32 of 8 f32
      const int nb = OUT_F32 ? 2 * nvec : nvec;
      const i32x4_t* src = reinterpret_cast<const i32x4_t*>(static_cast<const uint8_t*>(residual) +
                                                            o * d * (OUT_F32 ? 4 : 2));
      i32x4_t* dst = reinterpret_cast<i32x4_t*>(static_cast<uint8_t*>(y) + o * d * (OUT_F32 ? 4 : 2));
      for (int v = lane; v < nb; v += 64) dst[v] = src[v];
    } else if (OUT_F32) {
      f32x4_t* dst = reinterpret_cast<f32x4_t*>(static_cast<float*>(y) + o * d);
      const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
      for (int v = lane; v < nvec; v += 64) {
        dst[2 * v] = z;
        dst[2 * v + 1] = z;
      }
    } else {
      i32x4_t* dst = reinterpret_cast<i32x4_t*>(static_cast<uint16_t*>(y) + o * d);
      const i32x4_t z = {0, 0, 0, 0};
      for (int v = lane; v < nvec; v += 64) dst[v] = z;
    }
    return;
  }
  const float sc = scale ? scale[s] : 1.0f;
  // Source list of this row (fan <= 64): lane j holds source j.
  int my_src = -1;
  float my_w = 0.0f;
  if (lane < fan) {
    my_src = src_row[s * fan + lane];
    my_w = src_w[s * fan + lane];
  }
  const uint64_t live = __ballot(my_src >= 0);
  // Row vectors in groups of 4 x 64 (one per lane per group); sources in pairs, so
  // up to 8 16-byte loads are in flight per lane.  Accumulation order is the
  // source order, as written.
  for (int v0 = 0; v0 < nvec; v0 += 256) {
    float acc[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[u][q] = 0.0f;
    uint64_t m = live;
    while (m) {
      const int j0 = __builtin_ctzll(m);
      m &= m - 1;
      int j1 = -1;
      if (m) {
        j1 = __builtin_ctzll(m);
        m &= m - 1;
      }
      const int r0 = __shfl(my_src, j0, 64);
      const float w0 = __shfl(my_w, j0, 64);
      const int r1 = __shfl(my_src, j1 < 0 ? j0 : j1, 64);
      const float w1 = __shfl(my_w, j1 < 0 ? j0 : j1, 64);
      i32x4_t a[4], b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = v0 + u * 64 + lane;
        if (v < nvec) {
          a[u] = reinterpret_cast<const i32x4_t*>(yperm + (int64_t)r0 * d)[v];
          if (j1 >= 0) b[u] = reinterpret_cast<const i32x4_t*>(yperm + (int64_t)r1 * d)[v];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = v0 + u * 64 + lane;
        if (v < nvec) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[u][2 * q] = fmaf(w0, __uint_as_float(((uint32_t)a[u][q]) << 16), acc[u][2 * q]);
            acc[u][2 * q + 1] = fmaf(w0, __uint_as_float(((uint32_t)a[u][q]) & 0xffff0000u), acc[u][2 * q + 1]);
          }
          if (j1 >= 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              acc[u][2 * q] = fmaf(w1, __uint_as_float(((uint32_t)b[u][q]) << 16), acc[u][2 * q]);
              acc[u][2 * q + 1] = fmaf(w1, __uint_as_float(((uint32_t)b[u][q]) & 0xffff0000u), acc[u][2 * q + 1]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int v = v0 + u * 64 + lane;
      if (v >= nvec) continue;
      float res[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) res[q] = 0.0f;
      if constexpr (MASK) {
        // the dropout keep factors of these 8 elements, folded into the accumulators
        const uint2 kv = reinterpret_cast<const uint2*>(keep + o * d)[v];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t byte = ((q < 4 ? kv.x : kv.y) >> (8 * (q & 3))) & 0xffu;
          acc[u][q] *= byte ? keep_scale : 0.0f;
        }
      }
      if constexpr (RES) {
        if (OUT_F32) {
          const f32x4_t* rp = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(residual) + o * d) + 2 * v;
          const f32x4_t r0v = rp[0], r1v = rp[1];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            res[q] = r0v[q];
            res[4 + q] = r1v[q];
          }
        } else {
          const i32x4_t rv = reinterpret_cast<const i32x4_t*>(static_cast<const uint16_t*>(residual) + o * d)[v];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            res[2 * q] = __uint_as_float(((uint32_t)rv[q]) << 16);
            res[2 * q + 1] = __uint_as_float(((uint32_t)rv[q]) & 0xffff0000u);
          }
        }
      }
      if (OUT_F32) {
        f32x4_t* dst = reinterpret_cast<f32x4_t*>(static_cast<float*>(y) + o * d) + 2 * v;
        dst[0] = f32x4_t{fmaf(acc[u][0], sc, res[0]), fmaf(acc[u][1], sc, res[1]), fmaf(acc[u][2], sc, res[2]),
                         fmaf(acc[u][3], sc, res[3])};
        dst[1] = f32x4_t{fmaf(acc[u][4], sc, res[4]), fmaf(acc[u][5], sc, res[5]), fmaf(acc[u][6], sc, res[6]),
                         fmaf(acc[u][7], sc, res[7])};
      } else {
        i32x4_t out;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          out[q] = (int)((uint32_t)f32_to_bf16(fmaf(acc[u][2 * q], sc, res[2 * q])) |
                         ((uint32_t)f32_to_bf16(fmaf(acc[u][2 * q + 1], sc, res[2 * q + 1])) << 16));
        reinterpret_cast<i32x4_t*>(static_cast<uint16_t*>(y) + o * d)[v] = out;
      }
    }
  }
}

// Two sources per output row (token choice, top-2), bf16 out, d == 2048: one wave per
// row, its two source indices and weights loaded by two lanes and broadcast, all 8
// row loads of a lane issued at once.  The arithmetic is combine_kernel's for
// fan = 2 (fp32 fma from +0 in source order, dropped sources skipped), so the
// results are bit-identical; the straight-line form runs 37.8 -> 33.8 us at config 2
// (the source loop's ballot / shuffle / bounds bookkeeping delayed the loads).
constexpr int C2_D = 2048;
template <bool RES = false, bool MASK = false>
__global__ __launch_bounds__(256) void combine2_kernel(const uint16_t* __restrict__ yperm,
                                                       const int32_t* __restrict__ src_row,
                                                       const float* __restrict__ src_w,
                                                       const int32_t* __restrict__ out_map,
                                                       const float* __restrict__ scale, int64_t T_out,
                                                       uint16_t* __restrict__ y,
                                                       const uint16_t* __restrict__ residual,
                                                       const uint8_t* __restrict__ keep, float keep_scale) {
  constexpr int NV = C2_D / 8 / 64;  // 16-byte vectors per lane
  const int lane = threadIdx.x & 63;
  const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= T_out) return;
  const int64_t s = out_map ? (int64_t)out_map[o] : o;
  i32x4_t* dst = reinterpret_cast<i32x4_t*>(y + o * C2_D);
  if (s < 0) {
#pragma unroll
    for (int u = 0; u < NV; ++u)
      dst[u * 64 + lane] =
          RES ? reinterpret_cast<const i32x4_t*>(residual + o * C2_D)[u * 64 + lane] : i32x4_t{0, 0, 0, 0};
    return;
  }
  int ms = -1;
  float mw = 0.0f;
  if (lane < 2) {
    ms = src_row[s * 2 + lane];
    mw = src_w[s * 2 + lane];
  }
  const int r0 = __shfl(ms, 0, 64), r1 = __shfl(ms, 1, 64);
  const float w0 = __shfl(mw, 0, 64), w1 = __shfl(mw, 1, 64);
  const float sc = scale ? scale[s] : 1.0f;
  i32x4_t a[NV], b[NV], rr[RES ? NV : 1];
  uint2 kv[MASK ? NV : 1];
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    a[u] = r0 >= 0 ? reinterpret_cast<const i32x4_t*>(yperm + (int64_t)r0 * C2_D)[u * 64 + lane] : i32x4_t{0, 0, 0, 0};
    b[u] = r1 >= 0 ? reinterpret_cast<const i32x4_t*>(yperm + (int64_t)r1 * C2_D)[u * 64 + lane] : i32x4_t{0, 0, 0, 0};
    if constexpr (RES) rr[u] = reinterpret_cast<const i32x4_t*>(residual + o * C2_D)[u * 64 + lane];
    if constexpr (MASK) kv[u] = reinterpret_cast<const uint2*>(keep + o * C2_D)[u * 64 + lane];
  }
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    i32x4_t out;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float lo = 0.0f, hi = 0.0f;
      if (r0 >= 0) {
        lo = fmaf(w0, __uint_as_float(((uint32_t)a[u][q]) << 16), lo);
        hi = fmaf(w0, __uint_as_float(((uint32_t)a[u][q]) & 0xffff0000u), hi);
      }
      if (r1 >= 0) {
        lo = fmaf(w1, __uint_as_float(((uint32_t)b[u][q]) << 16), lo);
        hi = fmaf(w1, __uint_as_float(((uint32_t)b[u][q]) & 0xffff0000u), hi);
      }
      float rlo = 0.0f, rhi = 0.0f;
      if constexpr (RES) {
        rlo = __uint_as_float(((uint32_t)rr[u][q]) << 16);
        rhi = __uint_as_float(((uint32_t)rr[u][q]) & 0xffff0000u);
      }
      if constexpr (MASK) {
        // elements 2q and 2q+1 of this vector: bytes 2q, 2q+1 of the 8 keep bytes
        const uint32_t w32 = q < 2 ? kv[u].x : kv[u].y;
        lo *= ((w32 >> (16 * (q & 1))) & 0xffu) ? keep_scale : 0.0f;
        hi *= ((w32 >> (16 * (q & 1) + 8)) & 0xffu) ? keep_scale : 0.0f;
      }
      out[q] = (int)((uint32_t)f32_to_bf16(fmaf(lo, sc, rlo)) | ((uint32_t)f32_to_bf16(fmaf(hi, sc, rhi)) << 16));
    }
    dst[u * 64 + lane] = out;
  }
}

}  // namespace

namespace {
int combine_launch(const char* who, const void* yperm, int d, const int32_t* src_row, const float* src_w, int fan,
                   const int32_t* out_map, const float* scale, const void* residual, const uint8_t* keep,
                   float keep_scale, int64_t T_out, void* y, int y_dtype, void* stream) {
  KMOE_REQUIRE(yperm && src_row && src_w && y, KMOE_ERR_NULL, "%s: null buffer", who);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "%s: d=%d must be a positive multiple of 64", who, d);
  KMOE_REQUIRE(fan >= 1 && fan <= 64, KMOE_ERR_SHAPE, "%s: fan=%d not in [1,64]", who, fan);
  KMOE_REQUIRE(T_out >= 0, KMOE_ERR_SHAPE, "%s: T_out < 0", who);
  KMOE_REQUIRE(y_dtype == KMOE_DTYPE_BF16 || y_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "%s: y dtype must be bf16 or f32", who);
  if (T_out == 0) return KMOE_OK;
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T_out, CROWS));
  hipStream_t s = kmoe::as_stream(stream);
  const uint16_t* yp = static_cast<const uint16_t*>(yperm);
  const bool bf = y_dtype == KMOE_DTYPE_BF16;
  uint16_t* y16 = static_cast<uint16_t*>(y);
  const uint16_t* r16 = static_cast<const uint16_t*>(residual);
  if (bf && fan == 2 && d == C2_D) {
#define KMOE_COMBINE2(RES_, MASK_)                                                                             \
  hipLaunchKernelGGL((combine2_kernel<RES_, MASK_>), grid, dim3(256), 0, s, yp, src_row, src_w, out_map, scale, \
                     T_out, y16, r16, keep, keep_scale)
    if (keep)
      KMOE_COMBINE2(true, true);
    else if (residual)
      KMOE_COMBINE2(true, false);
    else
      KMOE_COMBINE2(false, false);
#undef KMOE_COMBINE2
  } else {
#define KMOE_COMBINE(F32_, RES_, MASK_)                                                                            \
  hipLaunchKernelGGL((combine_kernel<F32_, RES_, MASK_>), grid, dim3(64 * CROWS), 0, s, yp, d, src_row, src_w, fan, \
                     out_map, scale, T_out, y, residual, keep, keep_scale)
    if (bf && keep)
      KMOE_COMBINE(false, true, true);
    else if (bf && residual)
      KMOE_COMBINE(false, true, false);
    else if (bf)
      KMOE_COMBINE(false, false, false);
    else if (keep)
      KMOE_COMBINE(true, true, true);
    else if (residual)
      KMOE_COMBINE(true, true, false);
    else
      KMOE_COMBINE(true, false, false);
#undef KMOE_COMBINE
  }
  return kmoe::check_launch(who);
}
}  // namespace

extern "C" int kmoe_combine_residual(const void* yperm, int d, const int32_t* src_row, const float* src_w,
                                     int fan, const int32_t* out_map, const float* scale, const void* residual,
                                     int64_t T_out, void* y, int y_dtype, void* stream) {
  return combine_launch("kmoe_combine", yperm, d, src_row, src_w, fan, out_map, scale, residual, nullptr, 1.0f,
                        T_out, y, y_dtype, stream);
}

extern "C" int kmoe_combine_residual_dropout(const void* yperm, int d, const int32_t* src_row, const float* src_w,
                                             int fan, const int32_t* out_map, const float* scale,
                                             const void* residual, const uint8_t* keep, float keep_scale,
                                             int64_t T_out, void* y, int y_dtype, void* stream) {
  KMOE_REQUIRE(residual && keep, KMOE_ERR_NULL, "kmoe_combine_residual_dropout: null residual / keep mask");
  KMOE_REQUIRE(keep_scale >= 1.0f, KMOE_ERR_SHAPE,
               "kmoe_combine_residual_dropout: keep_scale=%g must be 1/(1-p) >= 1", (double)keep_scale);
  return combine_launch("kmoe_combine_residual_dropout", yperm, d, src_row, src_w, fan, out_map, scale, residual,
                        keep, keep_scale, T_out, y, y_dtype, stream);
}

extern "C" int kmoe_combine(const void* yperm, int d, const int32_t* src_row, const float* src_w, int fan,
                            const int32_t* out_map, const float* scale, int64_t T_out, void* y, int y_dtype,
                            void* stream) {
  return kmoe_combine_residual(yperm, d, src_row, src_w, fan, out_map, scale, nullptr, T_out, y, y_dtype, stream);
}
