// RMSNorm forward and backward at the MoE block's boundary, for the training path.
//
// RMSNorm (moe_arch/model/embeddings.py:167-195):  n = g * x * r,  r = 1/sqrt(mean(x^2) + eps)
// Backward, per row (d columns):
//   dx_c = r g_c dn_c - (r^3 / d) x_c sum_c' g_c' dn_c' x_c'   (+ dres_c, the residual's gradient)
//   dg_c = sum_t dn_tc x_tc r_t
// Both kernels hold one row per wave in registers (lane l holds the 8-element vectors
// l, l + 64, ... of the row), so each row is read once; HBM-bound.  The training
// forward materialises n (bf16): the backward's weight gradients need the normalised
// rows, which the inference path's fold of g into the weights never writes.
#include "kmoe_common.h"

namespace {

// Rows in flight per workgroup, and the most row segments of the backward (each writes a
// d-float partial of dg that a second kernel reduces).  Measured at T = 16384, d = 2048:
// 4 waves / 1024 segments 58 us, 4 / 512 52, 8 / 512 54, 8 / 256 50.5, 4 / 4096 121
// (the partial sums' reduction dominates with many segments).
constexpr int NORM_WAVES = 8;
constexpr int NORM_MAX_SEGS = 256;
constexpr int NORM_FWD_WAVES = 4;  // forward: one row per wave, 4 per workgroup (8: 32 -> 37 us)

// 8 consecutive elements (bf16 or f32) as floats
template <bool F32>
__device__ __forceinline__ void load8(const void* __restrict__ base, int64_t elem, float (&v)[8]) {
  if constexpr (F32) {
    const f32x4_t* p = reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + elem);
    const f32x4_t a = p[0], b = p[1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = a[q];
      v[4 + q] = b[q];
    }
  } else {
    const i32x4_t a = *reinterpret_cast<const i32x4_t*>(static_cast<const uint16_t*>(base) + elem);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(((uint32_t)a[q]) << 16);
      v[2 * q + 1] = __uint_as_float(((uint32_t)a[q]) & 0xffff0000u);
    }
  }
}

template <bool F32>
__device__ __forceinline__ void store8(void* __restrict__ base, int64_t elem, const float (&v)[8]) {
  if constexpr (F32) {
    f32x4_t a, b;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = v[q];
      b[q] = v[4 + q];
    }
    f32x4_t* p = reinterpret_cast<f32x4_t*>(static_cast<float*>(base) + elem);
    p[0] = a;
    p[1] = b;
  } else {
    i32x4_t a;
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = (int)((uint32_t)f32_to_bf16(v[2 * q]) | ((uint32_t)f32_to_bf16(v[2 * q + 1]) << 16));
    *reinterpret_cast<i32x4_t*>(static_cast<uint16_t*>(base) + elem) = a;
  }
}

__device__ __forceinline__ void load8_any(const void* __restrict__ base, bool f32, int64_t elem, float (&v)[8]) {
  if (f32)
    load8<true>(base, elem, v);
  else
    load8<false>(base, elem, v);
}

// n[t] = bf16(g * x[t] * r_t), rrms[t] = r_t.  One wave per row.  With w_mod, also
// mod_logits[t] = n[t] . w_mod over the rounded n, in the lane / vector / wave-sum order
// of the MoD selection's own logits kernel (so the selection is the same as from n).
template <int NV, bool XF32>
__global__ __launch_bounds__(64 * NORM_FWD_WAVES) void rmsnorm_kernel(const void* __restrict__ x,
                                                                  const void* __restrict__ g, bool g_f32, float eps,
                                                                  int64_t T, int d, uint16_t* __restrict__ n,
                                                                  float* __restrict__ rrms,
                                                                  const uint16_t* __restrict__ w_mod,
                                                                  float* __restrict__ mod_logits) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * NORM_FWD_WAVES + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nvec = d / 8;
  float xv[NV][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v < nvec) {
      load8<XF32>(x, t * d + (int64_t)v * 8, xv[i]);
#pragma unroll
      for (int q = 0; q < 8; ++q) ss = fmaf(xv[i][q], xv[i][q], ss);
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)d + eps);
  float ml = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v < nvec) {
      float gv[8], o[8];
      load8_any(g, g_f32, (int64_t)v * 8, gv);
#pragma unroll
      for (int q = 0; q < 8; ++q) o[q] = gv[q] * (xv[i][q] * r);
      store8<false>(n, t * d + (int64_t)v * 8, o);
      if (w_mod) {
        float wv[8];
        load8<false>(w_mod, (int64_t)v * 8, wv);
#pragma unroll
        for (int q = 0; q < 8; ++q) ml = fmaf(bf16_to_f32(f32_to_bf16(o[q])), wv[q], ml);
      }
    }
  }
  if (w_mod) {
    ml = wave_sum(ml);
    if (lane == 0) mod_logits[t] = ml;
  }
  if (lane == 0) rrms[t] = r;
}

// One row's inputs as loaded (bf16: one 16-byte vector per 8 elements, f32: two).
template <bool F32>
struct Raw8 {
  i32x4_t v[F32 ? 2 : 1];
};
template <bool F32>
__device__ __forceinline__ void load_raw(const void* __restrict__ base, int64_t elem, Raw8<F32>& r) {
  const i32x4_t* p = reinterpret_cast<const i32x4_t*>(static_cast<const uint8_t*>(base) + elem * (F32 ? 4 : 2));
  r.v[0] = p[0];
  if constexpr (F32) r.v[1] = p[1];
}
template <bool F32>
__device__ __forceinline__ void unpack_raw(const Raw8<F32>& r, float (&v)[8]) {
  if constexpr (F32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = __int_as_float(r.v[0][q]);
      v[4 + q] = __int_as_float(r.v[1][q]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(((uint32_t)r.v[0][q]) << 16);
      v[2 * q + 1] = __uint_as_float(((uint32_t)r.v[0][q]) & 0xffff0000u);
    }
  }
}

template <int NV, bool XF32>
struct NormRow {
  Raw8<XF32> x[NV], res[NV];
  Raw8<false> dn[NV];
  float r;
};

// dx (dtype of x) and the per-segment partial sums of dg.  Workgroup = NORM_WAVES waves
// over the rows [seg * seg_rows, ...) of its segment, wave w taking every NORM_WAVES-th
// row (its x, dn and dres loads issued together); the waves' dg sums are then added in
// wave order through LDS and written as partial[seg][:] (reduced over segments afterwards
// in a fixed order).
template <int NV, bool XF32>
__global__ __launch_bounds__(64 * NORM_WAVES) void rmsnorm_bwd_kernel(
    const uint16_t* __restrict__ dn, const void* __restrict__ x, const void* __restrict__ g, bool g_f32,
    const float* __restrict__ rrms, const void* __restrict__ dres, int64_t T, int d, int64_t seg_rows,
    void* __restrict__ dx, float* __restrict__ partial) {
  __shared__ float red[NORM_WAVES][512];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nvec = d / 8;
  float gv[NV][8], acc[NV][8];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      gv[i][q] = 0.0f;
      acc[i][q] = 0.0f;
    }
    if (v < nvec) load8_any(g, g_f32, (int64_t)v * 8, gv[i]);
  }
  const int64_t t0 = (int64_t)blockIdx.x * seg_rows;
  const int64_t t1 = t0 + seg_rows < T ? t0 + seg_rows : T;
  const float inv_d = 1.0f / (float)d;
  auto load_row = [&](int64_t t, NormRow<NV, XF32>& R) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) {
        load_raw<XF32>(x, t * d + (int64_t)v * 8, R.x[i]);
        load_raw<false>(dn, t * d + (int64_t)v * 8, R.dn[i]);
        if (dres) load_raw<XF32>(dres, t * d + (int64_t)v * 8, R.res[i]);
      }
    }
    R.r = rrms[t];
  };
  auto process = [&](int64_t t, const NormRow<NV, XF32>& R) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) {
        float xv[8], dv[8];
        unpack_raw<XF32>(R.x[i], xv);
        unpack_raw<false>(R.dn[i], dv);
#pragma unroll
        for (int q = 0; q < 8; ++q) s = fmaf(gv[i][q] * dv[q], xv[q], s);
      }
    }
    s = wave_sum(s);
    const float r = R.r;
    const float c = r * r * r * s * inv_d;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) {
        float xv[8], dv[8], rv[8], o[8];
        unpack_raw<XF32>(R.x[i], xv);
        unpack_raw<false>(R.dn[i], dv);
        if (dres) {
          unpack_raw<XF32>(R.res[i], rv);
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q) rv[q] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          o[q] = rv[q] + (r * gv[i][q] * dv[q] - c * xv[q]);
          acc[i][q] = fmaf(dv[q] * xv[q], r, acc[i][q]);
        }
        store8<XF32>(dx, t * d + (int64_t)v * 8, o);
      }
    }
  };
  // one row at a time: a second row in flight (prefetch) needs 256 VGPRs at d = 2048 and
  // the lower occupancy made the kernel slower (75 vs 58 us at T = 16384, d = 2048)
  NormRow<NV, XF32> ra;
  for (int64_t t = t0 + w; t < t1; t += NORM_WAVES) {
    load_row(t, ra);
    process(t, ra);
  }
  // dg: per 512-column chunk, the waves' sums added in wave order
  float* out = partial + (int64_t)blockIdx.x * d;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
#pragma unroll
    for (int q = 0; q < 8; ++q) red[w][lane * 8 + q] = acc[i][q];
    __syncthreads();
    for (int c = threadIdx.x; c < 512; c += 64 * NORM_WAVES) {
      const int col = i * 512 + c;
      if (col < d) {
        float sum = red[0][c];
#pragma unroll
        for (int q = 1; q < NORM_WAVES; ++q) sum += red[q][c];
        out[col] = sum;
      }
    }
    __syncthreads();
  }
}

int64_t norm_seg_rows(int64_t T) {
  int64_t rows = kmoe::ceil_div<int64_t>(T, NORM_MAX_SEGS);
  rows = kmoe::ceil_div<int64_t>(rows, NORM_WAVES) * NORM_WAVES;
  return rows < NORM_WAVES ? NORM_WAVES : rows;
}

template <bool XF32>
int launch_norm(const void* x, const void* g, bool g_f32, float eps, int64_t T, int d, uint16_t* n, float* rrms,
                const uint16_t* w_mod, float* mod_logits, hipStream_t s) {
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T, NORM_FWD_WAVES)), block(64 * NORM_FWD_WAVES);
  const int nv = kmoe::ceil_div(d / 8, 64);
#define KMOE_NORM_CASE(NVV)                                                                                   \
  if (nv <= NVV) {                                                                                            \
    hipLaunchKernelGGL((rmsnorm_kernel<NVV, XF32>), grid, block, 0, s, x, g, g_f32, eps, T, d, n, rrms,    \
                       w_mod, mod_logits);                                                                  \
    return KMOE_OK;                                                                                           \
  }
  KMOE_NORM_CASE(1)
  KMOE_NORM_CASE(2)
  KMOE_NORM_CASE(4)
  KMOE_NORM_CASE(8)
  KMOE_NORM_CASE(16)
#undef KMOE_NORM_CASE
  return KMOE_ERR_UNSUPPORTED;
}

template <bool XF32>
int launch_norm_bwd(const uint16_t* dn, const void* x, const void* g, bool g_f32, const float* rrms, const void* dres,
                    int64_t T, int d, int64_t seg_rows, void* dx, float* partial, hipStream_t s) {
  const dim3 grid((unsigned)kmoe::ceil_div<int64_t>(T, seg_rows)), block(64 * NORM_WAVES);
  const int nv = kmoe::ceil_div(d / 8, 64);
#define KMOE_NORM_CASE(NVV)                                                                              \
  if (nv <= NVV) {                                                                                       \
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<NVV, XF32>), grid, block, 0, s, dn, x, g, g_f32, rrms, dres, T, \
                       d, seg_rows, dx, partial);                                                        \
    return KMOE_OK;                                                                                      \
  }
  KMOE_NORM_CASE(1)
  KMOE_NORM_CASE(2)
  KMOE_NORM_CASE(4)
  KMOE_NORM_CASE(8)
  KMOE_NORM_CASE(16)
#undef KMOE_NORM_CASE
  return KMOE_ERR_UNSUPPORTED;
}

__global__ void zero_words_kernel(uint16_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

bool is_float_dtype(int dt) { return dt == KMOE_DTYPE_BF16 || dt == KMOE_DTYPE_F32; }

}  // namespace

extern "C" int kmoe_rmsnorm(const void* x, int x_dtype, const void* weight, int w_dtype, float eps, int64_t T, int d,
                            void* n, float* rrms, const void* w_mod, float* mod_logits, void* stream) {
  KMOE_REQUIRE(weight && (T == 0 || (x && n && rrms)), KMOE_ERR_NULL, "kmoe_rmsnorm: null buffer");
  KMOE_REQUIRE(!w_mod == !mod_logits, KMOE_ERR_NULL, "kmoe_rmsnorm: w_mod and mod_logits go together");
  KMOE_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(w_dtype), KMOE_ERR_DTYPE, "kmoe_rmsnorm: dtypes %d/%d",
               x_dtype, w_dtype);
  KMOE_REQUIRE(T >= 0 && d > 0 && d % 8 == 0, KMOE_ERR_SHAPE, "kmoe_rmsnorm: d=%d must be a positive multiple of 8",
               d);
  KMOE_REQUIRE(d <= 8192, KMOE_ERR_UNSUPPORTED, "kmoe_rmsnorm: d=%d > 8192", d);
  KMOE_REQUIRE(eps >= 0.0f, KMOE_ERR_SHAPE, "kmoe_rmsnorm: eps must be >= 0");
  if (T == 0) return KMOE_OK;
  hipStream_t s = kmoe::as_stream(stream);
  const bool g_f32 = w_dtype == KMOE_DTYPE_F32;
  const uint16_t* wm = static_cast<const uint16_t*>(w_mod);
  const int rc =
      x_dtype == KMOE_DTYPE_F32
          ? launch_norm<true>(x, weight, g_f32, eps, T, d, static_cast<uint16_t*>(n), rrms, wm, mod_logits, s)
          : launch_norm<false>(x, weight, g_f32, eps, T, d, static_cast<uint16_t*>(n), rrms, wm, mod_logits, s);
  if (rc != KMOE_OK) return rc;
  return kmoe::check_launch("kmoe_rmsnorm");
}

extern "C" size_t kmoe_rmsnorm_bwd_workspace_bytes(int64_t T, int d) {
  if (T <= 0 || d <= 0) return 0;
  return (size_t)kmoe::ceil_div<int64_t>(T, norm_seg_rows(T)) * (size_t)d * sizeof(float);
}

extern "C" int kmoe_rmsnorm_bwd(const void* dn, const void* x, int x_dtype, const void* weight, int w_dtype,
                                const float* rrms, const void* dres, int64_t T, int d, void* dx, void* dweight,
                                int dw_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  // with no rows only the weight gradient (zeros) is written
  KMOE_REQUIRE(weight && dweight && (T == 0 || (dn && x && rrms && dx)), KMOE_ERR_NULL,
               "kmoe_rmsnorm_bwd: null buffer");
  KMOE_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(w_dtype) && is_float_dtype(dw_dtype), KMOE_ERR_DTYPE,
               "kmoe_rmsnorm_bwd: dtypes %d/%d/%d", x_dtype, w_dtype, dw_dtype);
  KMOE_REQUIRE(T >= 0 && d > 0 && d % 8 == 0, KMOE_ERR_SHAPE,
               "kmoe_rmsnorm_bwd: d=%d must be a positive multiple of 8", d);
  KMOE_REQUIRE(d <= 8192, KMOE_ERR_UNSUPPORTED, "kmoe_rmsnorm_bwd: d=%d > 8192", d);
  hipStream_t s = kmoe::as_stream(stream);
  if (T == 0) {  // no rows: dg = 0 (a fill kernel, so the call stays capturable)
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)kmoe::ceil_div(d, 256)), dim3(256), 0, s,
                       static_cast<uint16_t*>(dweight), (int64_t)d * (dw_dtype == KMOE_DTYPE_F32 ? 2 : 1));
    return kmoe::check_launch("kmoe_rmsnorm_bwd");
  }
  const size_t need = kmoe_rmsnorm_bwd_workspace_bytes(T, d);
  KMOE_REQUIRE(workspace && workspace_bytes >= need, KMOE_ERR_WORKSPACE,
               "kmoe_rmsnorm_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  const int64_t seg_rows = norm_seg_rows(T);
  const int64_t nseg = kmoe::ceil_div<int64_t>(T, seg_rows);
  float* partial = static_cast<float*>(workspace);
  const bool g_f32 = w_dtype == KMOE_DTYPE_F32;
  const uint16_t* dnp = static_cast<const uint16_t*>(dn);
  const int rc = x_dtype == KMOE_DTYPE_F32
                     ? launch_norm_bwd<true>(dnp, x, weight, g_f32, rrms, dres, T, d, seg_rows, dx, partial, s)
                     : launch_norm_bwd<false>(dnp, x, weight, g_f32, rrms, dres, T, d, seg_rows, dx, partial, s);
  if (rc != KMOE_OK) return rc;
  const int rc2 = kmoe::check_launch("kmoe_rmsnorm_bwd");
  if (rc2 != KMOE_OK) return rc2;
  return kmoe_reduce_f32(partial, nseg, d, dweight, dw_dtype, stream);
}
