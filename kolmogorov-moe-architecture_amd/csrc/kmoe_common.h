// Shared device/host helpers for the kmoe HIP kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "kmoe.h"

// ---------------------------------------------------------------- vector types
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));

#define KMOE_LDS __attribute__((address_space(3)))

// ---------------------------------------------------------------- error state
namespace kmoe {

void set_error(const char* fmt, ...);
int check_launch(const char* what);
// compute units of the current device (cached per device): the grid of persistent kernels
int cu_count();
// Tokens per router workgroup for a call over T tokens (32 when 32-token tiles fit the
// device in one wave of workgroups, else 64): also the token span of one row of the
// router's aux partials and block histograms, which the aux-loss and dispatch
// reductions read.
int router_block_tokens(int64_t T);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

template <typename T>
inline T ceil_div(T a, T b) { return (a + b - 1) / b; }

}  // namespace kmoe

#define KMOE_REQUIRE(cond, code, ...)      \
  do {                                     \
    if (!(cond)) {                         \
      kmoe::set_error(__VA_ARGS__);        \
      return (code);                       \
    }                                      \
  } while (0)

// ---------------------------------------------------------------- device math
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }
// SiLU with a hardware reciprocal (1 ulp) instead of an IEEE divide: for values
// that are rounded to bf16 right after.
__device__ __forceinline__ float silu_fast_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// fp32 -> OCP e4m3fn, saturating to +-448, round-to-nearest-even.  Pure integer
// arithmetic, so it is specified exactly (the oracle restates it in numpy).
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  if (f != f) return sign | 0x7fu;  // NaN stays NaN
  float a = fminf(fabsf(f), 448.0f);
  uint32_t ua = __float_as_uint(a);
  int exp = (int)(ua >> 23) - 127;
  uint32_t code;
  if (exp < -6) {
    // subnormal range of e4m3: value = m * 2^-9, m in [0, 8]
    // a * 2^9 rounded to nearest even integer
    float s = a * 512.0f;              // exact (power-of-two scaling)
    float r = __builtin_rintf(s);      // RNE
    code = (uint32_t)r;                // 8 -> becomes the smallest normal (exp field 1, mant 0)
  } else {
    uint32_t mant = ua & 0x7fffffu;
    uint32_t m3 = mant >> 20;
    uint32_t rest = mant & 0xfffffu;
    uint32_t half = 0x80000u;
    uint32_t e = (uint32_t)(exp + 7);
    code = (e << 3) | m3;
    if (rest > half || (rest == half && (m3 & 1u))) code += 1u;  // carries into exponent correctly
    if (code > 0x7eu) code = 0x7eu;  // saturate (448 = 0x7e)
  }
  return sign | code;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t s = c & 0x80u, e = (c >> 3) & 15u, m = c & 7u;
  float v = e == 0 ? (float)m * (1.0f / 512.0f) : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

// Workgroup barrier without a memory fence.  __syncthreads() also waits for every
// outstanding global load (vmcnt(0)), which would drain in-flight prefetches of
// direct-to-LDS pipelines; callers wait explicitly for what they need (vmcnt(N)
// for their own tile loads, lgkmcnt(0) after LDS writes) before calling this.
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4): the 64 lanes'
// data lands at consecutive 16-byte slots from `lds` (a wave-uniform LDS address, M0).
// Issued through inline asm on purpose: the compiler does not see these LDS writes, so it
// adds no waits of its own for them.  For the builtin form it cannot tell the pipeline
// stages apart and puts a vmcnt(0) (wait for every load in flight, including the ones
// just issued for a later stage) in front of the next LDS read, which serialises a
// multi-stage pipeline.  Callers order these loads with explicit wait_vmcnt<N>() and a
// barrier before any lane reads the data.  Compiler-generated vmcnt waits for ordinary
// loads stay correct (vmcnt counts all vector-memory loads in issue order, so extra
// loads in flight only make them wait longer).
__device__ __forceinline__ void dma16_to_lds(const void* src, KMOE_LDS void* lds) {
  const uint32_t la = (uint32_t)(uintptr_t)lds;
  // s_nop: the wait states gfx9 requires between an SALU write of M0 and an LDS-DMA
  // instruction reading it (the compiler inserts them for its own instructions only)
  asm volatile("s_nop 1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(la)));
}

// Lane l's value from lane l ^ M (M = 1 or 2) of its group of four lanes, in one DPP
// move (quad_perm [1,0,3,2] / [2,3,0,1]) instead of an LDS-crossbar permute.  Every
// lane of the quad must be active.
template <int M>
__device__ __forceinline__ int quad_xor(int v) {
  static_assert(M == 1 || M == 2, "lanes of a quad");
  return __builtin_amdgcn_update_dpp(0, v, M == 1 ? 0xB1 : 0x4E, 0xF, 0xF, false);
}
template <int M>
__device__ __forceinline__ float quad_xor(float v) {
  return __int_as_float(quad_xor<M>(__float_as_int(v)));
}

// Wave-level reductions (64 lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Auxiliary losses from the router's per-block partial sums (moe.py:840-939): column c
// of block b is partials[b (E + 1) + c], the block's summed softmax probabilities of
// expert c (c < E) or its summed lse^2 (c = E).  aux_reduce_cols: wave w of `nw` waves
// reduces columns w, w + nw, ...; lane l sums blocks l, l + 64, ... in order, then the
// wave sums its lanes with a fixed shuffle tree, so the result does not depend on the
// launch (bit-reproducible).  The loads go out 16 at a time (4 columns x 4 blocks), the
// sums stay in block order.  col[] lives in LDS; the caller synchronises before
// aux_finish reads it.
__device__ __forceinline__ void aux_reduce_cols(const float* __restrict__ partials, int64_t nblk, int E, int wave,
                                                int nw, int lane, float* col) {
  for (int c0 = wave; c0 <= E; c0 += 4 * nw) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t b = lane;
    for (; b + 192 < nblk; b += 256) {
      float v[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = c0 + q * nw;
          v[q][u] = c <= E ? partials[(b + 64 * u) * (E + 1) + c] : 0.0f;
        }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) s[q] += v[q][u];
    }
    for (; b < nblk; b += 64)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = c0 + q * nw;
        if (c <= E) s[q] += partials[b * (E + 1) + c];
      }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = c0 + q * nw;  // wave-uniform
      if (c <= E) {
        const float t = wave_sum(s[q]);
        if (lane == 0) col[c] = t;
      }
    }
  }
}
// out = (w_lb lb + w_z z, lb, z): lb = E sum_e (counts[e] / (T k)) (P_e / T) (0 without
// counts), z = mean lse^2.  One thread.
__device__ __forceinline__ void aux_finish(const float* col, const int32_t* counts, int64_t T, int E, int k,
                                           float w_lb, float w_z, float* __restrict__ out) {
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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ---------------------------------------------------------------- fp8 rows
// One wave quantises one bf16 row of `nvec` 16-byte vectors to e4m3 with the
// per-row scale amax/448: the row is read once into registers (lane l holds
// vectors l, l+64, ...; up to ROW_REGS per lane, i.e. rows of up to 8192 bf16),
// its amax reduced across the wave, then quantised from the registers.
constexpr int ROW_REGS = 16;
struct RowRegs {
  i32x4_t v[ROW_REGS];
};
__device__ __forceinline__ float bf16_pair_absmax(uint32_t w) {
  return fmaxf(fabsf(__uint_as_float(w << 16)), fabsf(__uint_as_float(w & 0xffff0000u)));
}
__device__ __forceinline__ float load_row_amax(const i32x4_t* __restrict__ src, int nvec, int lane, RowRegs& r) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < ROW_REGS; ++i) {
    const int v = lane + 64 * i;
    if (v < nvec) {
      r.v[i] = src[v];
#pragma unroll
      for (int q = 0; q < 4; ++q) amax = fmaxf(amax, bf16_pair_absmax((uint32_t)r.v[i][q]));
    }
  }
  return wave_max(amax);
}
// Four values to e4m3 bytes (a in byte 0) with the rule of f32_to_e4m3, on the
// hardware converter: |x| > 448 (and +-inf) is clamped to +-448 first, so the
// converter only sees finite values in range, where its round-to-nearest-even
// equals the integer rule above on every fp32 bit pattern (checked exhaustively
// on gfx950); NaN keeps its sign as sign | 0x7f (the converter writes 0xff).
__device__ __forceinline__ float sat448(float f) { return fabsf(f) > 448.0f ? copysignf(448.0f, f) : f; }
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), r, true);
  uint32_t u = (uint32_t)r;
  if (a != a || b != b || c != c || d != d) {
    const float v[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (v[i] != v[i]) u = (u & ~(0xffu << (8 * i))) | ((((__float_as_uint(v[i]) >> 24) & 0x80u) | 0x7fu) << (8 * i));
  }
  return u;
}
// e4m3 bytes of one 16-byte bf16 vector (8 values) as two 32-bit words
__device__ __forceinline__ void quant_vec_e4m3(const i32x4_t& val, float inv, uint32_t& lo, uint32_t& hi) {
  const uint32_t w0 = (uint32_t)val[0], w1 = (uint32_t)val[1], w2 = (uint32_t)val[2], w3 = (uint32_t)val[3];
  lo = e4m3x4(__uint_as_float(w0 << 16) * inv, __uint_as_float(w0 & 0xffff0000u) * inv,
              __uint_as_float(w1 << 16) * inv, __uint_as_float(w1 & 0xffff0000u) * inv);
  hi = e4m3x4(__uint_as_float(w2 << 16) * inv, __uint_as_float(w2 & 0xffff0000u) * inv,
              __uint_as_float(w3 << 16) * inv, __uint_as_float(w3 & 0xffff0000u) * inv);
}
