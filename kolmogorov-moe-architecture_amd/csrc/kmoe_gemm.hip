// Grouped SwiGLU expert GEMMs on CDNA4 MFMA.
// Replaces moe_kernels.grouped_swiglu_forward (moe_arch/kernels/grouped_gemm.cu:186-257)
// and the padded bmm block of GroupedExperts.forward (moe_arch/model/moe.py:275-279):
//   gate_up:  h[r, f] = silu(x[r] . w1[e][:, f]) * (x[r] . w2[e][:, f])     (ffn.py:17-64)
//   down:     y[r, n] = h[r] . w3[e][:, n]
// for the rows r of expert e, [offsets[e], offsets[e+1]).
//
// Tiling: a workgroup of 8 waves (2 per SIMD) owns a 256-row x 256-B-row tile;
// waves form 2 (rows) x 4 (B rows) and each computes 128 x 64 as 4x2 blocks of
// v_mfma_f32_32x32x16_bf16 (fp8: v_mfma_scale_f32_32x32x64_f8f6f4).  K advances 64
// bf16 (128 fp8 bytes) per step.  A and B tiles go global -> LDS directly
// (global_load_lds_dwordx4, no register staging), double buffered (4 x 32 KiB), with
// 16-byte chunks XOR-swizzled by (row/2)%8 so that the 16 lanes of each LDS read
// pass hit distinct banks.  Operand fragments are double buffered in registers.
// The output tile is staged through LDS and written with 16-byte row stores.
//
// Ragged groups: every row tile ("slot") of every expert is enumerated from the
// device-resident offsets; the grid is sized for the worst case
// (ceil(max_rows/256) + E slots) and workgroups without a tile exit.  No host sync.
// Tile order is XCD-aware: workgroups are dispatched round-robin over the 8 XCDs,
// so consecutive ids of one XCD are given 32-tile super-blocks of 4 slots x 8
// column tiles, which then share their A and B K-slices in that XCD's L2.
//
// Weights are consumed in a packed, derived layout (kmoe_pack_weights):
//   w13: (E, 2*F_pad, d)   per 128-wide f block: 128 gate rows then 128 up rows,
//                          each row K(=d)-contiguous (w1/w2 transposed)
//   w3 : (E, d_pad, F_pad) row n K(=f)-contiguous (w3 transposed), d_pad = round_up(d, 256)
// Every packed row is followed by WPAD bytes of padding: with power-of-two row
// strides the 256 rows of a tile K-slice would all map to the same memory
// channels; the pad spreads them (measured: +20% on the gate/up GEMM).
#include "kmoe_common.h"

namespace {

constexpr int BM = 256;
constexpr int BN = 256;       // B rows per tile (gate_up: 128 gate + 128 up)
constexpr int GEMM_THREADS = 512;
constexpr int WPAD = 128;     // bytes of padding after every packed weight row
constexpr int NXCD = 8;
constexpr int SB_TILES = 32;  // tiles per XCD super-block (4 slots x 8 column tiles)
// output staging: 256 rows x up to 256 bf16 columns, rows padded by 16 bytes
constexpr int OUT_STRIDE_MAX = 256 * 2 + 16;

// K pipeline configuration: KB bytes of K per row per step (128 = 64 bf16, 64 = 32
// bf16), NST LDS stages (NST-1 steps of loads in flight).
template <int KB, int NST>
struct Pipe {
  static constexpr int TB = BM * KB;                       // bytes of one A or B stage tile
  static constexpr int CPR = KB / 16;                      // 16-byte chunks per row
  static constexpr int RPB = 1024 / KB;                    // rows per 1 KiB load block
  static constexpr int RS = (KB == 128) ? 1 : 2;           // swizzle row shift (256/KB = 2^RS)
  static constexpr int BLK_PER_WAVE = (BM / RPB) / 8;      // load blocks per wave per tile
  static constexpr int LOADS = 2 * BLK_PER_WAVE;           // A + B load instructions per wave per step
  static constexpr int LDS = (NST * 2 * TB > BM * OUT_STRIDE_MAX) ? NST * 2 * TB : BM * OUT_STRIDE_MAX;
  // Byte offset of 16-byte chunk `chunk` of row `row`: XOR by (row >> RS) spreads
  // the 16 lanes of each LDS read pass (16 consecutive rows) over distinct banks.
  __device__ static __forceinline__ int swz(int row, int chunk) {
    return row * KB + ((chunk ^ ((row >> RS) & (CPR - 1))) << 4);
  }
};

// K-pipeline configuration of the shipped kernels (bytes of K per step, stages).
#ifndef KMOE_GEMM_KB
#define KMOE_GEMM_KB 128
#endif
#ifndef KMOE_GEMM_NST
#define KMOE_GEMM_NST 2
#endif
// Static LDS of the kernel (a dependent array size would keep the host-side
// launch stub from being emitted).
constexpr int GEMM_LDS = Pipe<KMOE_GEMM_KB, KMOE_GEMM_NST>::LDS;

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// (expert, row-tile) of row-slot `slot`, from the offsets; returns false if none.
__device__ __forceinline__ bool find_row_tile(const int32_t* __restrict__ offsets, int E, int slot, int& e_out,
                                              int& m0, int& m_end) {
  int base = 0;
  int lo = offsets[0];
  for (int e = 0; e < E; ++e) {
    const int hi = offsets[e + 1];
    const int nt = (hi - lo + BM - 1) / BM;
    if (slot < base + nt) {
      e_out = e;
      m0 = lo + (slot - base) * BM;
      m_end = hi;
      return true;
    }
    base += nt;
    lo = hi;
  }
  return false;
}

// Workgroup id -> (slot, column tile), XCD-aware (see the file comment).
__device__ __forceinline__ void map_tile(int L, int n_tiles, int& slot, int& nt) {
  const int xcd = L % NXCD, i = L / NXCD;
  const int t = ((i / SB_TILES) * NXCD + xcd) * SB_TILES + (i % SB_TILES);
  const int per_group = 4 * n_tiles;
  const int g = t / per_group, r = t - g * per_group;
  nt = r >> 2;
  slot = g * 4 + (r & 3);
}

template <bool FP8>
struct Frag;
template <>
struct Frag<false> {
  bf16x8_t v;
};
template <>
struct Frag<true> {
  i32x8_t v;
};

// One MFMA operand fragment of K-substep `i` (bf16: 16 of K, chunk 2i+lh; fp8: 64
// of K, chunks 4i+2lh and 4i+2lh+1) for LDS tile row `r`.
template <class P, bool FP8>
__device__ __forceinline__ void read_frag(const uint8_t* l, int r, int i, int lh, Frag<FP8>& f) {
  if constexpr (!FP8) {
    f.v = *reinterpret_cast<const bf16x8_t*>(l + P::swz(r, 2 * i + lh));
  } else {
    const int ch = 4 * i + 2 * lh;
    const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(l + P::swz(r, ch));
    const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(l + P::swz(r, ch + 1));
    f.v = i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

template <bool FP8>
__device__ __forceinline__ void mfma(f32x16_t& acc, const Frag<FP8>& a, const Frag<FP8>& b) {
  if constexpr (!FP8)
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, acc, 0, 0, 0);
  else
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a.v, b.v, acc, 0, 0, 0, 127, 0, 127);
}

// B-tile row of the wave's j-th 32-row block (wn in 0..3, j in 0..1).
template <bool GATE_UP>
__device__ __forceinline__ int b_row(int wn, int j, int lr) {
  if (GATE_UP) return (j == 0 ? 0 : 128) + wn * 32 + lr;  // gate block, up block
  return wn * 64 + j * 32 + lr;
}

// FP8: A/B bytes are e4m3; a_scale per A row, b_scale per B row (global row index).
template <bool GATE_UP, bool FP8, int KB, int NST>
__global__ __launch_bounds__(GEMM_THREADS, 1) void grouped_gemm_kernel(
    const uint8_t* __restrict__ A, int64_t lda_bytes, const float* __restrict__ a_scale,
    const int32_t* __restrict__ offsets, int E, const uint8_t* __restrict__ B, int64_t b_expert_rows,
    int64_t ldb_bytes, const float* __restrict__ b_scale, int k_bytes, uint16_t* __restrict__ C, int64_t ldc,
    int n_valid, int n_tiles) {
  using P = Pipe<KB, NST>;
  static_assert(P::LDS <= GEMM_LDS, "LDS budget of this pipeline configuration");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[GEMM_LDS];
  constexpr int NSUB = FP8 ? KB / 64 : KB / 32;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wm = wave >> 2, wn = wave & 3;

  int slot, nt;
  map_tile(blockIdx.x, n_tiles, slot, nt);
  int e, m0, m_end;
  if (!find_row_tile(offsets, E, slot, e, m0, m_end)) return;

  const int64_t brow0 = (int64_t)e * b_expert_rows + (int64_t)nt * BN;
  const uint8_t* bexp = B + brow0 * ldb_bytes;
  const int nk = k_bytes / KB;
  // LDS stage s: [A tile | B tile]
  auto la_buf = [&](int st) { return lds + st * 2 * P::TB; };
  auto lb_buf = [&](int st) { return lds + st * 2 * P::TB + P::TB; };

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Direct-to-LDS tile loads: a 256-row tile is 256*KB/1024 blocks of 1 KiB; wave w
  // issues A and B blocks [w*BPW, (w+1)*BPW).  Block q fills tile rows [q*RPB,
  // (q+1)*RPB): lane l lands at byte 16*l of the block (row q*RPB + l/CPR, physical
  // chunk l%CPR) and so fetches the logical chunk that swz() maps there.  A rows
  // past the expert's last row are clamped to it (their results are never stored).
  constexpr int BPW = P::BLK_PER_WAVE;
  const int rsub = lane / P::CPR, pc = lane % P::CPR;
  static_assert(BPW <= 4, "load blocks per wave");
  uint32_t a_off[4], b_off[4];  // fixed size: a dependent array size drops the host launch stub
#pragma unroll
  for (int q = 0; q < BPW; ++q) {
    const int tr = (wave * BPW + q) * P::RPB + rsub;
    int ra = m0 + tr;
    ra = ra < m_end ? ra : m_end - 1;
    const uint32_t chunk = (uint32_t)(pc ^ ((tr >> P::RS) & (P::CPR - 1))) << 4;
    a_off[q] = (uint32_t)ra * (uint32_t)lda_bytes + chunk;
    b_off[q] = (uint32_t)tr * (uint32_t)ldb_bytes + chunk;
  }
  auto issue = [&](int kt) {
    uint8_t* adst = la_buf(kt % NST);
    uint8_t* bdst = lb_buf(kt % NST);
    const uint8_t* ag = A + (int64_t)kt * KB;
    const uint8_t* bg = bexp + (int64_t)kt * KB;
#pragma unroll
    for (int q = 0; q < BPW; ++q)
      __builtin_amdgcn_global_load_lds(ag + a_off[q], (KMOE_LDS void*)(adst + (wave * BPW + q) * 1024), 16, 0, 0);
#pragma unroll
    for (int q = 0; q < BPW; ++q)
      __builtin_amdgcn_global_load_lds(bg + b_off[q], (KMOE_LDS void*)(bdst + (wave * BPW + q) * 1024), 16, 0, 0);
  };
  // bf16: fragments double buffered across substeps; fp8 (8-register fragments):
  // single buffered to stay within 256 registers at 2 waves per SIMD.
  constexpr int NBUF = (FP8 || NSUB == 1) ? 1 : 2;
  Frag<FP8> fa[NBUF][4], fb[NBUF][2];
  auto rd = [&](const uint8_t* la, const uint8_t* lb, int i, Frag<FP8> (&a)[4], Frag<FP8> (&b)[2]) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) read_frag<P, FP8>(la, wm * 128 + mi * 32 + lr, i, lh, a[mi]);
#pragma unroll
    for (int j = 0; j < 2; ++j) read_frag<P, FP8>(lb, b_row<GATE_UP>(wn, j, lr), i, lh, b[j]);
  };

  // NST-stage pipeline: stage kt is waited for (own loads by vmcnt, everyone's by the
  // barrier), then the loads of step kt+NST-1 go into the buffer freed by step kt-1.
  for (int st = 0; st < NST - 1 && st < nk; ++st) issue(st);
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + NST - 2 < nk)
      wait_vmcnt<(NST - 2) * P::LOADS>();
    else
      wait_vmcnt<0>();
    barrier_nofence();
    if (kt + NST - 1 < nk) issue(kt + NST - 1);
    const uint8_t* la = la_buf(kt % NST);
    const uint8_t* lb = lb_buf(kt % NST);
    rd(la, lb, 0, fa[0], fb[0]);
#pragma unroll
    for (int i = 0; i < NSUB; ++i) {
      const int cb = i % NBUF;
      if (NBUF == 2 && i + 1 < NSUB) rd(la, lb, i + 1, fa[(i + 1) % NBUF], fb[(i + 1) % NBUF]);
      if (NBUF == 1 && i > 0) rd(la, lb, i, fa[0], fb[0]);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int j = 0; j < 2; ++j) mfma<FP8>(acc[mi][j], fa[cb][mi], fb[cb][j]);
    }
  }

  // ---- epilogue.  acc[mi][j][r] is (row 8*(r/4)+4*lh+r%4, col lr) of block (mi, j).
  // Results go to an LDS tile (rows padded by 16 bytes; even lanes store the bf16
  // pair of lanes lr, lr+1), then out with 16-byte stores along rows.
  constexpr int NC = GATE_UP ? 128 : 256;   // output columns of the tile
  constexpr int OSTR = NC * 2 + 16;          // LDS row stride (bytes)
  __syncthreads();
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int trow = wm * 128 + mi * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
      const int grow = m0 + trow;
      const float sa = (FP8 && grow < m_end) ? a_scale[grow] : 1.0f;
#pragma unroll
      for (int jo = 0; jo < (GATE_UP ? 1 : 2); ++jo) {
        float v;
        int col;
        if (GATE_UP) {
          float g = acc[mi][0][r], u = acc[mi][1][r];
          if (FP8) {
            g *= sa * b_scale[brow0 + b_row<true>(wn, 0, lr)];
            u *= sa * b_scale[brow0 + b_row<true>(wn, 1, lr)];
          }
          v = silu_f32(g) * u;
          col = wn * 32 + lr;
        } else {
          v = acc[mi][jo][r];
          if (FP8) v *= sa * b_scale[brow0 + b_row<false>(wn, jo, lr)];
          col = wn * 64 + jo * 32 + lr;
        }
        const uint32_t bits = f32_to_bf16(v);
        const uint32_t nb = (uint32_t)__shfl_xor((int)bits, 1, 64);
        if ((lr & 1) == 0) *reinterpret_cast<uint32_t*>(lds + trow * OSTR + col * 2) = bits | (nb << 16);
      }
    }
  }
  __syncthreads();
  constexpr int CPR = NC * 2 / 16;  // 16-byte chunks per row
  const int col0 = nt * NC;
  for (int c = tid; c < BM * CPR; c += GEMM_THREADS) {
    const int trow = c / CPR, ch = c % CPR;
    const int grow = m0 + trow;
    const int gcol = col0 + ch * 8;
    if (grow < m_end && gcol < n_valid)
      *reinterpret_cast<i32x4_t*>(C + (int64_t)grow * ldc + gcol) =
          *reinterpret_cast<const i32x4_t*>(lds + trow * OSTR + ch * 16);
  }
}

// ---------------------------------------------------------------- weight packing
// out[e][map(c)][r] = in[e][r][c] for in (E, R, Cn) row-major; rows of `out` have
// length out_ld (>= R, zero padded), out has out_rows rows per expert (zero padded).
// gate_up maps input column f of w1 (half 0) / w2 (half 1) to packed row
// (f/128)*256 + half*128 + f%128; down maps column n of w3 to row n.
template <bool IN_F32, bool FP8>
__global__ __launch_bounds__(256) void pack_transpose_kernel(const void* __restrict__ in, int R, int Cn,
                                                             int64_t in_expert_stride, int half, bool gate_up,
                                                             uint8_t* __restrict__ out, int64_t out_rows, int out_ld,
                                                             const float* __restrict__ row_scale) {
  __shared__ float tile[64][65];
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64;  // input rows (become output columns)
  const int c0 = blockIdx.x * 64;  // input cols (become output rows)
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    float v = 0.0f;
    if (r < R && c < Cn) {
      const int64_t off = (int64_t)e * in_expert_stride + (int64_t)r * Cn + c;
      v = IN_F32 ? static_cast<const float*>(in)[off] : bf16_to_f32(static_cast<const uint16_t*>(in)[off]);
    }
    tile[i][tx] = v;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i;  // output row source column
    const int r = r0 + tx;  // output column
    if (c >= Cn || r >= out_ld) continue;
    const int64_t orow = gate_up ? (int64_t)(c / 128) * 256 + half * 128 + (c % 128) : (int64_t)c;
    const int64_t o = ((int64_t)e * out_rows + orow) * out_ld + r;
    const float v = tile[tx][i];
    if (FP8) {
      // row_scale holds the row amax at this point (finalised to amax/448 afterwards)
      const float amax = row_scale[(int64_t)e * out_rows + orow];
      const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
      out[o] = (uint8_t)f32_to_e4m3(v * inv);
    } else {
      reinterpret_cast<uint16_t*>(out)[o] = f32_to_bf16(v);
    }
  }
}

// Column amax of in[e] (R x Cn) -> per packed row amax (turned into amax/448 by
// finalize_scale_kernel once the rows have been quantised).
template <bool IN_F32>
__global__ __launch_bounds__(256) void col_scale_kernel(const void* __restrict__ in, int R, int Cn,
                                                        int64_t in_expert_stride, int half, bool gate_up,
                                                        float* __restrict__ scale, int64_t out_rows) {
  const int e = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= Cn) return;
  float amax = 0.0f;
  for (int r = 0; r < R; ++r) {
    const int64_t off = (int64_t)e * in_expert_stride + (int64_t)r * Cn + c;
    const float v = IN_F32 ? static_cast<const float*>(in)[off] : bf16_to_f32(static_cast<const uint16_t*>(in)[off]);
    amax = fmaxf(amax, fabsf(v));
  }
  const int64_t orow = gate_up ? (int64_t)(c / 128) * 256 + half * 128 + (c % 128) : (int64_t)c;
  scale[(int64_t)e * out_rows + orow] = amax;
}

__global__ void finalize_scale_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = p[i] / 448.0f;
}

__global__ void zero_kernel(uint8_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}
__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

// Per-row fp8 quantisation of a bf16 matrix, one wave per row.
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ in, int64_t rows,
                                                         const int32_t* __restrict__ n_rows_dev, int cols,
                                                         uint8_t* __restrict__ out, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int64_t nr = rows;
  if (n_rows_dev) nr = min<int64_t>(nr, (int64_t)*n_rows_dev);
  if (r >= nr) return;
  const int nvec = cols / 8;
  const i32x4_t* src = reinterpret_cast<const i32x4_t*>(in + r * cols);
  float amax = 0.0f;
  for (int v = lane; v < nvec; v += 64) {
    const i32x4_t val = src[v];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      amax = fmaxf(amax, fabsf(__uint_as_float(((uint32_t)val[q]) << 16)));
      amax = fmaxf(amax, fabsf(__uint_as_float(((uint32_t)val[q]) & 0xffff0000u)));
    }
  }
  amax = wave_max(amax);
  const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + r * cols);
  for (int v = lane; v < nvec; v += 64) {
    const i32x4_t val = src[v];
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t w0 = (uint32_t)val[q];
      lo |= f32_to_e4m3(__uint_as_float(w0 << 16) * inv) << (16 * q);
      lo |= f32_to_e4m3(__uint_as_float(w0 & 0xffff0000u) * inv) << (16 * q + 8);
      const uint32_t w1 = (uint32_t)val[q + 2];
      hi |= f32_to_e4m3(__uint_as_float(w1 << 16) * inv) << (16 * q);
      hi |= f32_to_e4m3(__uint_as_float(w1 & 0xffff0000u) * inv) << (16 * q + 8);
    }
    dst[2 * v] = lo;
    dst[2 * v + 1] = hi;
  }
  if (lane == 0) scale[r] = amax / 448.0f;
}

int elem_bytes(int dtype) { return dtype == KMOE_DTYPE_FP8_E4M3 ? 1 : 2; }

int launch_gemm(bool gate_up, bool fp8, const void* A, const float* a_scale, const int32_t* offsets, int E, int K,
                int64_t max_rows, const void* B, int64_t b_expert_rows, const float* b_scale, void* C, int64_t ldc,
                int n_valid, int n_tiles, hipStream_t s) {
  const int eb = fp8 ? 1 : 2;
  const int64_t slots = kmoe::ceil_div<int64_t>(max_rows, BM) + E;
  // whole 4-slot groups, whole XCD super-blocks (map_tile covers [0, blocks))
  const int64_t blocks = kmoe::ceil_div<int64_t>(kmoe::ceil_div<int64_t>(slots, 4) * 4 * n_tiles,
                                                 (int64_t)NXCD * SB_TILES) * NXCD * SB_TILES;
  if (blocks > 0x7fffffff) {
    kmoe::set_error("kmoe gemm: grid too large");
    return KMOE_ERR_SHAPE;
  }
  const int kbytes = K * eb;
  if (kbytes % KMOE_GEMM_KB != 0) {
    kmoe::set_error("kmoe gemm: K bytes %d not a multiple of %d", kbytes, KMOE_GEMM_KB);
    return KMOE_ERR_SHAPE;
  }
  const uint8_t* a = static_cast<const uint8_t*>(A);
  const uint8_t* b = static_cast<const uint8_t*>(B);
  uint16_t* c = static_cast<uint16_t*>(C);
  const int64_t lda = kbytes, ldb = kbytes + WPAD;
  const dim3 grid((unsigned)blocks);
  constexpr int KB = KMOE_GEMM_KB, NST = KMOE_GEMM_NST;
  const dim3 block(GEMM_THREADS);
  if (gate_up && !fp8)
    hipLaunchKernelGGL((grouped_gemm_kernel<true, false, KB, NST>), grid, block, 0, s, a, lda, a_scale, offsets, E, b,
                       b_expert_rows, ldb, b_scale, kbytes, c, ldc, n_valid, n_tiles);
  else if (gate_up && fp8)
    hipLaunchKernelGGL((grouped_gemm_kernel<true, true, KB, NST>), grid, block, 0, s, a, lda, a_scale, offsets, E, b,
                       b_expert_rows, ldb, b_scale, kbytes, c, ldc, n_valid, n_tiles);
  else if (!fp8)
    hipLaunchKernelGGL((grouped_gemm_kernel<false, false, KB, NST>), grid, block, 0, s, a, lda, a_scale, offsets, E, b,
                       b_expert_rows, ldb, b_scale, kbytes, c, ldc, n_valid, n_tiles);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<false, true, KB, NST>), grid, block, 0, s, a, lda, a_scale, offsets, E, b,
                       b_expert_rows, ldb, b_scale, kbytes, c, ldc, n_valid, n_tiles);
  return KMOE_OK;
}

}  // namespace

extern "C" int kmoe_padded_ff(int F) { return round_up(F, 128); }

extern "C" size_t kmoe_packed_w13_bytes(int E, int d, int F, int dtype) {
  return (size_t)E * 2 * (size_t)round_up(F, 128) * ((size_t)d * (size_t)elem_bytes(dtype) + WPAD);
}

extern "C" size_t kmoe_packed_w3_bytes(int E, int d, int F, int dtype) {
  return (size_t)E * (size_t)round_up(d, 256) * ((size_t)round_up(F, 128) * (size_t)elem_bytes(dtype) + WPAD);
}

extern "C" int kmoe_pack_weights(const void* w1, const void* w2, const void* w3, int w_dtype, int E, int d, int F,
                                 int packed_dtype, void* w13_packed, float* w13_scale, void* w3_packed,
                                 float* w3_scale, void* stream) {
  KMOE_REQUIRE(w1 && w2 && w3 && w13_packed && w3_packed, KMOE_ERR_NULL, "kmoe_pack_weights: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_pack_weights: E=%d out of range", E);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "kmoe_pack_weights: d=%d must be a positive multiple of 64", d);
  KMOE_REQUIRE(F > 0, KMOE_ERR_SHAPE, "kmoe_pack_weights: F=%d must be > 0", F);
  KMOE_REQUIRE(w_dtype == KMOE_DTYPE_BF16 || w_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "kmoe_pack_weights: weight dtype must be bf16 or f32");
  KMOE_REQUIRE(packed_dtype == KMOE_DTYPE_BF16 || packed_dtype == KMOE_DTYPE_FP8_E4M3, KMOE_ERR_DTYPE,
               "kmoe_pack_weights: packed dtype must be bf16 or fp8_e4m3");
  const bool fp8 = packed_dtype == KMOE_DTYPE_FP8_E4M3;
  KMOE_REQUIRE(!fp8 || (w13_scale && w3_scale), KMOE_ERR_NULL, "kmoe_pack_weights: fp8 needs scale buffers");
  hipStream_t s = kmoe::as_stream(stream);
  const int Fp = round_up(F, 128), dp = round_up(d, 256);
  const int64_t rows13 = 2 * (int64_t)Fp, rows3 = dp;
  // zero the padding (whole buffers: simple and only done when weights change)
  hipLaunchKernelGGL(zero_kernel, dim3(1024), dim3(256), 0, s, static_cast<uint8_t*>(w13_packed),
                     (int64_t)kmoe_packed_w13_bytes(E, d, F, packed_dtype));
  hipLaunchKernelGGL(zero_kernel, dim3(1024), dim3(256), 0, s, static_cast<uint8_t*>(w3_packed),
                     (int64_t)kmoe_packed_w3_bytes(E, d, F, packed_dtype));
  const bool f32 = w_dtype == KMOE_DTYPE_F32;
  if (fp8) {
    hipLaunchKernelGGL(zero_f32_kernel, dim3(64), dim3(256), 0, s, w13_scale, (int64_t)E * rows13);
    hipLaunchKernelGGL(zero_f32_kernel, dim3(64), dim3(256), 0, s, w3_scale, (int64_t)E * rows3);
    const dim3 g13((unsigned)kmoe::ceil_div(F, 256), (unsigned)E), g3((unsigned)kmoe::ceil_div(d, 256), (unsigned)E);
    if (f32) {
      hipLaunchKernelGGL(col_scale_kernel<true>, g13, dim3(256), 0, s, w1, d, F, (int64_t)d * F, 0, true, w13_scale, rows13);
      hipLaunchKernelGGL(col_scale_kernel<true>, g13, dim3(256), 0, s, w2, d, F, (int64_t)d * F, 1, true, w13_scale, rows13);
      hipLaunchKernelGGL(col_scale_kernel<true>, g3, dim3(256), 0, s, w3, F, d, (int64_t)d * F, 0, false, w3_scale, rows3);
    } else {
      hipLaunchKernelGGL(col_scale_kernel<false>, g13, dim3(256), 0, s, w1, d, F, (int64_t)d * F, 0, true, w13_scale, rows13);
      hipLaunchKernelGGL(col_scale_kernel<false>, g13, dim3(256), 0, s, w2, d, F, (int64_t)d * F, 1, true, w13_scale, rows13);
      hipLaunchKernelGGL(col_scale_kernel<false>, g3, dim3(256), 0, s, w3, F, d, (int64_t)d * F, 0, false, w3_scale, rows3);
    }
  }
  // w1/w2: (E, d, F) -> rows f, cols d.  w3: (E, F, d) -> rows n, cols f.
  const int eb = elem_bytes(packed_dtype);
  const int ld13 = d + WPAD / eb, ld3 = Fp + WPAD / eb;  // packed row strides in elements
  const dim3 gt13((unsigned)kmoe::ceil_div(F, 64), (unsigned)kmoe::ceil_div(d, 64), (unsigned)E);
  const dim3 gt3((unsigned)kmoe::ceil_div(d, 64), (unsigned)kmoe::ceil_div(F, 64), (unsigned)E);
  uint8_t* o13 = static_cast<uint8_t*>(w13_packed);
  uint8_t* o3 = static_cast<uint8_t*>(w3_packed);
#define KMOE_PACK(F32_, FP8_)                                                                                        \
  do {                                                                                                               \
    hipLaunchKernelGGL((pack_transpose_kernel<F32_, FP8_>), gt13, dim3(256), 0, s, w1, d, F, (int64_t)d * F, 0, true, \
                       o13, rows13, ld13, w13_scale);                                                                   \
    hipLaunchKernelGGL((pack_transpose_kernel<F32_, FP8_>), gt13, dim3(256), 0, s, w2, d, F, (int64_t)d * F, 1, true, \
                       o13, rows13, ld13, w13_scale);                                                                   \
    hipLaunchKernelGGL((pack_transpose_kernel<F32_, FP8_>), gt3, dim3(256), 0, s, w3, F, d, (int64_t)d * F, 0, false, \
                       o3, rows3, ld3, w3_scale);                                                                     \
  } while (0)
  if (f32 && fp8)
    KMOE_PACK(true, true);
  else if (f32)
    KMOE_PACK(true, false);
  else if (fp8)
    KMOE_PACK(false, true);
  else
    KMOE_PACK(false, false);
#undef KMOE_PACK
  if (fp8) {
    hipLaunchKernelGGL(finalize_scale_kernel, dim3(64), dim3(256), 0, s, w13_scale, (int64_t)E * rows13);
    hipLaunchKernelGGL(finalize_scale_kernel, dim3(64), dim3(256), 0, s, w3_scale, (int64_t)E * rows3);
  }
  return kmoe::check_launch("kmoe_pack_weights");
}

static int check_gemm_args(const char* who, const void* a, const int32_t* offsets, int E, int d, int F,
                           int64_t max_rows, const void* w, const void* out, int in_dtype) {
  KMOE_REQUIRE(a && offsets && w && out, KMOE_ERR_NULL, "%s: null buffer", who);
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "%s: E=%d out of range", who, E);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "%s: d=%d must be a positive multiple of 64", who, d);
  KMOE_REQUIRE(F > 0, KMOE_ERR_SHAPE, "%s: F=%d must be > 0", who, F);
  KMOE_REQUIRE(max_rows >= 0 && max_rows < ((int64_t)1 << 31), KMOE_ERR_SHAPE, "%s: max_rows out of range", who);
  KMOE_REQUIRE(in_dtype == KMOE_DTYPE_BF16 || in_dtype == KMOE_DTYPE_FP8_E4M3, KMOE_ERR_DTYPE,
               "%s: input dtype must be bf16 or fp8_e4m3", who);
  return KMOE_OK;
}

extern "C" int kmoe_gemm_gate_up(const void* xperm, const float* xperm_scale, int in_dtype, const int32_t* offsets,
                                 int E, int d, int F, int64_t max_rows, const void* w13_packed, const float* w13_scale,
                                 void* h, void* stream) {
  int rc = check_gemm_args("kmoe_gemm_gate_up", xperm, offsets, E, d, F, max_rows, w13_packed, h, in_dtype);
  if (rc) return rc;
  const bool fp8 = in_dtype == KMOE_DTYPE_FP8_E4M3;
  KMOE_REQUIRE(!fp8 || (xperm_scale && w13_scale), KMOE_ERR_NULL, "kmoe_gemm_gate_up: fp8 needs scales");
  KMOE_REQUIRE(!fp8 || d % 128 == 0, KMOE_ERR_SHAPE, "kmoe_gemm_gate_up: fp8 needs d %% 128 == 0 (d=%d)", d);
  if (max_rows == 0) return KMOE_OK;
  const int Fp = round_up(F, 128);
  rc = launch_gemm(true, fp8, xperm, xperm_scale, offsets, E, d, max_rows, w13_packed, 2 * (int64_t)Fp, w13_scale, h,
                   Fp, Fp, Fp / 128, kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_gate_up");
}

extern "C" int kmoe_gemm_down(const void* h, const float* h_scale, int in_dtype, const int32_t* offsets, int E, int d,
                              int F, int64_t max_rows, const void* w3_packed, const float* w3_scale, void* y,
                              void* stream) {
  int rc = check_gemm_args("kmoe_gemm_down", h, offsets, E, d, F, max_rows, w3_packed, y, in_dtype);
  if (rc) return rc;
  const bool fp8 = in_dtype == KMOE_DTYPE_FP8_E4M3;
  KMOE_REQUIRE(!fp8 || (h_scale && w3_scale), KMOE_ERR_NULL, "kmoe_gemm_down: fp8 needs scales");
  if (max_rows == 0) return KMOE_OK;
  const int Fp = round_up(F, 128), dp = round_up(d, 256);
  rc = launch_gemm(false, fp8, h, h_scale, offsets, E, Fp, max_rows, w3_packed, dp, w3_scale, y, d, d, dp / BN,
                   kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_down");
}

extern "C" int kmoe_quant_rows_fp8(const void* in, int64_t rows, const int32_t* n_rows_dev, int cols, uint8_t* out,
                                   float* scale, void* stream) {
  KMOE_REQUIRE(in && out && scale, KMOE_ERR_NULL, "kmoe_quant_rows_fp8: null buffer");
  KMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, KMOE_ERR_SHAPE, "kmoe_quant_rows_fp8: bad shape");
  if (rows == 0) return KMOE_OK;
  hipLaunchKernelGGL(quant_rows_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(rows, 4)), dim3(256), 0,
                     kmoe::as_stream(stream), static_cast<const uint16_t*>(in), rows, n_rows_dev, cols, out, scale);
  return kmoe::check_launch("kmoe_quant_rows_fp8");
}

extern "C" int kmoe_grouped_swiglu(const void* xperm, const int32_t* offsets, int E, int d, int F, int64_t max_rows,
                                   const void* w13_packed, const void* w3_packed, void* h, void* y, void* stream) {
  int rc = kmoe_gemm_gate_up(xperm, nullptr, KMOE_DTYPE_BF16, offsets, E, d, F, max_rows, w13_packed, nullptr, h,
                             stream);
  if (rc) return rc;
  return kmoe_gemm_down(h, nullptr, KMOE_DTYPE_BF16, offsets, E, d, F, max_rows, w3_packed, nullptr, y, stream);
}
