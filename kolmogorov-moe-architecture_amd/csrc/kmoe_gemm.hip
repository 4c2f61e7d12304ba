// Grouped SwiGLU expert GEMMs on CDNA4 MFMA.
// Replaces moe_kernels.grouped_swiglu_forward (moe_arch/kernels/grouped_gemm.cu:186-257)
// and the padded bmm block of GroupedExperts.forward (moe_arch/model/moe.py:275-279):
//   gate_up:  h[r, f] = silu(x[r] . w1[e][:, f]) * (x[r] . w2[e][:, f])     (ffn.py:17-64)
//   down:     y[r, n] = h[r] . w3[e][:, n]
// for the rows r of expert e, [offsets[e], offsets[e+1]).
//
// Tiling: a workgroup of 4 waves (one per SIMD) owns a 256-row x 256-B-row tile;
// waves form 2 (rows) x 2 (B rows) and each computes 128 x 128, 256 fp32 accumulators
// per lane: bf16 as 8x8 blocks of v_mfma_f32_16x16x32_bf16, fp8 as 4x4 blocks of
// v_mfma_scale_f32_32x32x64_f8f6f4.  (The expert GEMMs run at the chip's power limit,
// and on random data the 16x16x32 bf16 form sustains a higher clock than 32x32x16:
// 0.81 against 0.70 of the bf16 peak in an MFMA-only loop; the fp8 16x16x128 form runs
// at half rate, so fp8 keeps 32x32x64.)  A 128x128 wave tile reads 0.5 KiB of LDS per
// 32 K-MACs of output, the least a 4-wave workgroup of this tile allows.  K advances 64
// bf16 (128 fp8 bytes) per pipeline step through 2 LDS stages of 2 x 32 KiB.  Tile
// data is loaded into registers with buffer loads (the K offset is a scalar operand)
// one step ahead and written to the stage not being read, 16-byte chunks XOR-swizzled
// so that both the 1 KiB block writes and every 16-lane fragment read pass are
// bank-conflict free.  bf16: the K loop is emitted in program order (each MFMA with
// the LDS or memory instruction assigned to it); fp8: interleaved by scheduling
// groups, fragments double buffered.  One barrier per step.
// The MFMAs take the B fragment as their first operand, so each lane accumulates
// runs of four consecutive output columns of one row; the epilogue packs them to
// 8-byte bf16 runs in registers, stages the tile through LDS and writes it with
// 16-byte row stores.
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
#include <type_traits>

#include "kmoe_common.h"

namespace {

constexpr int BM = 256;
constexpr int BN = 256;       // B rows per tile (gate_up: 128 gate + 128 up)
constexpr int GEMM_THREADS = 256;
constexpr int WPAD = 128;     // bytes of padding after every packed weight row
constexpr int NXCD = 8;
constexpr int SB_TILES = 32;  // tiles per XCD super-block (4 slots x 8 column tiles)
constexpr int KB = 128;       // K bytes per row per pipeline step (64 bf16 / 128 fp8)
constexpr int TB = BM * KB;   // bytes of one A or B stage tile (32 KiB)
constexpr int NST = 2;        // LDS stages: one read while the next is written
constexpr int CPR = KB / 16;  // 16-byte chunks per tile row
constexpr int RPB = 1024 / KB;                        // tile rows per 1 KiB load block
constexpr int BLK_PER_WAVE = (BM * KB / 1024) / 4;    // load blocks per wave per operand per step
// output staging: 256 rows x up to 256 bf16 columns, rows padded by 16 bytes
constexpr int OUT_STRIDE_MAX = 256 * 2 + 16;
constexpr int SCALE_LDS = (NST * 2 * TB > BM * OUT_STRIDE_MAX) ? NST * 2 * TB : BM * OUT_STRIDE_MAX;
// fp8: the tile's A-row and B-row scales (256 floats each) after the stages / output staging
constexpr int GEMM_LDS = SCALE_LDS + 2 * BM * 4;
static_assert(GEMM_LDS <= 160 * 1024, "LDS budget");

// Byte offset of 16-byte chunk `chunk` of tile row `row`.  A 128-byte row puts rows
// r and r+2 on the same banks; XOR-ing the chunk by (row/2)%8 gives the 16 lanes of
// an LDS read pass (16 consecutive rows, one chunk) 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int row, int chunk) { return row * KB + ((chunk ^ ((row >> 1) & (CPR - 1))) << 4); }

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// Row slots.  Lane e of a wave holds the row range [lo, hi) of expert e (E <= 64)
// and its number of 256-row slots; slots are numbered expert by expert.
struct SlotTable {
  int lo, hi, ns;  // this lane's expert
  int n_slots;     // all experts (wave-uniform)
};
__device__ __forceinline__ SlotTable load_slots(const int32_t* __restrict__ offsets, int E) {
  const int lane = threadIdx.x & 63;
  SlotTable t;
  t.lo = 0;
  t.hi = 0;
  if (lane < E) {
    t.lo = offsets[lane];
    t.hi = offsets[lane + 1];
  }
  t.ns = (t.hi - t.lo + BM - 1) / BM;
  int n = t.ns;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) n += __shfl_xor(n, o, 64);
  t.n_slots = __builtin_amdgcn_readfirstlane(n);
  return t;
}
// (expert, first row, row end) of slot `slot` < n_slots: a readlane walk over the
// experts' slot counts.
__device__ __forceinline__ void find_slot(const SlotTable& t, int E, int slot, int& e_out, int& m0, int& m_end) {
  int base = 0;
  e_out = 0;
  m0 = 0;
  m_end = 0;
  for (int e = 0; e < E; ++e) {
    const int n = __builtin_amdgcn_readlane(t.ns, e);
    if (slot < base + n) {
      e_out = e;
      m0 = __builtin_amdgcn_readlane(t.lo, e) + (slot - base) * BM;
      m_end = __builtin_amdgcn_readlane(t.hi, e);
      return;
    }
    base += n;
  }
}

// Dense tile order: slots in groups of 4, each group enumerated column tile by
// column tile (4 consecutive tiles share a column tile, so 32 consecutive tiles are
// 8 column tiles x 4 slots); the last, partial group likewise with its slots.
__device__ __forceinline__ void dense_tile(int t, int n_slots, int n_tiles, int& slot, int& nt) {
  const int full = (n_slots >> 2) * 4 * n_tiles;
  if (t < full) {
    const int g = t / (4 * n_tiles), r = t - g * 4 * n_tiles;
    nt = r >> 2;
    slot = g * 4 + (r & 3);
  } else {
    const int rem = n_slots & 3, u = t - full;
    nt = u / rem;
    slot = (n_slots & ~3) + (u - nt * rem);
  }
}

// Workgroup id L < n (n a multiple of 256) -> dense tile, XCD-aware: workgroups are
// dispatched round-robin over the 8 XCDs, so the consecutive ids one XCD receives
// are given 32-tile super-blocks, which share A and B K-slices in that XCD's L2.
__device__ __forceinline__ int xcd_tile(int L) {
  const int xcd = L % NXCD, i = L / NXCD;
  return ((i / SB_TILES) * NXCD + xcd) * SB_TILES + (i % SB_TILES);
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
template <bool FP8>
__device__ __forceinline__ void read_frag(const uint8_t* l, int r, int i, int lh, Frag<FP8>& f) {
  if constexpr (!FP8) {
    f.v = *reinterpret_cast<const bf16x8_t*>(l + swz(r, 2 * i + lh));
  } else {
    const int ch = 4 * i + 2 * lh;
    const i32x4_t lo = *reinterpret_cast<const i32x4_t*>(l + swz(r, ch));
    const i32x4_t hi = *reinterpret_cast<const i32x4_t*>(l + swz(r, ch + 1));
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

// bf16 tiles run on v_mfma_f32_16x16x32_bf16: on random data the 32x32x16 form holds the
// chip at 0.70 of the bf16 peak under its power limit (an MFMA-only loop, all CUs), the
// 16x16x32 form at 0.81 (it moves half the accumulator bytes per FLOP).  Fragment of
// K-substep `i` (32 of K: chunks 4i .. 4i+3) for LDS tile rows r0 .. r0+15: lane l reads
// row r0 + l%16 (`r`), chunk 4i + l/16 (`lq`); a 16-lane pass is 16 consecutive rows of
// one logical chunk, which the swizzle spreads over all banks.
__device__ __forceinline__ void read_frag16(const uint8_t* l, int r, int i, int lq, Frag<false>& f) {
  f.v = *reinterpret_cast<const bf16x8_t*>(l + swz(r, 4 * i + lq));
}
__device__ __forceinline__ void mfma16(f32x4_t& acc, const Frag<false>& a, const Frag<false>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}

// B-tile geometry of a tile whose waves hold WNB 32-row B blocks each (WNB = 4: the
// full 256 B rows; 2 and 1: the narrow tiles of the split tail, a half or a
// quarter `q` of a full tile's output columns).  LDS B row of block j of wave
// column wn:  down: 32 WNB wn + 32 j + lr;  gate_up (WNB >= 2): the first WNB/2
// blocks are gate rows and the rest the up rows of the same f columns;  gate_up
// WNB = 1: the wave's one block is 16 gate rows then the 16 up rows of the same f
// columns (LDS rows 32 wn + lr).
template <bool GATE_UP, int WNB>
__device__ __forceinline__ int b_lds_row(int wn, int j, int lr) {
  if constexpr (GATE_UP && WNB == 1) {
    return wn * 32 + lr;
  } else if constexpr (GATE_UP) {
    constexpr int H = WNB / 2;
    return (j / H) * (32 * WNB) + wn * (16 * WNB) + (j % H) * 32 + lr;
  } else {
    return wn * (32 * WNB) + j * 32 + lr;
  }
}
// Row of the 256-row packed B tile that LDS B row `lrow` holds (identity for WNB = 4).
// gate_up packs 128 gate rows then 128 up rows per full tile.
template <bool GATE_UP, int WNB>
__device__ __forceinline__ int b_packed_row(int lrow, int q) {
  if constexpr (GATE_UP && WNB == 1) {
    const int i = lrow & 31;  // f column 32 q + 16 (lrow / 32) + i % 16; up rows from i = 16
    return (i >> 4) * 128 + q * 32 + (lrow >> 5) * 16 + (i & 15);
  } else if constexpr (GATE_UP) {
    constexpr int HR = 32 * WNB;  // gate (or up) rows of the tile
    return (lrow / HR) * 128 + q * HR + lrow % HR;
  } else {
    return q * (64 * WNB) + lrow;
  }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [I0, N).
template <int I0, int N, class Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  if constexpr (I0 < N) {
    f(std::integral_constant<int, I0>{});
    static_for<I0 + 1, N>(f);
  }
}

// Scheduling groups for an NM-MFMA substep: the NRD fragment reads two after each
// of the first MFMAs (they feed the next substep), then the NWR LDS block writes and
// NVM memory loads spread evenly over the MFMAs from W0 = min(4, NM/2) on, so the
// writes do not queue in the LDS FIFO in front of the reads.  In-order issue means a
// DS instruction stalled on a full FIFO also holds back the MFMAs behind it: with
// reads and writes all front-loaded the K-loop took 8.6% (gate/up) and 5% (down)
// more cycles per step.
template <int NM, int NRD, int NWR, int NVM, int G = 0>
__device__ __forceinline__ void sched_spread() {
  if constexpr (G < NM) {
    constexpr int W0 = NM / 2 < 4 ? NM / 2 : 4;
    constexpr int span = NM - W0, gw = G - W0;
    constexpr int r = 2 * G < NRD ? (NRD - 2 * G < 2 ? NRD - 2 * G : 2) : 0;
    constexpr int w = G < W0 ? 0 : (NWR * (gw + 1)) / span - (NWR * gw) / span;
    constexpr int v = G < W0 ? 0 : (NVM * (gw + 1)) / span - (NVM * gw) / span;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // MFMA
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);  // DS read
    if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);  // DS write
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);  // VMEM read
    sched_spread<NM, NRD, NWR, NVM, G + 1>();
  }
}

// Scheduling groups for NM MFMAs with NWR LDS block writes and NVM memory loads spread
// evenly over them (no fragment reads among them).
template <int NM, int NWR, int NVM, int G = 0>
__device__ __forceinline__ void sched_even() {
  if constexpr (G < NM) {
    constexpr int w = (NWR * (G + 1)) / NM - (NWR * G) / NM;
    constexpr int v = (NVM * (G + 1)) / NM - (NVM * G) / NM;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // MFMA
    if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);  // DS write
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);  // VMEM read
    sched_even<NM, NWR, NVM, G + 1>();
  }
}

// Raw buffer resource over [base, base + 4 GiB): loads address it with a 32-bit
// per-lane offset plus a wave-uniform (SGPR) offset, so advancing K costs no VALU.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

struct GemmArgs {
  const uint8_t* A;
  int64_t lda_bytes;
  const float* a_scale;
  const int32_t* row_token;
  const int32_t* row_index;
  const uint8_t* B;
  int64_t b_expert_rows;
  int64_t ldb_bytes;
  const float* b_scale;
  int k_bytes;
  uint16_t* C;
  int64_t ldc;
  int n_valid;
  // weight-gradient tiles (OUT_SPLIT): output columns [128, 256) of a tile go to C2
  // and columns [0, 128) to C, both at column nt*128 (the gate and up halves of a
  // w13-ordered tile: the dw1 / dw2 split)
  uint16_t* C2;
  // gate/up tiles: when set, the pre-activation gate and up values are also written
  // (bf16) in the packed column order, row stride 2*ldc: the backward's saved g, u
  uint16_t* gu_out;
  // weight-gradient tiles (OUT_F32): the fp32 accumulators are stored here (row
  // stride ldc) instead of bf16 to C (split-K partial sums)
  float* Cf;
};

// Stores a tile staged in LDS (BM rows of OCPR 16-byte chunks, row stride OSTR bytes)
// to the rows [m0, m_end) of `out` (row stride ld elements, chunk ch at out + 8 ch;
// chunks from column col0 + 8 ch >= n_valid are not stored).  A thread always handles
// the same chunk of every GEMM_THREADS / OCPR-th row, so its addresses advance by a
// fixed stride; LDS reads go out eight at a time ahead of their stores (one read, wait,
// store per iteration serialised the loop on the LDS latency).
template <int OCPR, int OSTR>
__device__ __forceinline__ void store_staged(const uint8_t* lds, int tid, int m0, int m_end, uint16_t* out,
                                             int64_t ld, int col0, int n_valid) {
  constexpr int RPI = GEMM_THREADS / OCPR;  // rows per iteration
  constexpr int NIT = BM / RPI;             // iterations per thread
  constexpr int CH = NIT < 8 ? NIT : 8;
  static_assert(GEMM_THREADS % OCPR == 0 && NIT % CH == 0, "store layout");
  const int ch = tid % OCPR, tr0 = tid / OCPR;
  const bool col_ok = col0 + ch * 8 < n_valid;
  const uint8_t* lp = lds + tr0 * OSTR + ch * 16;
  uint16_t* gp = out + (int64_t)(m0 + tr0) * ld + ch * 8;
  const int rows = m_end - m0 - tr0;  // this thread's rows: tr0 + RPI i < m_end - m0
#pragma unroll
  for (int h = 0; h < NIT; h += CH) {
    i32x4_t v[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) v[u] = *reinterpret_cast<const i32x4_t*>(lp + (h + u) * RPI * OSTR);
#pragma unroll
    for (int u = 0; u < CH; ++u)
      if (col_ok && (h + u) * RPI < rows) *reinterpret_cast<i32x4_t*>(gp + (int64_t)(h + u) * RPI * ld) = v[u];
  }
}

// Output of a weight-gradient tile: bf16 to C; bf16 with the column tile split
// between C and C2 (the gate and up halves of a w13-ordered tile); fp32 to Cf.
constexpr int OUT_BF16 = 0, OUT_SPLIT = 1, OUT_F32 = 2;

// One output tile: rows [m0, min(m0 + 256, m_end)) of expert e against B rows of
// full column tile nt (narrow part q when WNB < 4).
// FP8: A/B bytes are e4m3; a_scale per A row, b_scale per B row (global row index).
// GATHER: A is the unpermuted activation matrix and permuted row r is its row
// row_index[row_token[r]] (row_token[r] without row_index): the dispatch gather is
// fused into the A loads.
// RSCALE (bf16 gathered gate/up tiles): a_scale[row_token[r]] scales row r's gate and
// up values before the SiLU (the per-token RMSNorm scale of x: the norm weight is
// folded into the packed w1 / w2 rows, and a per-row scale commutes with the product).
// NMA: the row blocks of this wave that hold rows of the expert.  A wave's 128 rows
// are 4 blocks of 32; a slot's last tile is often partly empty, and its waves then
// run with NMA < 4 (the first NMA blocks), which skips the other blocks' fragment
// reads, MFMAs and epilogue (their accumulators stay 0 and are never stored).  The
// waves of a workgroup may differ in NMA: loads, LDS writes and barriers are the same.
template <bool GATE_UP, bool FP8, bool GATHER, int WNB, bool SAVE_GU = false, bool RSCALE = false, int NMA = 4>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, uint8_t* lds, int e, int m0, int m_end, int nt,
                                          int q) {
  static_assert(WNB == 4 || WNB == 2 || WNB == 1, "tile width");
  // bf16: 16x16x32 MFMAs, 16-row A and B blocks (MA x NBB per wave, NAB of them holding
  // rows); fp8: 32x32x64, 32-row blocks
  constexpr bool M16 = !FP8;
  constexpr int MA = M16 ? 8 : 4;
  constexpr int NAB = M16 ? 2 * NMA : NMA;
  constexpr int NBB = M16 ? 2 * WNB : WNB;
  using Acc = std::conditional_t<M16, f32x4_t, f32x16_t>;
  constexpr int ACCN = M16 ? 4 : 16;
  constexpr int NSUB = KB / 64;  // MFMA K-substeps per pipeline step (bf16: 32 of K, fp8: 64)
  constexpr int BNT = 64 * WNB;                  // B rows of the tile
  constexpr int TBB = BNT * KB;                  // bytes of one B stage tile
  constexpr int BLK_B = BNT * KB / 1024 / 4;     // B load blocks per wave per step
  constexpr int NBLK = BLK_PER_WAVE + BLK_B;     // load blocks per wave per step
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 31, lh = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t brow0 = (int64_t)e * g.b_expert_rows + (int64_t)nt * BN;  // full packed tile
  const __amdgpu_buffer_rsrc_t arsrc = make_rsrc(GATHER ? g.A : g.A + (int64_t)m0 * g.lda_bytes);
  const __amdgpu_buffer_rsrc_t brsrc = make_rsrc(g.B + brow0 * g.ldb_bytes);
  const int nk = g.k_bytes / KB;
  // LDS stage s: [A tile | B tile]
  auto la_buf = [&](int st) { return lds + st * (TB + TBB); };
  auto lb_buf = [&](int st) { return lds + st * (TB + TBB) + TB; };

  Acc acc[MA][NBB];
#pragma unroll
  for (int i = 0; i < MA; ++i)
#pragma unroll
    for (int j = 0; j < NBB; ++j)
#pragma unroll
      for (int r = 0; r < ACCN; ++r) acc[i][j][r] = 0.0f;
  // fp8 scales of the tile's A rows (thread = row) and B rows (thread = LDS B row),
  // loaded now and put in LDS for the epilogue (rows past the expert's end: 0)
  float sa_v = 0.0f, sb_v = 0.0f;
  if constexpr (FP8) {
    const int row = m0 + tid;
    if (row < m_end) sa_v = g.a_scale[row];
    if (tid < BNT) sb_v = g.b_scale[brow0 + b_packed_row<GATE_UP, WNB>(tid, q)];
  }
  static_assert(!RSCALE || (GATE_UP && GATHER && !FP8 && !SAVE_GU), "row scales are for bf16 gathered gate/up tiles");
  if constexpr (RSCALE) {
    const int row = m0 + tid;
    if (row < m_end) sa_v = g.a_scale[g.row_token[row]];
  }

  // Tile loads: a stage tile is a set of 1 KiB blocks (8 rows of 128 B); wave w loads
  // A blocks [8w, 8w+8) and B blocks [BLK_B w, BLK_B w + BLK_B) into registers and
  // writes them to LDS.  Lane l of a block covers bytes [16l, 16l+16) of it (tile row
  // 8q + l/8, physical chunk l%8) and so loads the logical chunk that swz() maps
  // there: the LDS write of a block is one contiguous, conflict-free 1 KiB.  A rows
  // past the expert's last row read as zeros (their results are never stored).
  const int rsub = lane / CPR, pc = lane % CPR;
  uint32_t a_off[BLK_PER_WAVE], b_off[8];
  const int a_last = m_end - 1 - m0;
  int ra[BLK_PER_WAVE];
#pragma unroll
  for (int qa = 0; qa < BLK_PER_WAVE; ++qa) {
    const int tr = (wave * BLK_PER_WAVE + qa) * RPB + rsub;
    ra[qa] = tr < a_last ? tr : a_last;
  }
  if constexpr (GATHER) {
    // batched: all row_token loads, then all row_index loads (two round trips)
#pragma unroll
    for (int qa = 0; qa < BLK_PER_WAVE; ++qa) ra[qa] = g.row_token[m0 + ra[qa]];
    if (g.row_index) {
#pragma unroll
      for (int qa = 0; qa < BLK_PER_WAVE; ++qa) ra[qa] = g.row_index[ra[qa]];
    }
  }
  // Tile rows past the expert's end load zeros instead: an offset beyond the buffer
  // window's 2 GiB record count makes the hardware return 0 without a memory access
  // (the scalar K offset is not range-checked, the per-lane offset is).  Their results
  // are never stored; zero operands spare the memory traffic and the MFMA power of
  // real data (the expert GEMMs run power-limited).
  constexpr uint32_t A_OOB = 0x80000000u;
#pragma unroll
  for (int qa = 0; qa < BLK_PER_WAVE; ++qa) {
    const int tr = (wave * BLK_PER_WAVE + qa) * RPB + rsub;
    const uint32_t chunk = (uint32_t)(pc ^ ((tr >> 1) & (CPR - 1))) << 4;
    a_off[qa] = tr > a_last ? A_OOB + chunk : (uint32_t)ra[qa] * (uint32_t)g.lda_bytes + chunk;
  }
#pragma unroll
  for (int qb = 0; qb < BLK_B; ++qb) {
    const int tr = (wave * BLK_B + qb) * RPB + rsub;
    const uint32_t chunk = (uint32_t)(pc ^ ((tr >> 1) & (CPR - 1))) << 4;
    b_off[qb] = (uint32_t)b_packed_row<GATE_UP, WNB>(tr, q) * (uint32_t)g.ldb_bytes + chunk;
  }
  i32x4_t stg[16];  // one step of this wave's tile data: A blocks, then B blocks
  // block qq: global -> registers (K-step kt, clamped to the last step)
  auto load_block = [&](int qq, int kt) {
    const int ks = kt < nk ? kt : nk - 1;
    if (qq < BLK_PER_WAVE)
      stg[qq] = __builtin_amdgcn_raw_buffer_load_b128(arsrc, a_off[qq], ks * KB, 0);
    else
      stg[qq] = __builtin_amdgcn_raw_buffer_load_b128(brsrc, b_off[qq - BLK_PER_WAVE], ks * KB, 0);
  };
  // block qq: registers -> LDS stage st
  auto write_block = [&](int qq, int st) {
    uint8_t* dst = qq < BLK_PER_WAVE ? la_buf(st) + (wave * BLK_PER_WAVE + qq) * 1024
                                     : lb_buf(st) + (wave * BLK_B + qq - BLK_PER_WAVE) * 1024;
    *reinterpret_cast<i32x4_t*>(dst + lane * 16) = stg[qq];
  };
  Frag<FP8> fa[2][MA], fb[2][NBB];
  const int r16 = lane & 15, lq = lane >> 4;
  auto rd = [&](int st, int i, Frag<FP8> (&a)[MA], Frag<FP8> (&b)[NBB]) {
    if constexpr (NMA > 0) {
      const uint8_t* la = la_buf(st);
      const uint8_t* lb = lb_buf(st);
      if constexpr (M16) {
#pragma unroll
        for (int j = 0; j < NBB; ++j)
          read_frag16(lb, b_lds_row<GATE_UP, WNB>(wn, j >> 1, 16 * (j & 1) + r16), i, lq, b[j]);
#pragma unroll
        for (int mi = 0; mi < NAB; ++mi) read_frag16(la, wm * 128 + mi * 16 + r16, i, lq, a[mi]);
      } else {
#pragma unroll
        for (int mi = 0; mi < NMA; ++mi) read_frag<FP8>(la, wm * 128 + mi * 32 + lr, i, lh, a[mi]);
#pragma unroll
        for (int j = 0; j < WNB; ++j) read_frag<FP8>(lb, b_lds_row<GATE_UP, WNB>(wn, j, lr), i, lh, b[j]);
      }
    }
  };
  auto mma1 = [&](Acc& c, const Frag<FP8>& b, const Frag<FP8>& a) {
    if constexpr (M16)
      mfma16(c, b, a);
    else
      mfma<FP8>(c, b, a);
  };
  auto mma = [&](const Frag<FP8> (&a)[MA], const Frag<FP8> (&b)[NBB]) {
#pragma unroll
    for (int mi = 0; mi < NAB; ++mi)
#pragma unroll
      for (int j = 0; j < NBB; ++j) mma1(acc[mi][j], b[j], a[mi]);
  };
  // MFMAs [lo, hi) of a substep (linear index mi * NBB + j)
  auto mma_part = [&](const Frag<FP8> (&a)[MA], const Frag<FP8> (&b)[NBB], auto lo_tag, auto hi_tag) {
    static_for<decltype(lo_tag)::value, decltype(hi_tag)::value>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      mma1(acc[x / NBB][x % NBB], b[x % NBB], a[x / NBB]);
    });
  };

  // Pipeline.  Step kt computes LDS stage kt%2 while the registers hold step kt+1's
  // tile data.  Those blocks are written into stage (kt+1)%2 (which every wave
  // stopped reading at step kt-1's barrier) over the substeps, each block reloaded
  // with step kt+2's data right after its write, so a load has a whole step to land
  // and the LDS write traffic is spread (bf16: about 6/5/5 sixteenths of the blocks
  // in substeps 0-2; fp8: half in each substep).  In the last substep, after most of
  // its MFMAs, the wave waits for its LDS writes and reads, then one barrier publishes
  // stage kt+1, whose first fragments are read under the last few MFMAs.  Register
  // dependencies give the vmcnt waits; the scheduling groups interleave the LDS and
  // memory operations with the MFMAs, fragment reads first.
  constexpr int RD = NMA > 0 ? (FP8 ? 2 : 1) * (NAB + NBB) : 0;  // LDS reads of a substep's fragments
  constexpr int NMS = NAB * NBB;                                    // MFMAs per substep
  for (int qq = 0; qq < NBLK; ++qq) load_block(qq, 0);
  for (int qq = 0; qq < NBLK; ++qq) write_block(qq, 0);
  for (int qq = 0; qq < NBLK; ++qq) load_block(qq, 1);
  wait_lgkmcnt0();
  barrier_nofence();
  if constexpr (!M16) rd(0, 0, fa[0], fb[0]);

  // bf16 (16x16 blocks): the K loop is emitted in program order, one MFMA at a time,
  // each followed by the LDS reads, block writes or reloads assigned to it and fenced
  // with sched_barrier.  (With scheduling groups the scheduler may take the MFMAs out of
  // order, and the register allocator then stops tying each MFMA's accumulator input to
  // its output: hundreds of accumulator copies per K-step.)  A 16x16x32 MFMA keeps the
  // matrix pipe 16 cycles, about what a 1 KiB LDS block write takes to issue, so the
  // schedule gives each MFMA at most one LDS or memory instruction where it can.
  // Substep i uses B fragment set fb[i] and the one A set fa[0]; MFMAs go row block by
  // row block.  Substep 0 reads substep 1's B fragments into fb[1] and each row block's
  // next A fragment right after that row block's last MFMA (an A ring: no second A set).
  // Substep 1 meets the other waves at the barrier that publishes stage nxt after MFMA
  // GB, then reads that stage's substep-0 fragments (B0, A0, B1, ..., each A after its
  // row block's last MFMA).  The block writes into stage nxt and the reloads of step kt+2
  // go over substep 0 and the part of substep 1 before the barrier, each reload a few
  // MFMAs after the write that frees its registers.
  constexpr bool FULL16 = NMS == 64 && NBB == 8 && NAB == 8 && NBLK == 16;
  constexpr int NR16 = NMS > 0 ? ((NBB + NAB) < NMS - 1 ? NBB + NAB : NMS - 1) : 0;
  constexpr int GB = FULL16 ? 31 : NMS - 1 - NR16;  // substep 1: the barrier follows MFMA GB
  constexpr int H0 = NBLK / 2;                      // block writes in substep 0 (the rest in substep 1)
  auto rdB16 = [&](int st, int i, int j, Frag<FP8>& b) {
    if constexpr (M16) read_frag16(lb_buf(st), b_lds_row<GATE_UP, WNB>(wn, j >> 1, 16 * (j & 1) + r16), i, lq, b);
  };
  auto rdA16 = [&](int st, int i, int mi) {
    if constexpr (M16) read_frag16(la_buf(st), wm * 128 + mi * 16 + r16, i, lq, fa[0][mi]);
  };
  auto sub16 = [&](int kt, auto i_tag, auto last_tag) {
    constexpr int i = decltype(i_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    const int cur = kt & 1, nxt = cur ^ 1;
    constexpr int NW = LAST ? 0 : (i == 0 ? H0 : NBLK - H0), QB = i == 0 ? 0 : H0;
    if constexpr (NMS == 0) {
      // a wave without rows: only its share of the tile loads and the barrier
      if constexpr (NW > 0) {
        static_for<0, NW>([&](auto wc) {
          write_block(QB + decltype(wc)::value, nxt);
          load_block(QB + decltype(wc)::value, kt + 2);
        });
      }
      if constexpr (i == 1 && !LAST) {
        wait_lgkmcnt0();
        barrier_nofence();
      }
      return;
    }
    // MFMA after which block write w / its reload go (w < NW; NW1 keeps the division
    // defined in the instantiations without block writes)
    constexpr int NW1 = NW > 0 ? NW : 1;
    constexpr auto w_at = [](int w) constexpr {
      if (FULL16) return i == 0 ? 16 + 6 * w : 4 * w;
      const int span = i == 0 ? NMS - 2 : GB - 2;
      return span > 0 ? 1 + (w * span) / NW1 : 0;
    };
    constexpr auto l_at = [](int w) constexpr {
      if (FULL16) return i == 0 ? 18 + 6 * w : 4 * w + 2;
      const int span = i == 0 ? NMS - 2 : GB - 2;
      return span > 0 ? 1 + (w * span) / NW1 : 0;
    };
    // substep 0: MFMA after which next-substep read B_j / A_mi goes
    constexpr auto b0_at = [](int j) constexpr { return FULL16 ? 2 * j : (j < NMS ? j : NMS - 1); };
    // substep 1: post-barrier read k (0: B0, 1: A0, 2 ..: B1 .. B_{NBB-1}, then A1 ..)
    constexpr auto post_at = [](int k, int kind, int idx) constexpr {
      const int e0 = GB + 1 + (FULL16 ? 2 * k + 1 : k);
      const int e1 = kind == 1 ? idx * NBB + NBB - 1 : 0;
      const int at = e0 > e1 ? e0 : e1;
      return at < NMS - 1 ? at : NMS - 1;
    };
    static_for<0, NMS>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      constexpr int mi = g / NBB, j = g % NBB;
      mma1(acc[mi][j], fb[i][j], fa[0][mi]);
      __builtin_amdgcn_sched_barrier(0);
      // block writes, then reloads (substep 1: all before the barrier)
      static_for<0, NW>([&](auto wc) {
        constexpr int w = decltype(wc)::value;
        if constexpr (w_at(w) == g) write_block(QB + w, nxt);
      });
      static_for<0, NW>([&](auto wc) {
        constexpr int w = decltype(wc)::value;
        if constexpr (l_at(w) == g) load_block(QB + w, kt + 2);
      });
      if constexpr (i == 0) {
        static_for<0, NBB>([&](auto jc) {
          constexpr int jj = decltype(jc)::value;
          if constexpr (b0_at(jj) == g) rdB16(cur, 1, jj, fb[1][jj]);
        });
        if constexpr (j == NBB - 1) rdA16(cur, 1, mi);
      } else if constexpr (!LAST) {
        if constexpr (g == GB) {
          wait_lgkmcnt0();
          barrier_nofence();
        }
        static_for<0, NBB + NAB>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          constexpr int kind = k == 0 ? 0 : k == 1 ? 1 : k < NBB + 1 ? 0 : 1;
          constexpr int idx = k == 0 ? 0 : k == 1 ? 0 : k < NBB + 1 ? k - 1 : k - NBB;
          if constexpr (post_at(k, kind, idx) == g) {
            if constexpr (kind == 0)
              rdB16(nxt, 0, idx, fb[0][idx]);
            else
              rdA16(nxt, 0, idx);
          }
        });
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  auto step16 = [&](int kt, auto last_tag) {
    sub16(kt, std::integral_constant<int, 0>{}, last_tag);
    sub16(kt, std::integral_constant<int, 1>{}, last_tag);
  };
  if constexpr (M16) {
    if constexpr (NMA > 0) {
#pragma unroll
      for (int j = 0; j < NBB; ++j) rdB16(0, 0, j, fb[0][j]);
#pragma unroll
      for (int mi = 0; mi < NAB; ++mi) rdA16(0, 0, mi);
    }
  }
  auto step = [&](int kt, auto last_tag) {
    if constexpr (M16) {
      step16(kt, last_tag);
      return;
    }
    constexpr bool LAST = decltype(last_tag)::value;
    const int cur = kt & 1, nxt = cur ^ 1;
    static_for<0, NSUB>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr int bi = i & 1;
      // blocks [q0, q1) are written and reloaded in this substep.  bf16 (4 substeps):
      // about 6/5/5 sixteenths in substeps 0-2.  fp8 (2 substeps): half in each, the
      // last substep's before its barrier (all in substep 0 crowded the LDS queue with
      // that substep's fragment reads: 3% slower).
      constexpr int C1 = (NBLK * 6 + 8) / 16, C2 = (NBLK * 11 + 8) / 16;
      constexpr int q0 = NSUB == 4 ? (i == 0 ? 0 : i == 1 ? C1 : i == 2 ? C2 : NBLK) : i * NBLK / NSUB;
      constexpr int q1 = NSUB == 4 ? (i == 0 ? C1 : i == 1 ? C2 : NBLK) : (i + 1) * NBLK / NSUB;
      constexpr int nq = LAST ? 0 : q1 - q0;
      constexpr bool RDN = i + 1 < NSUB || !LAST;
      // next substep's fragments first: they are on the MFMA critical path
      if constexpr (i + 1 < NSUB) {
        rd(cur, i + 1, fa[bi ^ 1], fb[bi ^ 1]);
      } else if constexpr (!LAST) {
        // last substep: its share of the block writes and most of its MFMAs go out before
        // the wait and the barrier that publish the next stage (the MFMAs read registers
        // only), so the MFMA pipe is busy while the waves meet; the next stage's first
        // fragment reads then issue two per MFMA under the remaining NA.  (Barrier first:
        // each step lost the pipe for the wait on the writes plus the barrier.)
        constexpr int NA = (RD + 1) / 2 < NMS ? (RD + 1) / 2 : NMS;
        if constexpr (nq > 0) {
          static_for<q0, q1>([&](auto qc) { write_block(decltype(qc)::value, nxt); });
          static_for<q0, q1>([&](auto qc) { load_block(decltype(qc)::value, kt + 2); });
        }
        if constexpr (NMS - NA > 0) {
          mma_part(fa[bi], fb[bi], std::integral_constant<int, 0>{}, std::integral_constant<int, NMS - NA>{});
          sched_even<NMS - NA, nq, nq>();
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_lgkmcnt0();
        barrier_nofence();
        rd(nxt, 0, fa[bi ^ 1], fb[bi ^ 1]);
        if constexpr (NA > 0) {
          mma_part(fa[bi], fb[bi], std::integral_constant<int, NMS - NA>{}, std::integral_constant<int, NMS>{});
          sched_spread<NA, RD, 0, 0>();
        }
        __builtin_amdgcn_sched_barrier(0);
        return;
      }
      if constexpr (nq > 0) {
        static_for<q0, q1>([&](auto qc) { write_block(decltype(qc)::value, nxt); });
        static_for<q0, q1>([&](auto qc) { load_block(decltype(qc)::value, kt + 2); });
      }
      mma(fa[bi], fb[bi]);
      sched_spread<NMS, (RDN ? RD : 0), nq, nq>();
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  for (int kt = 0; kt + 1 < nk; ++kt) step(kt, std::false_type{});
  step(nk - 1, std::true_type{});

  // ---- epilogue.  The MFMAs take the B fragment as their first operand, so block
  // (mi, j) accumulates the transposed product: acc[mi][j][4c+t] is A row mi*32 + lr
  // against B row 8c + 4lh + t of B block j, i.e. output row wm*128 + mi*32 + lr and
  // four consecutive output columns per c.  A lane packs each such run to 8 bytes of
  // bf16 in registers and writes it to an LDS tile (rows padded by 16 bytes), which
  // then goes out with 16-byte stores along rows.
  static_assert(!SAVE_GU || GATE_UP, "g/u saving is for gate/up tiles");
  static_assert(!(SAVE_GU && FP8 && M16), "fp8 tiles use 32x32 blocks");
  constexpr int NC = GATE_UP ? 32 * WNB : 64 * WNB;  // output columns of the tile
  // output column blocks per wave, and 4-column runs per block and lane: a gate/up
  // WNB = 1 block holds its gate values in runs c = 0, 1 and the up values of the same
  // columns in runs c + 2
  constexpr bool GU1 = GATE_UP && WNB == 1;
  constexpr int NJ = GU1 ? 1 : GATE_UP ? WNB / 2 : WNB;
  constexpr int NCR = GU1 ? 2 : 4;
  constexpr int OSTR = NC * 2 + 16;                  // LDS row stride (bytes)
  float* const sa_l = reinterpret_cast<float*>(lds + SCALE_LDS);
  float* const sb_l = sa_l + BM;
  if constexpr (FP8) {
    sa_l[tid] = sa_v;
    if (tid < BNT) sb_l[tid] = sb_v;
  }
  if constexpr (RSCALE) sa_l[tid] = sa_v;
  __syncthreads();
  // The scales go to registers first: the B-row scales of the lane's 16 B rows of each
  // block once, the A-row scale of each row block before its results.  Read from LDS
  // per output element, they were re-read after every staging write (the compiler
  // cannot tell the two LDS areas apart).
  float sbr[WNB][16];
#pragma unroll
  for (int j = 0; j < WNB; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      sbr[j][r] = FP8 ? sb_l[b_lds_row<GATE_UP, WNB>(wn, j, 8 * (r >> 2) + 4 * lh + (r & 3))] : 1.0f;
  float sar = 1.0f;
  auto result = [&](int mi, int r, int jo) -> float {
    if (GATE_UP) {
      constexpr int UJ = GU1 ? 0 : WNB / 2, UR = GU1 ? 8 : 0;  // up value: block jo + UJ, run + UR/4
      float gg = acc[mi][jo][r], u = acc[mi][jo + UJ][r + UR];
      if (FP8) {
        gg *= sar * sbr[jo][r];
        u *= sar * sbr[jo + UJ][r + UR];
      }
      if (RSCALE) {
        gg *= sar;
        u *= sar;
      }
      return silu_fast_f32(gg) * u;
    } else {
      float v = acc[mi][jo][r];
      if (FP8) v *= sar * sbr[jo][r];
      return v;
    }
  };
  auto pack4 = [](float a, float b, float c, float d) {
    const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{c, d}, bf16x2_t));
    return i32x2_t{(int)lo, (int)hi};
  };
  if constexpr (M16) {
    // 16x16 blocks: acc[mi][j][t] is output row wm*128 + mi*16 + l%16 against B row
    // 4 (l/16) + t of 16-row B block j: one run of four output columns per block (gate/up:
    // gate block jo, up block jo + NBB/2, same columns)
    constexpr int NJ16 = GATE_UP ? NBB / 2 : NBB;
    uint8_t* const wb16 = lds + (wm * 128 + r16) * OSTR + (wn * (NC / 2) + 4 * lq) * 2;
#pragma unroll
    for (int mi = 0; mi < NAB; ++mi) {
      if constexpr (RSCALE) sar = sa_l[wm * 128 + mi * 16 + r16];
#pragma unroll
      for (int jo = 0; jo < NJ16; ++jo) {
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if constexpr (GATE_UP) {
            float gg = acc[mi][jo][t], u = acc[mi][jo + NBB / 2][t];
            if constexpr (RSCALE) {
              gg *= sar;
              u *= sar;
            }
            v[t] = silu_fast_f32(gg) * u;
          } else {
            v[t] = acc[mi][jo][t];
          }
        }
        *reinterpret_cast<i32x2_t*>(wb16 + mi * 16 * OSTR + jo * 32) = pack4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
    // lane's row of block 0 and its first column (c = 0) of output column block 0
    uint8_t* const wbase = lds + (wm * 128 + lr) * OSTR + (wn * (NC / 2) + 4 * lh) * 2;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      if (mi >= NMA) break;  // rows past the expert's end: never stored
      if constexpr (FP8 || RSCALE) sar = sa_l[wm * 128 + mi * 32 + lr];
#pragma unroll
      for (int jo = 0; jo < NJ; ++jo)
#pragma unroll
        for (int c = 0; c < NCR; ++c)
          *reinterpret_cast<i32x2_t*>(wbase + mi * 32 * OSTR + (jo * 32 + 8 * c) * 2) =
              pack4(result(mi, 4 * c, jo), result(mi, 4 * c + 1, jo), result(mi, 4 * c + 2, jo),
                    result(mi, 4 * c + 3, jo));
    }
  }
  __syncthreads();
  constexpr int OCPR = NC * 2 / 16;  // 16-byte chunks per output row
  const int col0 = (GATE_UP ? nt * 128 : nt * 256) + q * NC;
  store_staged<OCPR, OSTR>(lds, tid, m0, m_end, g.C + col0, g.ldc, col0, g.n_valid);

  // training forward: the pre-activation gate and up values of the tile, bf16, in the
  // packed column order (row stride 2*ldc), for the SwiGLU backward (fp8: descaled by
  // the row and column scales, the values the SwiGLU of the epilogue took)
  if constexpr (SAVE_GU) {
    constexpr int NC2 = 64 * WNB;
    constexpr int OSTR2 = NC2 * 2 + 16;
    __syncthreads();
    if constexpr (M16) {
      uint8_t* const wb2 = lds + (wm * 128 + r16) * OSTR2 + 4 * lq * 2;
#pragma unroll
      for (int mi = 0; mi < NAB; ++mi)
#pragma unroll
        for (int j = 0; j < NBB; ++j) {
          const int col = b_lds_row<true, WNB>(wn, j >> 1, 16 * (j & 1));
          *reinterpret_cast<i32x2_t*>(wb2 + mi * 16 * OSTR2 + col * 2) =
              pack4(acc[mi][j][0], acc[mi][j][1], acc[mi][j][2], acc[mi][j][3]);
        }
    } else {
      uint8_t* const wb2 = lds + (wm * 128 + lr) * OSTR2 + 4 * lh * 2;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (mi >= NMA) break;
        if constexpr (FP8) sar = sa_l[wm * 128 + mi * 32 + lr];
#pragma unroll
        for (int j = 0; j < WNB; ++j) {
          const int col = b_lds_row<true, WNB>(wn, j, 0);
          auto gv = [&](int r) { return FP8 ? acc[mi][j][r] * (sar * sbr[j][r]) : acc[mi][j][r]; };
#pragma unroll
          for (int c = 0; c < 4; ++c)
            *reinterpret_cast<i32x2_t*>(wb2 + mi * 32 * OSTR2 + (col + 8 * c) * 2) =
                pack4(gv(4 * c), gv(4 * c + 1), gv(4 * c + 2), gv(4 * c + 3));
        }
      }
    }
    __syncthreads();
    constexpr int OCPR2 = NC2 * 2 / 16;
    // chunk ch of a staged row lands at packed column b_packed_row(8 ch): contiguous
    // within each 8-column chunk, so the per-thread base column is that of its chunk
    const int ch2 = tid % OCPR2;
    const int gcol2 = nt * 256 + b_packed_row<true, WNB>(ch2 * 8, q);
    store_staged<OCPR2, OSTR2>(lds, tid, m0, m_end, g.gu_out + gcol2 - ch2 * 8, 2 * g.ldc, 0, 1 << 30);
  }
}

// Work of workgroup blockIdx.x.  The tiles (slot, column tile) are numbered densely
// (dense_tile); with n_cu workgroups resident at a time, the first R = N/n_cu full
// rounds take one tile per workgroup in the XCD-aware order.  The N - R n_cu tiles
// left would occupy few compute units for a whole tile time, so when they fit
// (split > 1: at most n_cu / split of them) each is split into `split` narrow tiles
// of 1/split of its columns (the full K), which all run at once.  A narrow tile
// computes every output element with the same MFMA sequence as the full tile, so
// the results are identical.  split = 1 keeps the tail tiles whole.
template <bool GATE_UP, bool FP8, bool GATHER, bool SAVE_GU = false, bool RSCALE = false>
__global__ __launch_bounds__(GEMM_THREADS, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void grouped_gemm_kernel(
    GemmArgs g, const int32_t* __restrict__ offsets, int E, int n_tiles, int n_cu, int allow_split) {
  static_assert(!(GATHER && FP8), "the fp8 path reads rows quantised by the dispatch");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[GEMM_LDS];
  const SlotTable st = load_slots(offsets, E);
  const int n_all = st.n_slots * n_tiles;
  const int rounds = n_all / n_cu, base = rounds * n_cu, n_rest = n_all - base;
  int split = 1;
  if (allow_split && n_rest > 0) {
    if (4 * n_rest <= n_cu)
      split = 4;
    else if (2 * n_rest <= n_cu)
      split = 2;
  }
  const int L = blockIdx.x;
  int t, q = 0;
  if (L < base) {
    t = (base % (NXCD * SB_TILES)) == 0 ? xcd_tile(L) : L;
  } else if (split == 1) {
    if (L >= n_all) return;
    t = L;
  } else {
    const int u = L - base;
    if (u >= n_rest * split) return;
    t = base + u / split;
    q = u % split;
  }
  int slot, nt, e, m0, m_end;
  dense_tile(t, st.n_slots, n_tiles, slot, nt);
  find_slot(st, E, slot, e, m0, m_end);
  if (L < base || split == 1) {
    // row blocks of this wave holding rows (wave-uniform): 4 (more than 64 rows), 2, 1, 0
    const int wrows = m_end - m0 - (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 1) * 128;
    if (wrows > 64)
      gemm_tile<GATE_UP, FP8, GATHER, 4, SAVE_GU, RSCALE, 4>(g, lds, e, m0, m_end, nt, 0);
    else if (wrows > 32)
      gemm_tile<GATE_UP, FP8, GATHER, 4, SAVE_GU, RSCALE, 2>(g, lds, e, m0, m_end, nt, 0);
    else if (wrows > 0)
      gemm_tile<GATE_UP, FP8, GATHER, 4, SAVE_GU, RSCALE, 1>(g, lds, e, m0, m_end, nt, 0);
    else
      gemm_tile<GATE_UP, FP8, GATHER, 4, SAVE_GU, RSCALE, 0>(g, lds, e, m0, m_end, nt, 0);
  } else if (split == 2)
    gemm_tile<GATE_UP, FP8, GATHER, 2, SAVE_GU, RSCALE>(g, lds, e, m0, m_end, nt, q);
  else
    gemm_tile<GATE_UP, FP8, GATHER, 1, SAVE_GU, RSCALE>(g, lds, e, m0, m_end, nt, q);
}

// ---------------------------------------------------------------- weight gradients, row-major operands
// C_e[m, n] = sum over expert e's rows r of A[r, m] * B[r, n] with A (rows, lda) and B
// (rows, ldb) row-major and the rows of expert e = [offsets[e], offsets[e+1]): the
// weight gradients read straight from the permuted row buffers, no transposes.
// K advances 64 rows per step.  A stage holds 64 rows x 256 columns (512 B per row) of
// A and of B, row-major, with the 64-byte segments of row r XOR-ed by
// f(r) = (r & 3) | ((r >> 1) & 4).  MFMA operands come from ds_read_b64_tr_b16: in each
// 16-lane group, lane i receives element i mod 4 of the 8-byte chunks addressed by
// lanes 4p + i/4 (p = 0..3), so lanes 4p + c addressing row k0 + p, columns c0 + 4c
// give lane i column c0 + i at rows k0 .. k0 + 3: half an operand fragment (the
// second read takes rows k0 + 4 .. k0 + 7).  The 8 rows of one read fall in 8 distinct
// segments, two per bank group: the 512 bytes take the minimum two LDS passes.
// Rows past the expert's end read as zero: each operand's buffer window ends at the
// expert's last row (raw buffer loads past the window return 0).
constexpr int TN_KR = 64;                 // K rows per step
constexpr int TN_ROWB = 512;              // bytes of a 256-column bf16 tile row
constexpr int TN_TILE = TN_KR * TN_ROWB;  // 32 KiB
__device__ __forceinline__ int tn_f(int r) { return (r & 3) | ((r >> 1) & 4); }
// LDS byte offset of 16-byte chunk c (0..31) of stage-tile row r
__device__ __forceinline__ int tn_chunk(int r, int c) { return r * TN_ROWB + ((((c >> 2) ^ tn_f(r)) << 2) | (c & 3)) * 16; }
// LDS byte offset of the 8 bytes at column col (a multiple of 4) of stage-tile row r
__device__ __forceinline__ int tn_elem(int r, int col) { return r * TN_ROWB + (((col >> 5) ^ tn_f(r)) << 6) + ((col & 31) << 1); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_window(const void* base, int64_t bytes) {
  const int n = bytes < 0 ? 0 : (bytes > 0x7fffffffll ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

typedef short tr4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ Frag<false> read_frag_tr(const uint8_t* l, int row, int col) {
  const tr4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (KMOE_LDS tr4_t*)(l + tn_elem(row, col)));
  const tr4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (KMOE_LDS tr4_t*)(l + tn_elem(row + 4, col)));
  Frag<false> f;
  f.v = __builtin_bit_cast(bf16x8_t, (short __attribute__((ext_vector_type(8)))){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1],
                                                                                 hi[2], hi[3]});
  return f;
}

// One 256 x 256 output tile of expert rows [row0, row0 + nrows), output rows [m0, ...),
// columns [256 nt, ...); g.C / g.C2 / g.Cf already point at the expert's output.
template <int OUT>
__device__ __forceinline__ void wgrad_tn_tile(const GemmArgs& g, uint8_t* lds, int64_t row0, int nrows, int m0, int M,
                                              int nt) {
  constexpr int NBLK = 16;  // 8 A + 8 B blocks of 1 KiB (2 rows x 512 B) per wave per step
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = nt * 256;
  const __amdgpu_buffer_rsrc_t arsrc =
      make_rsrc_window(g.A + row0 * g.lda_bytes + (int64_t)m0 * 2, (int64_t)nrows * g.lda_bytes - (int64_t)m0 * 2);
  const __amdgpu_buffer_rsrc_t brsrc =
      make_rsrc_window(g.B + row0 * g.ldb_bytes + (int64_t)n0 * 2, (int64_t)nrows * g.ldb_bytes - (int64_t)n0 * 2);
  const int nk = (nrows + TN_KR - 1) / TN_KR;
  auto la_buf = [&](int st) { return lds + st * 2 * TN_TILE; };
  auto lb_buf = [&](int st) { return lds + st * 2 * TN_TILE + TN_TILE; };

  // 8 x 8 blocks of 16 x 16 per wave (v_mfma_f32_16x16x32_bf16, as the forward tiles)
  f32x4_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // block qq < 8: A block 8 wave + qq (tile rows 2b, 2b + 1; lane: row 2b + lane/32,
  // 16-byte chunk lane % 32); qq >= 8: the B block likewise
  uint32_t voff[NBLK];
  int dst[8];
#pragma unroll
  for (int qq = 0; qq < 8; ++qq) {
    const int tr = 2 * (wave * 8 + qq) + (lane >> 5), c = lane & 31;
    voff[qq] = (uint32_t)tr * (uint32_t)g.lda_bytes + (uint32_t)c * 16u;
    voff[qq + 8] = (uint32_t)tr * (uint32_t)g.ldb_bytes + (uint32_t)c * 16u;
    dst[qq] = tn_chunk(tr, c);
  }
  i32x4_t stg[NBLK];
  // The step's row offset goes into the per-lane (VGPR) offset: the buffer range check
  // covers the VGPR and instruction offsets but not the scalar one, and it is what
  // turns the rows past the expert's end into zeros.  Offsets and the window are
  // multiples of 16 bytes, so a 16-byte load is either wholly inside or wholly outside.
  const uint32_t astep = (uint32_t)TN_KR * (uint32_t)g.lda_bytes, bstep = (uint32_t)TN_KR * (uint32_t)g.ldb_bytes;
  auto load_block = [&](int qq, int kt) {
    const uint32_t ks = (uint32_t)(kt < nk ? kt : nk - 1);
    if (qq < 8)
      stg[qq] = __builtin_amdgcn_raw_buffer_load_b128(arsrc, voff[qq] + ks * astep, 0, 0);
    else
      stg[qq] = __builtin_amdgcn_raw_buffer_load_b128(brsrc, voff[qq] + ks * bstep, 0, 0);
  };
  auto write_block = [&](int qq, int st) {
    uint8_t* base = qq < 8 ? la_buf(st) : lb_buf(st);
    *reinterpret_cast<i32x4_t*>(base + dst[qq & 7]) = stg[qq];
  };
  // operand fragments of K-substep i (32 rows of K): lane group kq = lane/16 takes rows
  // 32 i + 8 kq .. + 7, lane l%16 one column of a 16-column block: two transpose reads
  // (rows 8 kq + (l%16)/4 and + 4, columns base + 4 (l%4)) give lane l column base + l%16
  // at eight consecutive rows, the 16x16x32 operand fragment
  const int kq = lane >> 4, i16 = lane & 15;
  const int frow = 8 * kq + (i16 >> 2), fcol = 4 * (i16 & 3);
  Frag<false> fa[8], fb[2][8];
  auto rdA = [&](int st, int i, int mb) { fa[mb] = read_frag_tr(la_buf(st), 32 * i + frow, wm * 128 + mb * 16 + fcol); };
  auto rdB = [&](int st, int i, int nb, Frag<false>& b) {
    b = read_frag_tr(lb_buf(st), 32 * i + frow, wn * 128 + nb * 16 + fcol);
  };
  // the tile's pipeline: step kt computes stage kt%2 while the registers hold step kt+1's
  // data, written into the other stage and reloaded with step kt+2's; one barrier per step.
  // As in the forward tiles, the MFMAs go in program order, one at a time, each followed
  // by the LDS reads, block writes or reloads assigned to it (sched_barrier fences).  Two
  // K = 32 substeps per 64-row step; substep i uses B set fb[i] and the A ring fa: substep
  // 0 reads substep 1's B fragments (MFMAs 0, 2, .., 14) and each A fragment after its row
  // block's last MFMA; substep 1 meets the other waves at the barrier after MFMA 31, then
  // reads the next step's substep-0 fragments from stage nxt.  Block writes into stage nxt
  // and the reloads of step kt+2 go over substep 0 (from MFMA 16) and substep 1 before the
  // barrier, each reload two MFMAs after the write that frees its registers.
  constexpr int GB = 31;
  auto sub = [&](int kt, auto i_tag, auto last_tag) {
    constexpr int i = decltype(i_tag)::value;
    constexpr bool LAST = decltype(last_tag)::value;
    const int cur = kt & 1, nxt = cur ^ 1;
    constexpr int NW = LAST ? 0 : NBLK / 2, QB = i == 0 ? 0 : NBLK / 2;
    constexpr auto w_at = [](int w) constexpr { return i == 0 ? 16 + 6 * w : 4 * w; };
    constexpr auto post_at = [](int k, int kind, int idx) constexpr {
      const int e0 = GB + 2 + 2 * k;
      const int e1 = kind == 1 ? idx * 8 + 7 : 0;
      const int at = e0 > e1 ? e0 : e1;
      return at < 63 ? at : 63;
    };
    static_for<0, 64>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      constexpr int mb = g / 8, nb = g % 8;
      // transposed product: lane l holds row m0 + .. + l%16, columns 4 (l/16) .. + 3
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[i][nb].v, fa[mb].v, acc[mb][nb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, NW>([&](auto wc) {
        constexpr int w = decltype(wc)::value;
        if constexpr (w_at(w) == g) write_block(QB + w, nxt);
      });
      static_for<0, NW>([&](auto wc) {
        constexpr int w = decltype(wc)::value;
        if constexpr (w_at(w) + 2 == g) load_block(QB + w, kt + 2);
      });
      if constexpr (i == 0) {
        if constexpr (g < 16 && g % 2 == 0) rdB(cur, 1, g / 2, fb[1][g / 2]);
        if constexpr (nb == 7) rdA(cur, 1, mb);
      } else if constexpr (!LAST) {
        if constexpr (g == GB) {
          wait_lgkmcnt0();
          barrier_nofence();
        }
        // post-barrier reads k: 0: B0, 1: A0, 2 .. 8: B1 .. B7, 9 .. 15: A1 .. A7
        static_for<0, 16>([&](auto kc) {
          constexpr int k = decltype(kc)::value;
          constexpr int kind = k == 0 ? 0 : k == 1 ? 1 : k < 9 ? 0 : 1;
          constexpr int idx = k == 0 ? 0 : k == 1 ? 0 : k < 9 ? k - 1 : k - 8;
          if constexpr (post_at(k, kind, idx) == g) {
            if constexpr (kind == 0)
              rdB(nxt, 0, idx, fb[0][idx]);
            else
              rdA(nxt, 0, idx);
          }
        });
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  for (int qq = 0; qq < NBLK; ++qq) load_block(qq, 0);
  for (int qq = 0; qq < NBLK; ++qq) write_block(qq, 0);
  for (int qq = 0; qq < NBLK; ++qq) load_block(qq, 1);
  wait_lgkmcnt0();
  barrier_nofence();
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) rdB(0, 0, nb, fb[0][nb]);
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) rdA(0, 0, mb);
  auto step = [&](int kt, auto last_tag) {
    sub(kt, std::integral_constant<int, 0>{}, last_tag);
    sub(kt, std::integral_constant<int, 1>{}, last_tag);
  };
  for (int kt = 0; kt + 1 < nk; ++kt) step(kt, std::false_type{});
  step(nk - 1, std::true_type{});

  // ---- epilogue: acc[mb][nb][t] is row wm*128 + mb*16 + l%16, column wn*128 + nb*16 +
  // 4 (l/16) + t of the tile
  if constexpr (OUT == OUT_F32) {
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int row = m0 + wm * 128 + mb * 16 + i16;
          const int col = n0 + wn * 128 + nb * 16 + 4 * kq + t;
          if (row < M && col < g.n_valid) g.Cf[(int64_t)row * g.ldc + col] = acc[mb][nb][t];
        }
  } else {
    // bf16 through LDS (rows padded by 16 bytes): a lane's four columns as 8 bytes, then
    // 16-byte row stores
    constexpr int OSTR = 256 * 2 + 16;
    __syncthreads();
    uint8_t* const wbase = lds + (wm * 128 + i16) * OSTR + (wn * 128 + 4 * kq) * 2;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{acc[mb][nb][0], acc[mb][nb][1]}, bf16x2_t));
        const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{acc[mb][nb][2], acc[mb][nb][3]}, bf16x2_t));
        *reinterpret_cast<i32x2_t*>(wbase + mb * 16 * OSTR + nb * 32) = i32x2_t{(int)lo, (int)hi};
      }
    __syncthreads();
    for (int c = tid; c < BM * 32; c += GEMM_THREADS) {
      const int trow = c >> 5, tc = (c & 31) * 8;  // tile row, first column of the 8
      const int grow = m0 + trow;
      uint16_t* base = g.C;
      int gcol = n0 + tc;
      if constexpr (OUT == OUT_SPLIT) {
        base = tc < 128 ? g.C : g.C2;
        gcol = nt * 128 + (tc & 127);
      }
      if (grow < M && gcol < g.n_valid)
        *reinterpret_cast<i32x4_t*>(base + (int64_t)grow * g.ldc + gcol) =
            *reinterpret_cast<const i32x4_t*>(lds + trow * OSTR + tc * 2);
    }
  }
}

template <int OUT>
__global__ __launch_bounds__(GEMM_THREADS, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void wgrad_rows_kernel(
    GemmArgs g, const int32_t* __restrict__ offsets, int E, int M, int n_mt, int n_nt, int64_t c_expert_stride) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * TN_TILE > BM * (256 * 2 + 16) ? 4 * TN_TILE : BM * (256 * 2 + 16)];
  const int n_all = E * n_mt * n_nt;
  const int L = blockIdx.x;
  if (L >= n_all) return;
  const int t = (n_all % (NXCD * SB_TILES)) == 0 ? xcd_tile(L) : L;
  const int per_e = n_mt * n_nt;
  const int e = t / per_e, rem = t - e * per_e;
  int mt, nt;
  dense_tile(rem, n_mt, n_nt, mt, nt);
  const int row0 = __builtin_amdgcn_readfirstlane(offsets[e]);
  const int nrows = __builtin_amdgcn_readfirstlane(offsets[e + 1]) - row0;
  GemmArgs ge = g;
  ge.C = g.C ? g.C + (int64_t)e * c_expert_stride : nullptr;
  ge.C2 = g.C2 ? g.C2 + (int64_t)e * c_expert_stride : nullptr;
  ge.Cf = g.Cf ? g.Cf + (int64_t)e * c_expert_stride : nullptr;
  const int m0 = mt * BM;
  if (nrows <= 0) {
    // no rows: a zero gradient tile
    for (int c = threadIdx.x; c < BM * 128; c += GEMM_THREADS) {
      const int grow = m0 + c / 128, tc = 2 * (c % 128);
      if (grow >= M) continue;
      if constexpr (OUT == OUT_F32) {
        const int gcol = nt * 256 + tc;
        if (gcol < g.n_valid) ge.Cf[(int64_t)grow * g.ldc + gcol] = 0.0f;
        if (gcol + 1 < g.n_valid) ge.Cf[(int64_t)grow * g.ldc + gcol + 1] = 0.0f;
      } else {
        uint16_t* base = ge.C;
        int gcol = nt * 256 + tc;
        if constexpr (OUT == OUT_SPLIT) {
          base = tc < 128 ? ge.C : ge.C2;
          gcol = nt * 128 + (tc & 127);
        }
        if (gcol < g.n_valid) *reinterpret_cast<uint32_t*>(base + (int64_t)grow * g.ldc + gcol) = 0u;
      }
    }
    return;
  }
  wgrad_tn_tile<OUT>(ge, lds, row0, nrows, m0, M, nt);
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
// finalize_scale_kernel once the rows have been quantised).  Workgroup (column block,
// row block, expert): each thread takes the max over COLS_ROWS rows of its column and
// merges it with an integer atomicMax on the float's bits (non-negative floats order
// like their bit patterns; max is order-independent, so the result is deterministic).
// The scale buffer starts at 0 (zero_f32_kernel).
constexpr int COLS_ROWS = 64;
template <bool IN_F32>
__global__ __launch_bounds__(256) void col_scale_kernel(const void* __restrict__ in, int R, int Cn,
                                                        int64_t in_expert_stride, int half, bool gate_up,
                                                        float* __restrict__ scale, int64_t out_rows) {
  const int e = blockIdx.z;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= Cn) return;
  const int r0 = blockIdx.y * COLS_ROWS, r1 = min(R, r0 + COLS_ROWS);
  float amax = 0.0f;
  for (int r = r0; r < r1; ++r) {
    const int64_t off = (int64_t)e * in_expert_stride + (int64_t)r * Cn + c;
    const float v = IN_F32 ? static_cast<const float*>(in)[off] : bf16_to_f32(static_cast<const uint16_t*>(in)[off]);
    amax = fmaxf(amax, fabsf(v));
  }
  const int64_t orow = gate_up ? (int64_t)(c / 128) * 256 + half * 128 + (c % 128) : (int64_t)c;
  atomicMax(reinterpret_cast<unsigned int*>(scale + (int64_t)e * out_rows + orow), __float_as_uint(amax));
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

// bf16 pack of one weight matrix per expert, in[e] (R x Cn) row-major -> out rows
// (out[e][map(c)][r] = in[e][r][c], map as in pack_transpose_kernel), 16 bytes per
// global access: a 64 x 64 tile is read as 8-element row vectors (bf16 16 B, f32 2 x
// 16 B), transposed through LDS, and written as 8-element vectors of output rows.
// Entries of out that no input element maps to (the pad after each row, padding
// rows) are left alone (pack_pad_kernel zeroes them).
template <bool IN_F32>
__global__ __launch_bounds__(256) void pack_t16_kernel(const void* __restrict__ in, int R, int Cn,
                                                       int64_t in_expert_stride, int half, bool gate_up,
                                                       uint16_t* __restrict__ out, int64_t out_rows, int out_ld) {
  __shared__ uint16_t tile[64][72];  // [input col][input row], rows padded to 144 B
  const int e = blockIdx.z;
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tid = threadIdx.x;
  // load: thread -> (row r0 + tid/8 + 32 i, cols c0 + 8 (tid%8) .. +8), i = 0, 1
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rr = tid / 8 + 32 * i, cc = 8 * (tid % 8);
    const int r = r0 + rr, c = c0 + cc;
    uint16_t v[8];
    const int64_t off = (int64_t)e * in_expert_stride + (int64_t)r * Cn + c;
    if (r < R && c + 8 <= Cn && off % (IN_F32 ? 4 : 8) == 0) {
      if (IN_F32) {
        const f32x4_t a = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(in) + off);
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(in) + off + 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = f32_to_bf16(a[q]);
          v[4 + q] = f32_to_bf16(b[q]);
        }
      } else {
        const i32x4_t a = *reinterpret_cast<const i32x4_t*>(static_cast<const uint16_t*>(in) + off);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[2 * q] = (uint16_t)((uint32_t)a[q] & 0xffffu);
          v[2 * q + 1] = (uint16_t)((uint32_t)a[q] >> 16);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int cq = c + q;
        float f = 0.0f;
        if (r < R && cq < Cn) {
          const int64_t off = (int64_t)e * in_expert_stride + (int64_t)r * Cn + cq;
          f = IN_F32 ? static_cast<const float*>(in)[off] : bf16_to_f32(static_cast<const uint16_t*>(in)[off]);
        }
        v[q] = f32_to_bf16(f);
      }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) tile[cc + q][rr] = v[q];
  }
  __syncthreads();
  // store: thread -> (output row for input col c0 + tid/8 + 32 i, 8 elements r0 + 8 (tid%8))
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int cc = tid / 8 + 32 * i, rr = 8 * (tid % 8);
    const int c = c0 + cc, r = r0 + rr;
    if (c >= Cn || r >= R) continue;
    const int64_t orow = gate_up ? (int64_t)(c / 128) * 256 + half * 128 + (c % 128) : (int64_t)c;
    uint16_t* dst = out + ((int64_t)e * out_rows + orow) * out_ld + r;
    if (r + 8 <= R) {
      i32x4_t w;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[q] = (int)((uint32_t)tile[cc][rr + 2 * q] | ((uint32_t)tile[cc][rr + 2 * q + 1] << 16));
      *reinterpret_cast<i32x4_t*>(dst) = w;
    } else {
      for (int q = 0; r + q < R; ++q) dst[q] = tile[cc][rr + q];
    }
  }
}

// Zeroes what pack_t16_kernel leaves: in every packed row the elements [valid_cols,
// out_ld), and the whole rows that no input column maps to.  One thread per row; the
// pad of a row that holds data starts at an 8-byte boundary (valid_cols % 4 == 0) or
// is first finished element by element.
__global__ __launch_bounds__(256) void pack_pad_kernel(uint16_t* __restrict__ out, int64_t n_rows, int out_ld,
                                                       int valid_cols, int rows_per_expert, int valid_in_cols,
                                                       bool gate_up) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= n_rows) return;
  const int pr = (int)(row % rows_per_expert);
  // the input column this packed row holds (gate_up: w1 / w2 column f of block f/128)
  const int c = gate_up ? (pr / 256) * 128 + (pr % 128) : pr;
  uint16_t* p = out + row * out_ld;
  int from = c >= valid_in_cols ? 0 : valid_cols;
  for (; (from & 3) != 0 && from < out_ld; ++from) p[from] = 0;
  uint64_t* w = reinterpret_cast<uint64_t*>(p);
  for (int i = from / 4; i < out_ld / 4; ++i) w[i] = 0ull;
}

// Backward packed layouts (rows K-contiguous, WPAD bytes after every row, zero padded):
//   mode ROWS_W3N : (E, round_up(F, 256), d)        row f = w3[e][f][:]      (dh = dY . w3^T, K = d)
//   mode ROWS_W13T: (E, round_up(d, 256), 2*F_pad)  row i = w1[e][i][:], w2[e][i][:] interleaved per 128
//                                                    columns like w13's rows  (dX = [dg|du] . w13, K = 2*F_pad)
//   mode ROWS_W1N : (E, round_up(d, 256), F_pad)    row i = w1[e][i][:]      (non-gated experts: dX = dp . w1^T)
// All are row copies with the columns rearranged (no transpose), 16 bytes per access;
// rows past F (w3n) or d (w13t, w1n) and the pads are written as zeros.
enum { ROWS_W3N = 0, ROWS_W13T = 1, ROWS_W1N = 2 };
template <bool IN_F32>
__global__ __launch_bounds__(256) void pack_rows16_kernel(const void* __restrict__ w1, const void* __restrict__ w2,
                                                          const void* __restrict__ w3, int d, int F, int mode,
                                                          uint16_t* __restrict__ out, int64_t out_rows, int out_ld,
                                                          int E) {
  const int nv = out_ld / 8;  // 16-byte vectors per packed row
  const int64_t n = (int64_t)E * out_rows * nv;
  const int Fp = round_up(F, 128);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t grow = i / nv;
    const int v = (int)(i - grow * nv);
    const int e = (int)(grow / out_rows);
    const int64_t row = grow - (int64_t)e * out_rows;
    const int c = 8 * v;  // first packed column of the vector
    const void* src = nullptr;
    int64_t off = 0;
    int n_ok = 0;  // source elements that exist (the rest are zero)
    if (mode == ROWS_W13T) {
      if (row < d && c < 2 * Fp) {
        const int half = (c >> 7) & 1, f = (c >> 8) * 128 + (c & 127);
        src = half ? w2 : w1;
        off = ((int64_t)e * d + row) * F + f;
        n_ok = F - f < 8 ? (F - f > 0 ? F - f : 0) : 8;
      }
    } else if (mode == ROWS_W1N) {
      if (row < d && c < Fp) {
        src = w1;
        off = ((int64_t)e * d + row) * F + c;
        n_ok = F - c < 8 ? (F - c > 0 ? F - c : 0) : 8;
      }
    } else if (row < F && c < d) {
      src = w3;
      off = ((int64_t)e * F + row) * d + c;
      n_ok = d - c < 8 ? d - c : 8;
    }
    i32x4_t wv = {0, 0, 0, 0};
    if (n_ok == 8 && (off % (IN_F32 ? 4 : 8)) == 0) {
      if (IN_F32) {
        const float* p = static_cast<const float*>(src) + off;
        const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p);
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          wv[q] = (int)((uint32_t)f32_to_bf16(a[2 * q]) | ((uint32_t)f32_to_bf16(a[2 * q + 1]) << 16));
          wv[2 + q] = (int)((uint32_t)f32_to_bf16(b[2 * q]) | ((uint32_t)f32_to_bf16(b[2 * q + 1]) << 16));
        }
      } else {
        wv = *reinterpret_cast<const i32x4_t*>(static_cast<const uint16_t*>(src) + off);
      }
    } else {
      uint16_t t[8];
#pragma unroll
      for (int q = 0; q < 8; ++q)
        t[q] = q < n_ok ? (IN_F32 ? f32_to_bf16(static_cast<const float*>(src)[off + q])
                                  : static_cast<const uint16_t*>(src)[off + q])
                        : (uint16_t)0;
#pragma unroll
      for (int q = 0; q < 4; ++q) wv[q] = (int)((uint32_t)t[2 * q] | ((uint32_t)t[2 * q + 1] << 16));
    }
    *reinterpret_cast<i32x4_t*>(out + grow * out_ld + c) = wv;
  }
}

// Per-row fp8 quantisation of a bf16 matrix: each wave takes rows w, w + W, ... (W waves
// in the grid) and loads its next row into a second register set before it reduces and
// stores the current one, so a wave's reads and writes overlap (one row per wave, all
// resident at once, read every row first and wrote them all after).  NV: 16-byte vectors
// per lane of a row (the register sets are sized for the row, not for the largest one).
// PREFETCH = false (rows of more than 8 vectors per lane, where two register sets leave one
// wave per SIMD): one row per wave, no second set.
template <int NV, bool PREFETCH = true>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ in, int64_t rows,
                                                         const int32_t* __restrict__ n_rows_dev, int cols,
                                                         uint8_t* __restrict__ out, float* __restrict__ scale) {
  struct Regs {
    i32x4_t v[NV];
  };
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int64_t nr = rows;
  if (n_rows_dev) nr = min<int64_t>(nr, (int64_t)*n_rows_dev);
  const int nvec = cols / 8;  // <= 64 * NV (chosen on the host)
  auto load = [&](int64_t row, Regs& rr) {
    const i32x4_t* src = reinterpret_cast<const i32x4_t*>(in + row * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) rr.v[i] = src[v];
    }
  };
  auto finish = [&](int64_t row, const Regs& rr) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (lane + 64 * i < nvec) {
#pragma unroll
        for (int q = 0; q < 4; ++q) amax = fmaxf(amax, bf16_pair_absmax((uint32_t)rr.v[i][q]));
      }
    amax = wave_max(amax);
    const float inv = amax > 0.0f ? 448.0f / amax : 0.0f;
    uint32_t* dst = reinterpret_cast<uint32_t*>(out + row * cols);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int v = lane + 64 * i;
      if (v < nvec) {
        uint32_t lo, hi;
        quant_vec_e4m3(rr.v[i], inv, lo, hi);
        *reinterpret_cast<uint2*>(dst + 2 * v) = make_uint2(lo, hi);
      }
    }
    if (lane == 0) scale[row] = amax / 448.0f;
  };
  Regs a;
  if constexpr (!PREFETCH) {
    if (r < nr) {
      load(r, a);
      finish(r, a);
    }
    return;
  }
  Regs b;
  if (r < nr) load(r, a);
  while (r < nr) {
    if (r + nw < nr) load(r + nw, b);
    finish(r, a);
    r += nw;
    if (r >= nr) break;
    if (r + nw < nr) load(r + nw, a);
    finish(r, b);
    r += nw;
  }
}

int elem_bytes(int dtype) { return dtype == KMOE_DTYPE_FP8_E4M3 ? 1 : 2; }

// A rows: the permuted rows (row_token == nullptr) or gathered rows of the
// activation matrix A (n_a_rows rows) through row_token / row_index.
int launch_gemm(bool gate_up, bool fp8, const void* A, const float* a_scale, const int32_t* row_token,
                const int32_t* row_index, int64_t n_a_rows, const int32_t* offsets, int E, int K, int64_t max_rows,
                const void* B, int64_t b_expert_rows, const float* b_scale, void* C, int64_t ldc, int n_valid,
                int n_tiles, hipStream_t s, void* C2 = nullptr, void* gu_out = nullptr) {
  const int eb = fp8 ? 1 : 2;
  const int64_t slots = kmoe::ceil_div<int64_t>(max_rows, BM) + E;
  // every tile of the worst-case slot count, plus one narrow tile per resident
  // workgroup for the split tail
  const int n_cu = kmoe::cu_count();
  const int64_t blocks = slots * n_tiles + n_cu;
  if (blocks > 0x7fffffff) {
    kmoe::set_error("kmoe gemm: grid too large");
    return KMOE_ERR_SHAPE;
  }
  const int kbytes = K * eb;
  if (kbytes % KB != 0) {
    kmoe::set_error("kmoe gemm: K bytes %d not a multiple of %d", kbytes, KB);
    return KMOE_ERR_SHAPE;
  }
  GemmArgs g{};  // value-initialised: every optional output (C2, gu_out, Cf) starts null
  g.A = static_cast<const uint8_t*>(A);
  g.lda_bytes = kbytes;
  g.a_scale = a_scale;
  g.row_token = row_token;
  g.row_index = row_index;
  g.B = static_cast<const uint8_t*>(B);
  g.b_expert_rows = b_expert_rows;
  g.ldb_bytes = kbytes + WPAD;
  g.b_scale = b_scale;
  g.k_bytes = kbytes;
  g.C = static_cast<uint16_t*>(C);
  g.ldc = ldc;
  g.n_valid = n_valid;
  g.C2 = static_cast<uint16_t*>(C2);
  g.gu_out = static_cast<uint16_t*>(gu_out);
  g.Cf = nullptr;
  // tile loads address a 2 GiB buffer window from the tile's first A / B row (from
  // the first row of A when gathering)
  if ((int64_t)(BM + 1) * g.ldb_bytes >= ((int64_t)1 << 31) ||
      (row_token && (n_a_rows + 1) * g.lda_bytes >= ((int64_t)1 << 31))) {
    kmoe::set_error("kmoe gemm: operand too large for 32-bit tile offsets (K bytes %d)", kbytes);
    return KMOE_ERR_SHAPE;
  }
  const dim3 grid((unsigned)blocks);
  const dim3 block(GEMM_THREADS);
  const int allow_split = 1;
#define KMOE_LAUNCH_GEMM(GU, F8, GA)                                                                         \
  hipLaunchKernelGGL((grouped_gemm_kernel<GU, F8, GA>), grid, block, 0, s, g, offsets, E, n_tiles, n_cu, \
                     allow_split)
  if (row_token && gu_out)
    hipLaunchKernelGGL((grouped_gemm_kernel<true, false, true, true>), grid, block, 0, s, g, offsets, E, n_tiles,
                       n_cu, allow_split);
  else if (row_token && a_scale)
    hipLaunchKernelGGL((grouped_gemm_kernel<true, false, true, false, true>), grid, block, 0, s, g, offsets, E,
                       n_tiles, n_cu, allow_split);
  else if (row_token)
    KMOE_LAUNCH_GEMM(true, false, true);
  else if (gate_up && !fp8)
    KMOE_LAUNCH_GEMM(true, false, false);
  else if (gate_up && gu_out)
    hipLaunchKernelGGL((grouped_gemm_kernel<true, true, false, true>), grid, block, 0, s, g, offsets, E, n_tiles,
                       n_cu, allow_split);
  else if (gate_up && fp8)
    KMOE_LAUNCH_GEMM(true, true, false);
  else if (!fp8)
    KMOE_LAUNCH_GEMM(false, false, false);
  else
    KMOE_LAUNCH_GEMM(false, true, false);
#undef KMOE_LAUNCH_GEMM
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
  const bool f32 = w_dtype == KMOE_DTYPE_F32;
  if (!fp8) {
    // bf16: vectorised transposes, then zeros in the pads and padding rows only
    const int ld13 = d + WPAD / 2, ld3 = Fp + WPAD / 2;
    uint16_t* o13 = static_cast<uint16_t*>(w13_packed);
    uint16_t* o3 = static_cast<uint16_t*>(w3_packed);
    const dim3 g13((unsigned)kmoe::ceil_div(F, 64), (unsigned)kmoe::ceil_div(d, 64), (unsigned)E);
    const dim3 g3((unsigned)kmoe::ceil_div(d, 64), (unsigned)kmoe::ceil_div(F, 64), (unsigned)E);
#define KMOE_PACK16(F32_)                                                                                         \
  do {                                                                                                            \
    hipLaunchKernelGGL(pack_t16_kernel<F32_>, g13, dim3(256), 0, s, w1, d, F, (int64_t)d * F, 0, true, o13, rows13, \
                       ld13);                                                                                     \
    hipLaunchKernelGGL(pack_t16_kernel<F32_>, g13, dim3(256), 0, s, w2, d, F, (int64_t)d * F, 1, true, o13, rows13, \
                       ld13);                                                                                     \
    hipLaunchKernelGGL(pack_t16_kernel<F32_>, g3, dim3(256), 0, s, w3, F, d, (int64_t)d * F, 0, false, o3, rows3,  \
                       ld3);                                                                                      \
  } while (0)
    if (f32)
      KMOE_PACK16(true);
    else
      KMOE_PACK16(false);
#undef KMOE_PACK16
    hipLaunchKernelGGL(pack_pad_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(E * rows13, 256)), dim3(256), 0, s, o13,
                       (int64_t)E * rows13, ld13, d, (int)rows13, F, true);
    hipLaunchKernelGGL(pack_pad_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(E * rows3, 256)), dim3(256), 0, s, o3,
                       (int64_t)E * rows3, ld3, F, (int)rows3, d, false);
    return kmoe::check_launch("kmoe_pack_weights");
  }
  // fp8: zero the padding (whole buffers: simple; the fp8 pack runs once per weight version)
  hipLaunchKernelGGL(zero_kernel, dim3(1024), dim3(256), 0, s, static_cast<uint8_t*>(w13_packed),
                     (int64_t)kmoe_packed_w13_bytes(E, d, F, packed_dtype));
  hipLaunchKernelGGL(zero_kernel, dim3(1024), dim3(256), 0, s, static_cast<uint8_t*>(w3_packed),
                     (int64_t)kmoe_packed_w3_bytes(E, d, F, packed_dtype));
  if (fp8) {
    hipLaunchKernelGGL(zero_f32_kernel, dim3(64), dim3(256), 0, s, w13_scale, (int64_t)E * rows13);
    hipLaunchKernelGGL(zero_f32_kernel, dim3(64), dim3(256), 0, s, w3_scale, (int64_t)E * rows3);
    const dim3 g13((unsigned)kmoe::ceil_div(F, 256), (unsigned)kmoe::ceil_div(d, COLS_ROWS), (unsigned)E);
    const dim3 g3((unsigned)kmoe::ceil_div(d, 256), (unsigned)kmoe::ceil_div(F, COLS_ROWS), (unsigned)E);
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
  rc = launch_gemm(true, fp8, xperm, xperm_scale, nullptr, nullptr, 0, offsets, E, d, max_rows, w13_packed,
                   2 * (int64_t)Fp, w13_scale, h, Fp, Fp, Fp / 128, kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_gate_up");
}

extern "C" int kmoe_gemm_gate_up_rows(const void* x, const int32_t* row_index, int64_t n_x_rows,
                                      const int32_t* row_token, const int32_t* offsets, int E, int d, int F,
                                      int64_t max_rows, const void* w13_packed, void* h, void* stream) {
  int rc = check_gemm_args("kmoe_gemm_gate_up_rows", x, offsets, E, d, F, max_rows, w13_packed, h, KMOE_DTYPE_BF16);
  if (rc) return rc;
  KMOE_REQUIRE(row_token, KMOE_ERR_NULL, "kmoe_gemm_gate_up_rows: null row_token");
  KMOE_REQUIRE(n_x_rows >= 1, KMOE_ERR_SHAPE, "kmoe_gemm_gate_up_rows: n_x_rows=%lld must be >= 1",
               (long long)n_x_rows);
  if (max_rows == 0) return KMOE_OK;
  const int Fp = round_up(F, 128);
  rc = launch_gemm(true, false, x, nullptr, row_token, row_index, n_x_rows, offsets, E, d, max_rows, w13_packed,
                   2 * (int64_t)Fp, nullptr, h, Fp, Fp, Fp / 128, kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_gate_up_rows");
}

extern "C" int kmoe_gemm_gate_up_rows_scaled(const void* x, const int32_t* row_index, int64_t n_x_rows,
                                             const int32_t* row_token, const int32_t* offsets, int E, int d, int F,
                                             int64_t max_rows, const void* w13_packed, const float* rscale, void* h,
                                             void* stream) {
  int rc = check_gemm_args("kmoe_gemm_gate_up_rows_scaled", x, offsets, E, d, F, max_rows, w13_packed, h,
                           KMOE_DTYPE_BF16);
  if (rc) return rc;
  KMOE_REQUIRE(row_token && rscale, KMOE_ERR_NULL, "kmoe_gemm_gate_up_rows_scaled: null row_token / rscale");
  KMOE_REQUIRE(n_x_rows >= 1, KMOE_ERR_SHAPE, "kmoe_gemm_gate_up_rows_scaled: n_x_rows=%lld must be >= 1",
               (long long)n_x_rows);
  if (max_rows == 0) return KMOE_OK;
  const int Fp = round_up(F, 128);
  rc = launch_gemm(true, false, x, rscale, row_token, row_index, n_x_rows, offsets, E, d, max_rows, w13_packed,
                   2 * (int64_t)Fp, nullptr, h, Fp, Fp, Fp / 128, kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_gate_up_rows_scaled");
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
  rc = launch_gemm(false, fp8, h, h_scale, nullptr, nullptr, 0, offsets, E, Fp, max_rows, w3_packed, dp, w3_scale, y,
                   d, d, dp / BN, kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_down");
}

extern "C" int kmoe_quant_rows_fp8(const void* in, int64_t rows, const int32_t* n_rows_dev, int cols, uint8_t* out,
                                   float* scale, void* stream) {
  KMOE_REQUIRE(in && out && scale, KMOE_ERR_NULL, "kmoe_quant_rows_fp8: null buffer");
  KMOE_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, KMOE_ERR_SHAPE, "kmoe_quant_rows_fp8: bad shape");
  KMOE_REQUIRE(cols <= 64 * 8 * ROW_REGS, KMOE_ERR_UNSUPPORTED, "kmoe_quant_rows_fp8: cols=%d > %d", cols,
               64 * 8 * ROW_REGS);
  if (rows == 0) return KMOE_OK;
  // up to 8 vectors per lane: as many workgroups per CU as are resident at once (the
  // kernel's register use for NV = 2, 4, 8: 7, 4, 3 waves per SIMD), each wave looping
  // over its rows; wider rows: one row per wave
  const int nv = kmoe::ceil_div(cols / 8, 64);
  const int per_cu = nv <= 2 ? 6 : nv <= 4 ? 4 : 3;
  const int64_t all_rows = kmoe::ceil_div<int64_t>(rows, 4);  // one row per wave
  const int64_t blocks = nv <= 8 ? std::min<int64_t>(all_rows, (int64_t)kmoe::cu_count() * per_cu) : all_rows;
  hipStream_t s = kmoe::as_stream(stream);
  const uint16_t* ip = static_cast<const uint16_t*>(in);
  if (nv <= 2)
    hipLaunchKernelGGL(quant_rows_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, ip, rows, n_rows_dev, cols, out, scale);
  else if (nv <= 4)
    hipLaunchKernelGGL(quant_rows_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, ip, rows, n_rows_dev, cols, out, scale);
  else if (nv <= 8)
    hipLaunchKernelGGL(quant_rows_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, s, ip, rows, n_rows_dev, cols, out, scale);
  else
    hipLaunchKernelGGL((quant_rows_kernel<ROW_REGS, false>), dim3((unsigned)blocks), dim3(256), 0, s, ip, rows,
                       n_rows_dev, cols, out, scale);
  return kmoe::check_launch("kmoe_quant_rows_fp8");
}

extern "C" int kmoe_grouped_swiglu(const void* xperm, const int32_t* offsets, int E, int d, int F, int64_t max_rows,
                                   const void* w13_packed, const void* w3_packed, void* h, void* y, void* stream) {
  int rc = kmoe_gemm_gate_up(xperm, nullptr, KMOE_DTYPE_BF16, offsets, E, d, F, max_rows, w13_packed, nullptr, h,
                             stream);
  if (rc) return rc;
  return kmoe_gemm_down(h, nullptr, KMOE_DTYPE_BF16, offsets, E, d, F, max_rows, w3_packed, nullptr, y, stream);
}

// ---------------------------------------------------------------- backward pass

extern "C" int kmoe_gemm_gate_up_rows_gu(const void* x, const int32_t* row_index, int64_t n_x_rows,
                                         const int32_t* row_token, const int32_t* offsets, int E, int d, int F,
                                         int64_t max_rows, const void* w13_packed, void* h, void* gu, void* stream) {
  int rc = check_gemm_args("kmoe_gemm_gate_up_rows_gu", x, offsets, E, d, F, max_rows, w13_packed, h,
                           KMOE_DTYPE_BF16);
  if (rc) return rc;
  KMOE_REQUIRE(row_token && gu, KMOE_ERR_NULL, "kmoe_gemm_gate_up_rows_gu: null row_token / gu");
  KMOE_REQUIRE(n_x_rows >= 1, KMOE_ERR_SHAPE, "kmoe_gemm_gate_up_rows_gu: n_x_rows=%lld must be >= 1",
               (long long)n_x_rows);
  if (max_rows == 0) return KMOE_OK;
  const int Fp = round_up(F, 128);
  rc = launch_gemm(true, false, x, nullptr, row_token, row_index, n_x_rows, offsets, E, d, max_rows, w13_packed,
                   2 * (int64_t)Fp, nullptr, h, Fp, Fp, Fp / 128, kmoe::as_stream(stream), nullptr, gu);
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_gate_up_rows_gu");
}

extern "C" int kmoe_gemm_gate_up_fp8_gu(const void* xperm, const float* xperm_scale, const int32_t* offsets, int E,
                                        int d, int F, int64_t max_rows, const void* w13_packed, const float* w13_scale,
                                        void* h, void* gu, void* stream) {
  int rc = check_gemm_args("kmoe_gemm_gate_up_fp8_gu", xperm, offsets, E, d, F, max_rows, w13_packed, h,
                           KMOE_DTYPE_FP8_E4M3);
  if (rc) return rc;
  KMOE_REQUIRE(xperm_scale && w13_scale && gu, KMOE_ERR_NULL, "kmoe_gemm_gate_up_fp8_gu: null scale / gu");
  KMOE_REQUIRE(d % 128 == 0, KMOE_ERR_SHAPE, "kmoe_gemm_gate_up_fp8_gu: fp8 needs d %% 128 == 0 (d=%d)", d);
  if (max_rows == 0) return KMOE_OK;
  const int Fp = round_up(F, 128);
  rc = launch_gemm(true, true, xperm, xperm_scale, nullptr, nullptr, 0, offsets, E, d, max_rows, w13_packed,
                   2 * (int64_t)Fp, w13_scale, h, Fp, Fp, Fp / 128, kmoe::as_stream(stream), nullptr, gu);
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_gate_up_fp8_gu");
}

extern "C" size_t kmoe_packed_w3n_bytes(int E, int d, int F) {
  return (size_t)E * (size_t)round_up(F, 256) * ((size_t)d * 2 + WPAD);
}

extern "C" size_t kmoe_packed_w13t_bytes(int E, int d, int F) {
  return (size_t)E * (size_t)round_up(d, 256) * ((size_t)2 * round_up(F, 128) * 2 + WPAD);
}

extern "C" int kmoe_pack_weights_bwd(const void* w1, const void* w2, const void* w3, int w_dtype, int E, int d, int F,
                                     void* w3n_packed, void* w13t_packed, void* stream) {
  KMOE_REQUIRE(w1 && w2 && w3 && w3n_packed && w13t_packed, KMOE_ERR_NULL, "kmoe_pack_weights_bwd: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_pack_weights_bwd: E=%d out of range", E);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "kmoe_pack_weights_bwd: d=%d must be a positive multiple of 64", d);
  KMOE_REQUIRE(F > 0, KMOE_ERR_SHAPE, "kmoe_pack_weights_bwd: F=%d must be > 0", F);
  KMOE_REQUIRE(w_dtype == KMOE_DTYPE_BF16 || w_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "kmoe_pack_weights_bwd: weight dtype must be bf16 or f32");
  hipStream_t s = kmoe::as_stream(stream);
  const bool f32 = w_dtype == KMOE_DTYPE_F32;
  const int Fp = round_up(F, 128);
  const int64_t r3 = round_up(F, 256), r13 = round_up(d, 256);
  const int ld3 = d + WPAD / 2, ld13 = 2 * Fp + WPAD / 2;
  if (f32) {
    hipLaunchKernelGGL(pack_rows16_kernel<true>, dim3(4096), dim3(256), 0, s, w1, w2, w3, d, F, (int)ROWS_W3N,
                       static_cast<uint16_t*>(w3n_packed), r3, ld3, E);
    hipLaunchKernelGGL(pack_rows16_kernel<true>, dim3(4096), dim3(256), 0, s, w1, w2, w3, d, F, (int)ROWS_W13T,
                       static_cast<uint16_t*>(w13t_packed), r13, ld13, E);
  } else {
    hipLaunchKernelGGL(pack_rows16_kernel<false>, dim3(4096), dim3(256), 0, s, w1, w2, w3, d, F, (int)ROWS_W3N,
                       static_cast<uint16_t*>(w3n_packed), r3, ld3, E);
    hipLaunchKernelGGL(pack_rows16_kernel<false>, dim3(4096), dim3(256), 0, s, w1, w2, w3, d, F, (int)ROWS_W13T,
                       static_cast<uint16_t*>(w13t_packed), r13, ld13, E);
  }
  return kmoe::check_launch("kmoe_pack_weights_bwd");
}

// ---- non-gated experts (silu(x . w1) . w2, moe.py:187-191,281-283): w1 (E, d, F), w2 (E, F, d)
extern "C" size_t kmoe_packed_w1t_bytes(int E, int d, int F) {
  return (size_t)E * (size_t)round_up(F, 256) * ((size_t)d * 2 + WPAD);
}

extern "C" size_t kmoe_packed_w1n_bytes(int E, int d, int F) {
  return (size_t)E * (size_t)round_up(d, 256) * ((size_t)round_up(F, 128) * 2 + WPAD);
}

static int check_plain_pack(const char* who, const void* w1, const void* w2, const void* o1, const void* o2,
                            int w_dtype, int E, int d, int F) {
  KMOE_REQUIRE(w1 && w2 && o1 && o2, KMOE_ERR_NULL, "%s: null buffer", who);
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "%s: E=%d out of range", who, E);
  KMOE_REQUIRE(d > 0 && d % 64 == 0, KMOE_ERR_SHAPE, "%s: d=%d must be a positive multiple of 64", who, d);
  KMOE_REQUIRE(F > 0, KMOE_ERR_SHAPE, "%s: F=%d must be > 0", who, F);
  KMOE_REQUIRE(w_dtype == KMOE_DTYPE_BF16 || w_dtype == KMOE_DTYPE_F32, KMOE_ERR_DTYPE,
               "%s: weight dtype must be bf16 or f32", who);
  return KMOE_OK;
}

extern "C" int kmoe_pack_weights_plain(const void* w1, const void* w2, int w_dtype, int E, int d, int F,
                                       void* w1t_packed, void* w2t_packed, void* stream) {
  const int rc = check_plain_pack("kmoe_pack_weights_plain", w1, w2, w1t_packed, w2t_packed, w_dtype, E, d, F);
  if (rc) return rc;
  hipStream_t s = kmoe::as_stream(stream);
  const int Fp = round_up(F, 128);
  const int64_t r1 = round_up(F, 256), r2 = round_up(d, 256);
  const int ld1 = d + WPAD / 2, ld2 = Fp + WPAD / 2;
  uint16_t* o1 = static_cast<uint16_t*>(w1t_packed);
  uint16_t* o2 = static_cast<uint16_t*>(w2t_packed);
  // w1t: row f = w1[e][:, f] (K = d); w2t: row n = w2[e][:, n] (K = F_pad), the down pack's layout
  const dim3 g1((unsigned)kmoe::ceil_div(F, 64), (unsigned)kmoe::ceil_div(d, 64), (unsigned)E);
  const dim3 g2((unsigned)kmoe::ceil_div(d, 64), (unsigned)kmoe::ceil_div(F, 64), (unsigned)E);
  if (w_dtype == KMOE_DTYPE_F32) {
    hipLaunchKernelGGL(pack_t16_kernel<true>, g1, dim3(256), 0, s, w1, d, F, (int64_t)d * F, 0, false, o1, r1, ld1);
    hipLaunchKernelGGL(pack_t16_kernel<true>, g2, dim3(256), 0, s, w2, F, d, (int64_t)d * F, 0, false, o2, r2, ld2);
  } else {
    hipLaunchKernelGGL(pack_t16_kernel<false>, g1, dim3(256), 0, s, w1, d, F, (int64_t)d * F, 0, false, o1, r1, ld1);
    hipLaunchKernelGGL(pack_t16_kernel<false>, g2, dim3(256), 0, s, w2, F, d, (int64_t)d * F, 0, false, o2, r2, ld2);
  }
  hipLaunchKernelGGL(pack_pad_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(E * r1, 256)), dim3(256), 0, s, o1,
                     (int64_t)E * r1, ld1, d, (int)r1, F, false);
  hipLaunchKernelGGL(pack_pad_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>(E * r2, 256)), dim3(256), 0, s, o2,
                     (int64_t)E * r2, ld2, F, (int)r2, d, false);
  return kmoe::check_launch("kmoe_pack_weights_plain");
}

extern "C" int kmoe_pack_weights_plain_bwd(const void* w1, const void* w2, int w_dtype, int E, int d, int F,
                                           void* w2n_packed, void* w1n_packed, void* stream) {
  const int rc = check_plain_pack("kmoe_pack_weights_plain_bwd", w1, w2, w2n_packed, w1n_packed, w_dtype, E, d, F);
  if (rc) return rc;
  hipStream_t s = kmoe::as_stream(stream);
  const int Fp = round_up(F, 128);
  const int64_t r2 = round_up(F, 256), r1 = round_up(d, 256);
  const int ld2 = d + WPAD / 2, ld1 = Fp + WPAD / 2;
  // w2n: row f = w2[e][f][:] (dh = dY . w2^T, K = d), the w3n layout of w2; w1n: row i = w1[e][i][:] (K = F_pad)
  if (w_dtype == KMOE_DTYPE_F32) {
    hipLaunchKernelGGL(pack_rows16_kernel<true>, dim3(4096), dim3(256), 0, s, w1, nullptr, w2, d, F, (int)ROWS_W3N,
                       static_cast<uint16_t*>(w2n_packed), r2, ld2, E);
    hipLaunchKernelGGL(pack_rows16_kernel<true>, dim3(4096), dim3(256), 0, s, w1, nullptr, w2, d, F, (int)ROWS_W1N,
                       static_cast<uint16_t*>(w1n_packed), r1, ld1, E);
  } else {
    hipLaunchKernelGGL(pack_rows16_kernel<false>, dim3(4096), dim3(256), 0, s, w1, nullptr, w2, d, F, (int)ROWS_W3N,
                       static_cast<uint16_t*>(w2n_packed), r2, ld2, E);
    hipLaunchKernelGGL(pack_rows16_kernel<false>, dim3(4096), dim3(256), 0, s, w1, nullptr, w2, d, F, (int)ROWS_W1N,
                       static_cast<uint16_t*>(w1n_packed), r1, ld1, E);
  }
  return kmoe::check_launch("kmoe_pack_weights_plain_bwd");
}

extern "C" int kmoe_gemm_grouped(const void* a, const int32_t* offsets, int E, int K, int64_t max_rows,
                                 const void* b_packed, int64_t b_expert_rows, int N, void* c, int64_t ldc, int n_valid,
                                 void* stream) {
  KMOE_REQUIRE(a && offsets && b_packed && c, KMOE_ERR_NULL, "kmoe_gemm_grouped: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_gemm_grouped: E=%d out of range", E);
  KMOE_REQUIRE(K > 0 && K % 64 == 0, KMOE_ERR_SHAPE, "kmoe_gemm_grouped: K=%d must be a positive multiple of 64", K);
  KMOE_REQUIRE(N > 0 && b_expert_rows >= round_up(N, BN) && b_expert_rows % BN == 0, KMOE_ERR_SHAPE,
               "kmoe_gemm_grouped: b_expert_rows=%lld must be a multiple of %d covering N=%d",
               (long long)b_expert_rows, BN, N);
  KMOE_REQUIRE(n_valid > 0 && n_valid <= ldc, KMOE_ERR_SHAPE, "kmoe_gemm_grouped: n_valid=%d, ldc=%lld", n_valid,
               (long long)ldc);
  KMOE_REQUIRE(max_rows >= 0 && max_rows < ((int64_t)1 << 31), KMOE_ERR_SHAPE, "kmoe_gemm_grouped: max_rows");
  if (max_rows == 0) return KMOE_OK;
  const int rc = launch_gemm(false, false, a, nullptr, nullptr, nullptr, 0, offsets, E, K, max_rows, b_packed,
                             b_expert_rows, nullptr, c, ldc, n_valid, (int)(round_up(N, BN) / BN),
                             kmoe::as_stream(stream));
  if (rc) return rc;
  return kmoe::check_launch("kmoe_gemm_grouped");
}

extern "C" int kmoe_gemm_wgrad_rows(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t max_rows,
                                    const int32_t* offsets, int E, int M, int N, void* c, void* c2, int c_dtype,
                                    int64_t ldc, int n_valid, void* stream) {
  KMOE_REQUIRE(a && b && offsets && c, KMOE_ERR_NULL, "kmoe_gemm_wgrad_rows: null buffer");
  KMOE_REQUIRE(E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_gemm_wgrad_rows: E=%d out of range", E);
  KMOE_REQUIRE(M > 0 && N > 0 && N % BN == 0, KMOE_ERR_SHAPE, "kmoe_gemm_wgrad_rows: M=%d, N=%d (N a multiple of %d)",
               M, N, BN);
  KMOE_REQUIRE(lda >= M && ldb >= 1 && lda % 8 == 0 && ldb % 8 == 0, KMOE_ERR_SHAPE,
               "kmoe_gemm_wgrad_rows: lda=%lld, ldb=%lld (multiples of 8, lda >= M)", (long long)lda, (long long)ldb);
  KMOE_REQUIRE(c_dtype == KMOE_DTYPE_BF16 || (c_dtype == KMOE_DTYPE_F32 && c2 == nullptr), KMOE_ERR_DTYPE,
               "kmoe_gemm_wgrad_rows: c dtype must be bf16, or f32 without c2");
  KMOE_REQUIRE(n_valid > 0 && n_valid <= ldc && n_valid % 8 == 0 && ldc % 8 == 0, KMOE_ERR_SHAPE,
               "kmoe_gemm_wgrad_rows: n_valid=%d, ldc=%lld (multiples of 8, n_valid <= ldc)", n_valid, (long long)ldc);
  // an expert's row window (at most max_rows + one K-step of rows) must fit the
  // buffer's 31-bit record count and the 32-bit per-lane offsets
  KMOE_REQUIRE(max_rows >= 0 && (max_rows + TN_KR) * (lda > ldb ? lda : ldb) * 2 < ((int64_t)1 << 31),
               KMOE_ERR_SHAPE, "kmoe_gemm_wgrad_rows: %lld rows too large for 32-bit buffer offsets",
               (long long)max_rows);

  GemmArgs g{};
  g.A = static_cast<const uint8_t*>(a);
  g.lda_bytes = lda * 2;
  g.B = static_cast<const uint8_t*>(b);
  g.ldb_bytes = ldb * 2;
  const bool f32 = c_dtype == KMOE_DTYPE_F32;
  g.C = f32 ? nullptr : static_cast<uint16_t*>(c);
  g.C2 = static_cast<uint16_t*>(c2);
  g.Cf = f32 ? static_cast<float*>(c) : nullptr;
  g.ldc = ldc;
  g.n_valid = n_valid;
  const int n_mt = kmoe::ceil_div(M, BM), n_nt = N / BN;
  const dim3 grid((unsigned)((int64_t)E * n_mt * n_nt)), block(GEMM_THREADS);
  hipStream_t s = kmoe::as_stream(stream);
  const int64_t stride = (int64_t)M * ldc;
  if (f32)
    hipLaunchKernelGGL(wgrad_rows_kernel<OUT_F32>, grid, block, 0, s, g, offsets, E, M, n_mt, n_nt, stride);
  else if (c2)
    hipLaunchKernelGGL(wgrad_rows_kernel<OUT_SPLIT>, grid, block, 0, s, g, offsets, E, M, n_mt, n_nt, stride);
  else
    hipLaunchKernelGGL(wgrad_rows_kernel<OUT_BF16>, grid, block, 0, s, g, offsets, E, M, n_mt, n_nt, stride);
  return kmoe::check_launch("kmoe_gemm_wgrad_rows");
}
