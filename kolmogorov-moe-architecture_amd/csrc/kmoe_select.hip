// Per-sequence top-C selection for expert-choice routing and Mixture-of-Depths.
//   kmoe_ec_select   follows ExpertChoiceRouter.forward (moe_arch/model/moe.py:494-530)
//   kmoe_mod_select  follows MoDRouter.forward (moe_arch/model/mod.py:67-122) plus the
//                    gather/scatter index bookkeeping of TransformerBlock.forward
//                    (moe_arch/model/layers.py:148-185)
//
// Selection is an exact radix select over order-preserving uint32 images of the
// fp32 scores (passes of 12, 10 and 10 bits, LDS histograms), followed by an index-ordered
// compaction: every score above the threshold is taken, and of the scores equal
// to it the lowest indices are taken first.  One 1024-thread workgroup per
// (sequence, expert); keys live in LDS.
#include "kmoe_common.h"

namespace {

constexpr int SEL_THREADS = 1024;
constexpr int SEL_MAX_S = 16384;  // keys held in LDS
constexpr int SEL_MAX_C = 8192;   // sort buffer for the expert-choice order

// Order-preserving uint32 image of a float: a > b  <=>  key(a) > key(b), and
// a == b  <=>  key(a) == key(b); -0.0 and +0.0 compare equal, so they get one key
// (they then tie, and the lower index wins, as for any equal scores).
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0u;  // NaN ranks last
  const uint32_t u = f == 0.0f ? 0u : __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {  // inverse of order_key (non-NaN keys)
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ float block_sum(float v, float* s_red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float t = 0.0f;
  for (int w = 0; w < nw; ++w) t += s_red[w];
  __syncthreads();
  return t;
}

// Finds the key `thr` of the C-th largest element and how many elements equal to
// thr must be taken (`need`): an MSD radix select over digits of 12, 10 and 10 bits
// with one shared histogram (s_hist: RS_BINS bins).  The 12-bit first digit (sign,
// exponent and three mantissa bits of the score) spreads typical logits over many
// bins; with an 8-bit first digit (sign and 7 exponent bits) every score in [0.5, 2)
// shares one bin, and the histogram's LDS atomics from one wave to one address
// serialise (measured: 9k cycles per pass).  The keys are in registers (key_index;
// slots at or past n are ignored).  When the chosen bin holds a single key, that key
// is the threshold and the remaining passes are skipped.
constexpr int RS_BINS = 4096;
// Register layout of the keys: lane l of wave w holds key w * 64 PER + 64 u + l in
// slot u, so each wave owns one contiguous segment of 64 PER keys.
template <int PER>
__device__ __forceinline__ int key_index(int u) {
  return (int)(threadIdx.x >> 6) * (64 * PER) + 64 * u + (int)(threadIdx.x & 63);
}
template <int PER>
__device__ void radix_select_desc(const uint32_t (&kr)[PER], int n, int C, uint32_t* s_hist, uint32_t* s_bcast,
                                  uint32_t& thr, int& need) {
  __shared__ __attribute__((aligned(16))) int s_scan[SEL_THREADS / 64];
  uint32_t prefix = 0, pmask = 0;
  int remaining = C;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int nthr = blockDim.x;
  for (int pass = 0; pass < 3; ++pass) {
    const int shift = pass == 0 ? 20 : pass == 1 ? 10 : 0;
    const int nb = pass == 0 ? RS_BINS : 1024;
    for (int i = t; i < nb; i += nthr) s_hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if (key_index<PER>(u) < n && (kr[u] & pmask) == prefix)
        atomicAdd(&s_hist[(kr[u] >> shift) & (uint32_t)(nb - 1)], 1u);
    __syncthreads();
    // bucket choice: thread t owns `per` consecutive digits counted from the top
    // (digit nb - 1 - (t per + j)); an inclusive scan of the threads' sums gives the
    // count at or above each range, and the one thread whose range crosses
    // `remaining` walks its digits and publishes the digit, what is left of
    // `remaining` inside it and the digit's count
    const int per = nb > nthr ? nb / nthr : 1;  // 4 or 1
    int h[RS_BINS / SEL_THREADS];
    int tsum = 0;
#pragma unroll
    for (int j = 0; j < RS_BINS / SEL_THREADS; ++j) {
      const int r = t * per + j;
      h[j] = (j < per && r < nb) ? (int)s_hist[nb - 1 - r] : 0;
      tsum += h[j];
    }
    int incl = tsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64);
      if (lane >= o) incl += u;
    }
    if (lane == 63) s_scan[w] = incl;
    __syncthreads();
    // the sums of the waves before this one: the wave totals read as four vectors
#pragma unroll
    for (int q4 = 0; q4 < SEL_THREADS / 256; ++q4) {
      const i32x4_t v = reinterpret_cast<const i32x4_t*>(s_scan)[q4];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (4 * q4 + c < w) incl += v[c];
    }
    int c = incl - tsum;  // count above this thread's range
    if (c < remaining && incl >= remaining) {
#pragma unroll
      for (int j = 0; j < RS_BINS / SEL_THREADS; ++j) {
        if (j < per && c + h[j] >= remaining) {
          s_bcast[0] = (uint32_t)(nb - 1 - (t * per + j));
          s_bcast[1] = (uint32_t)(remaining - c);
          s_bcast[2] = (uint32_t)h[j];
          break;
        }
        c += h[j];
      }
    }
    __syncthreads();
    prefix |= s_bcast[0] << shift;
    pmask |= (uint32_t)(nb - 1) << shift;
    remaining = (int)s_bcast[1];
    const bool single = s_bcast[2] == 1u && pass < 2;
    __syncthreads();
    if (single) {
      // the bin's one key (remaining is 1): its owner publishes it
#pragma unroll
      for (int u = 0; u < PER; ++u)
        if (key_index<PER>(u) < n && (kr[u] & pmask) == prefix) s_bcast[3] = kr[u];
      __syncthreads();
      prefix = s_bcast[3];
      __syncthreads();
      break;
    }
  }
  thr = prefix;
  need = remaining;
}

// Index-ordered compaction of the selection from the register keys (key_index: each
// wave owns a contiguous segment and reads it 64 consecutive keys per slot); calls
// emit(i, pos, key) for each selected index i with its position pos in index order,
// skip(i) for the others.  Each wave counts its keys above and equal to thr; one
// exchange gives every wave its first position and its first rank among the equal
// keys (of which the lowest `need` indices are taken); positions inside a wave come
// from ballots.
template <int PER, typename Emit, typename Skip>
__device__ void compact_selected(const uint32_t (&kr)[PER], int n, uint32_t thr, int need, int* s_wave, Emit emit,
                                 Skip skip) {
  __shared__ int s_gt[SEL_THREADS / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto mbcnt = [&](uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  };
  int gt_w = 0, eq_w = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const bool v = key_index<PER>(u) < n;
    gt_w += (int)__builtin_popcountll(__ballot(v && kr[u] > thr));
    eq_w += (int)__builtin_popcountll(__ballot(v && kr[u] == thr));
  }
  if (lane == 0) {
    s_wave[wave] = eq_w;
    s_gt[wave] = gt_w;
  }
  __syncthreads();
  int eqr = 0, pos = 0;
  for (int q = 0; q < wave; ++q) {
    const int eqq = s_wave[q];
    pos += s_gt[q] + min(eqq, max(0, need - eqr));
    eqr += eqq;
  }
  __syncthreads();  // callers reuse s_wave
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = key_index<PER>(u);
    const bool v = i < n;
    const uint32_t k = kr[u];
    const bool eq = v && k == thr;
    const uint64_t em = __ballot(eq);
    const bool take = (v && k > thr) || (eq && eqr + mbcnt(em) < need);
    const uint64_t tm = __ballot(take);
    if (take)
      emit(i, pos + mbcnt(tm), k);
    else if (v)
      skip(i);
    eqr += (int)__builtin_popcountll(em);
    pos += (int)__builtin_popcountll(tm);
  }
}

// Expert-choice preparation: the logits (B*S, E) transposed to lt (B, E, S), so each
// selection block reads its (sequence, expert) column as contiguous floats (a column
// read with a stride of E floats touches a cache line per two tokens), and the combine
// table src_row (B*S, E) filled with -1 in the same coalesced pass (the selection then
// writes only its C rows per block).  A block moves 64 tokens x E through LDS.
__global__ __launch_bounds__(256) void ec_prep_kernel(const float* __restrict__ logits, int B, int S, int E,
                                                      float* __restrict__ lt, int32_t* __restrict__ src_row) {
  __shared__ float tile[64][KMOE_MAX_EXPERTS + 1];
  const int64_t T = (int64_t)B * S;
  const int64_t t0 = (int64_t)blockIdx.x * 64;
  const int64_t nt = min<int64_t>(64, T - t0);
  const int64_t n = nt * E;  // the block's logits are contiguous
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    tile[i / E][i % E] = logits[t0 * E + i];
    src_row[t0 * E + i] = -1;
  }
  __syncthreads();
  const int tl = threadIdx.x & 63;
  if (tl < nt) {
    const int64_t t = t0 + tl;
    const int64_t b = t / S, s = t - b * S;
    for (int e = threadIdx.x >> 6; e < E; e += 4) lt[(b * E + e) * S + s] = tile[tl][e];
  }
}

// PER: keys per thread held in registers (S <= PER * SEL_THREADS)
template <int PER>
__global__ __launch_bounds__(SEL_THREADS) void ec_select_kernel(const float* __restrict__ logits, int B, int S, int E,
                                                                int C, int order, int64_t* __restrict__ idx,
                                                                float* __restrict__ w,
                                                                int32_t* __restrict__ row_token,
                                                                int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ src_row,
                                                                float* __restrict__ src_w) {
  __shared__ uint64_t sorted[SEL_MAX_C];
  __shared__ uint32_t hist[RS_BINS];
  __shared__ uint32_t bc[4];
  __shared__ int s_wave[SEL_THREADS / 64];
  __shared__ float s_red[SEL_THREADS / 64];
  const int b = blockIdx.x / E, e = blockIdx.x % E;
  const float* lg = logits + ((int64_t)b * E + e) * S;  // the transposed logits (ec_prep_kernel)

  // the sequence's column of logits: all of a thread's loads in flight at once
  float v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = key_index<PER>(u);
    v[u] = i < S ? lg[i] : 0.0f;
  }
  float mx = -INFINITY;
  uint32_t kr[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    kr[u] = order_key(v[u]);
    if (key_index<PER>(u) < S) mx = fmaxf(mx, v[u]);
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = s_red[0];
  for (int q = 1; q < SEL_THREADS / 64; ++q) mx = fmaxf(mx, s_red[q]);
  __syncthreads();
  // softmax denominator over the whole sequence (moe.py:520)
  float den = 0.0f;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (key_index<PER>(u) < S) den += __expf(v[u] - mx);
  den = block_sum(den, s_red);

  uint32_t thr;
  int need;
  radix_select_desc(kr, S, C, hist, bc, thr, need);

  int Cp = 1;
  while (Cp < C) Cp <<= 1;
  for (int i = threadIdx.x; i < Cp; i += blockDim.x) sorted[i] = 0ull;
  __syncthreads();
  // selected: into the sort buffer in token order (the combine table's -1 entries of
  // the others were written by ec_prep_kernel; the selected ones get their rows with
  // the weights below)
  compact_selected(
      kr, S, thr, need, s_wave,
      [&](int i, int pos, uint32_t k) {
        if (pos < C) sorted[pos] = ((uint64_t)k << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
      },
      [&](int) {});
  __syncthreads();
  // sum of the selected probabilities, over the selection in token order (the same
  // sum whichever output order is asked for)
  float psel = 0.0f;
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    psel += __expf(key_value((uint32_t)(sorted[c] >> 32)) - mx) / den;
  }
  psel = block_sum(psel, s_red);
  if (order == 1) {
  // bitonic sort, descending by (key, -index).  Element i lives in thread i % 1024,
  // register slot i / 1024 (Cp <= 8192: up to 8 per thread): strides < 64 are
  // exchanged with wave shuffles, strides >= 1024 inside the thread, and only the
  // strides 64..512 go through LDS.
  {
    constexpr int MAXPER = SEL_MAX_C / SEL_THREADS;
    const int t = threadIdx.x;
    const int per = Cp > SEL_THREADS ? Cp / SEL_THREADS : 1;
    uint64_t v[MAXPER];
#pragma unroll
    for (int h = 0; h < MAXPER; ++h) v[h] = (h < per) ? sorted[t + h * SEL_THREADS] : 0ull;
    __syncthreads();
    // element i of the pair (i, partner) keeps the larger value in a descending block
    // when it is the lower index, else the smaller
    auto pick = [](uint64_t x, uint64_t y, int i, int partner, int kk) -> uint64_t {
      const bool keep_max = (((i & kk) == 0) == (i < partner));
      return keep_max ? (x > y ? x : y) : (x < y ? x : y);
    };
    for (int kk = 2; kk <= Cp; kk <<= 1) {
      for (int jj = kk >> 1; jj > 0; jj >>= 1) {
        if (jj >= SEL_THREADS) {  // partner in the same thread, slot h ^ (jj / 1024)
          const int hs = jj / SEL_THREADS;
          uint64_t nv[MAXPER];
#pragma unroll
          for (int h = 0; h < MAXPER; ++h) {
            const int i = t + h * SEL_THREADS;
            nv[h] = h < per ? pick(v[h], v[h ^ hs], i, i ^ jj, kk) : v[h];
          }
#pragma unroll
          for (int h = 0; h < MAXPER; ++h) v[h] = nv[h];
        } else if (jj < 64) {
#pragma unroll
          for (int h = 0; h < MAXPER; ++h) {
            if (h >= per) continue;
            const int i = t + h * SEL_THREADS;
            const uint32_t lo = (uint32_t)v[h], hi = (uint32_t)(v[h] >> 32);
            const uint64_t y = ((uint64_t)(uint32_t)__shfl_xor((int)hi, jj, 64) << 32) |
                               (uint64_t)(uint32_t)__shfl_xor((int)lo, jj, 64);
            v[h] = pick(v[h], y, i, i ^ jj, kk);
          }
        } else {
#pragma unroll
          for (int h = 0; h < MAXPER; ++h)
            if (h < per) sorted[t + h * SEL_THREADS] = v[h];
          __syncthreads();
#pragma unroll
          for (int h = 0; h < MAXPER; ++h) {
            if (h >= per) continue;
            const int i = t + h * SEL_THREADS;
            v[h] = pick(v[h], sorted[i ^ jj], i, i ^ jj, kk);
          }
          __syncthreads();
        }
      }
    }
#pragma unroll
    for (int h = 0; h < MAXPER; ++h)
      if (h < per) sorted[t + h * SEL_THREADS] = v[h];
    __syncthreads();
  }
  }
  // weights: p / (sum_sel p + 1e-9)  (moe.py:528)
  const float inv = 1.0f / (psel + 1e-9f);
  const int64_t BC = (int64_t)B * C;
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    const int s = (int)(0xffffffffu - (uint32_t)(sorted[c] & 0xffffffffu));
    const float p = __expf(key_value((uint32_t)(sorted[c] >> 32)) - mx) / den;
    const float wv = p * inv;
    const int64_t o = ((int64_t)b * E + e) * C + c;
    idx[o] = s;
    w[o] = wv;
    const int64_t row = (int64_t)e * BC + (int64_t)b * C + c;
    const int64_t tok = (int64_t)b * S + s;
    row_token[row] = (int32_t)tok;
    src_row[tok * E + e] = (int32_t)row;
    src_w[tok * E + e] = wv;
  }
  if (b == 0 && threadIdx.x == 0) {
    offsets[e] = (int32_t)(e * BC);
    if (e == E - 1) offsets[E] = (int32_t)(E * BC);
  }
}

// r[t] = x[t,:] . w_mod: each wave takes tokens w, w + n_waves, ... two at a time, the
// loads of both rows in flight together (one token per wave in T/4 small workgroups
// left the 32 MiB read of config 5 at 3.6 TB/s).  The per-token sum order is fixed: lane
// partial sums over its vectors in order, then the wave reduction.
__global__ __launch_bounds__(256) void mod_logits_kernel(const uint16_t* __restrict__ x, int64_t T, int d,
                                                         const uint16_t* __restrict__ wm, float* __restrict__ r) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  const i32x4_t* wv = reinterpret_cast<const i32x4_t*>(wm);
  const int nvec = d / 8;
  auto dot8 = [](const i32x4_t& a, const i32x4_t& c, float acc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc = fmaf(__uint_as_float(((uint32_t)a[q]) << 16), __uint_as_float(((uint32_t)c[q]) << 16), acc);
      acc = fmaf(__uint_as_float(((uint32_t)a[q]) & 0xffff0000u), __uint_as_float(((uint32_t)c[q]) & 0xffff0000u), acc);
    }
    return acc;
  };
  for (int64_t t0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t0 < T; t0 += 2 * nw) {
    const int64_t t1 = t0 + nw;
    const bool has1 = t1 < T;
    const i32x4_t* x0 = reinterpret_cast<const i32x4_t*>(x + t0 * d);
    const i32x4_t* x1 = reinterpret_cast<const i32x4_t*>(x + (has1 ? t1 : t0) * d);
    float a0 = 0.0f, a1 = 0.0f;
    for (int v0 = 0; v0 < nvec; v0 += 64 * 4) {
      i32x4_t r0[4], r1[4], w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = v0 + lane + 64 * i;
        if (v < nvec) {
          r0[i] = x0[v];
          r1[i] = x1[v];
          w[i] = wv[v];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (v0 + lane + 64 * i < nvec) {
          a0 = dot8(r0[i], w[i], a0);
          a1 = dot8(r1[i], w[i], a1);
        }
    }
    a0 = wave_sum(a0);
    a1 = wave_sum(a1);
    if (lane == 0) {
      r[t0] = a0;
      if (has1) r[t1] = a1;
    }
  }
}

template <int PER>
__global__ __launch_bounds__(SEL_THREADS) void mod_select_kernel(const float* __restrict__ r, int S, int keep,
                                                                 int64_t* __restrict__ sel_idx,
                                                                 float* __restrict__ sel_w,
                                                                 int32_t* __restrict__ token_rows,
                                                                 int32_t* __restrict__ out_map) {
  __shared__ float s_p[SEL_MAX_S];  // exp(r - max) of the kept tokens, by output position
  __shared__ uint32_t hist[RS_BINS];
  __shared__ uint32_t bc[4];
  __shared__ int s_wave[SEL_THREADS / 64];
  __shared__ float s_red[SEL_THREADS / 64];
  __shared__ uint32_t s_kmax;
  const int b = blockIdx.x;
  const float* rb = r + (int64_t)b * S;
  if (threadIdx.x == 0) s_kmax = 0u;
  __syncthreads();
  uint32_t kr[PER];
  uint32_t kmax = 0u;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = key_index<PER>(u);
    kr[u] = i < S ? order_key(rb[i]) : 0u;
    kmax = kr[u] > kmax ? kr[u] : kmax;
  }
  // the largest key (its value is the max over the sequence: fmaxf's result on
  // non-NaN scores; all NaN: key 0, max -inf)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t q = (uint32_t)__shfl_xor((int)kmax, o, 64);
    kmax = q > kmax ? q : kmax;
  }
  if ((threadIdx.x & 63) == 0) atomicMax(&s_kmax, kmax);
  __syncthreads();
  const float mx = s_kmax == 0u ? -INFINITY : key_value(s_kmax);
  uint32_t thr;
  int need;
  radix_select_desc(kr, S, keep, hist, bc, thr, need);
  // positions + softmax denominator over the kept tokens (mod.py:112); a key's value
  // is its score (-0.0 reads as +0.0: the same exp)
  float den = 0.0f;
  compact_selected(kr, S, thr, need, s_wave, [&](int i, int pos, uint32_t k) {
    if (pos >= keep) return;
    const int64_t o = (int64_t)b * keep + pos;
    sel_idx[o] = i;
    token_rows[o] = (int32_t)((int64_t)b * S + i);
    out_map[(int64_t)b * S + i] = (int32_t)o;
    const float e = __expf(key_value(k) - mx);
    s_p[pos] = e;
    den += e;
  }, [&](int i) { out_map[(int64_t)b * S + i] = -1; });
  den = block_sum(den, s_red);
  const float inv = 1.0f / den;
  for (int p = threadIdx.x; p < keep; p += blockDim.x) sel_w[(int64_t)b * keep + p] = s_p[p] * inv;
}

}  // namespace

extern "C" size_t kmoe_ec_workspace_bytes(int B, int64_t S, int E) {
  return B > 0 && S > 0 && E > 0 ? (size_t)B * (size_t)S * (size_t)E * sizeof(float) : 0;
}

extern "C" int kmoe_ec_select(const float* logits, int B, int64_t S, int E, int64_t C, int order, int64_t* idx,
                              float* w, int32_t* row_token, int32_t* offsets, int32_t* src_row, float* src_w,
                              void* workspace, size_t workspace_bytes, void* stream) {
  KMOE_REQUIRE(logits && idx && w && row_token && offsets && src_row && src_w, KMOE_ERR_NULL,
               "kmoe_ec_select: null buffer");
  KMOE_REQUIRE(B >= 1 && E >= 1 && E <= KMOE_MAX_EXPERTS, KMOE_ERR_SHAPE, "kmoe_ec_select: bad B=%d/E=%d", B, E);
  KMOE_REQUIRE(S >= 1 && S <= SEL_MAX_S, KMOE_ERR_UNSUPPORTED, "kmoe_ec_select: S=%lld not in [1,%d]", (long long)S,
               SEL_MAX_S);
  KMOE_REQUIRE(C >= 1 && C <= S && C <= SEL_MAX_C, KMOE_ERR_SHAPE, "kmoe_ec_select: C=%lld not in [1,min(S,%d)]",
               (long long)C, SEL_MAX_C);
  KMOE_REQUIRE((int64_t)E * B * C < ((int64_t)1 << 31), KMOE_ERR_SHAPE, "kmoe_ec_select: E*B*C must fit in int32");
  KMOE_REQUIRE(order == 0 || order == 1, KMOE_ERR_SHAPE, "kmoe_ec_select: order=%d not 0 or 1", order);
  const size_t need_ws = kmoe_ec_workspace_bytes(B, S, E);
  KMOE_REQUIRE(workspace && workspace_bytes >= need_ws, KMOE_ERR_WORKSPACE,
               "kmoe_ec_select: workspace of %zu bytes needed (kmoe_ec_workspace_bytes)", need_ws);
  hipStream_t s = kmoe::as_stream(stream);
  float* lt = static_cast<float*>(workspace);
  hipLaunchKernelGGL(ec_prep_kernel, dim3((unsigned)kmoe::ceil_div<int64_t>((int64_t)B * S, 64)), dim3(256), 0, s,
                     logits, B, (int)S, E, lt, src_row);
#define KMOE_EC_SELECT(P_)                                                                                      \
  hipLaunchKernelGGL(ec_select_kernel<P_>, dim3((unsigned)(B * E)), dim3(SEL_THREADS), 0, s, lt, B, (int)S, E, (int)C, \
                     order, idx, w, row_token, offsets, src_row, src_w)
  if (S <= SEL_THREADS)
    KMOE_EC_SELECT(1);
  else if (S <= 2 * SEL_THREADS)
    KMOE_EC_SELECT(2);
  else if (S <= 4 * SEL_THREADS)
    KMOE_EC_SELECT(4);
  else if (S <= 8 * SEL_THREADS)
    KMOE_EC_SELECT(8);
  else
    KMOE_EC_SELECT(16);
#undef KMOE_EC_SELECT
  return kmoe::check_launch("kmoe_ec_select");
}

extern "C" size_t kmoe_mod_workspace_bytes(int B, int64_t S) { return (size_t)B * (size_t)S * sizeof(float); }

extern "C" int kmoe_mod_select(const void* x, int B, int64_t S, int d, const void* w_mod, int64_t keep, float* logits,
                               int64_t* sel_idx, float* sel_w, int32_t* token_rows, int32_t* out_map, void* workspace,
                               size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  KMOE_REQUIRE((!x || w_mod) && logits && sel_idx && sel_w && token_rows && out_map, KMOE_ERR_NULL,
               "kmoe_mod_select: null buffer");
  KMOE_REQUIRE(B >= 1, KMOE_ERR_SHAPE, "kmoe_mod_select: B=%d", B);
  KMOE_REQUIRE(S >= 1 && S <= SEL_MAX_S, KMOE_ERR_UNSUPPORTED, "kmoe_mod_select: S=%lld not in [1,%d]", (long long)S,
               SEL_MAX_S);
  KMOE_REQUIRE(keep >= 1 && keep <= S, KMOE_ERR_SHAPE, "kmoe_mod_select: keep=%lld not in [1,S]", (long long)keep);
  KMOE_REQUIRE(!x || (d > 0 && d % 8 == 0), KMOE_ERR_SHAPE, "kmoe_mod_select: d=%d must be a multiple of 8", d);
  hipStream_t s = kmoe::as_stream(stream);
  const int64_t T = (int64_t)B * S;
  if (x) {  // else the caller's logits are used as they are
    int64_t blocks = kmoe::ceil_div<int64_t>(T, 8);
    const int64_t cap = (int64_t)kmoe::cu_count() * 8;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(mod_logits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<const uint16_t*>(x), T,
                       d, static_cast<const uint16_t*>(w_mod), logits);
  }
#define KMOE_MOD_SELECT(P_)                                                                                      \
  hipLaunchKernelGGL(mod_select_kernel<P_>, dim3((unsigned)B), dim3(SEL_THREADS), 0, s, logits, (int)S, (int)keep, \
                     sel_idx, sel_w, token_rows, out_map)
  if (S <= SEL_THREADS)
    KMOE_MOD_SELECT(1);
  else if (S <= 2 * SEL_THREADS)
    KMOE_MOD_SELECT(2);
  else if (S <= 4 * SEL_THREADS)
    KMOE_MOD_SELECT(4);
  else if (S <= 8 * SEL_THREADS)
    KMOE_MOD_SELECT(8);
  else
    KMOE_MOD_SELECT(16);
#undef KMOE_MOD_SELECT
  return kmoe::check_launch("kmoe_mod_select");
}
