// Output head for gfx950:
//
//   amla_bf16_logits  <- hidden.float() @ lm_head_w.float().T, inference/forward.py:70-72
//   amla_argmax       <- sample(..., temperature=0), inference/engine.py:172-173
//   amla_sample_top_p <- sample(...) with temperature and nucleus filtering, engine.py:175-186
//   amla_sample       <- the whole of sample(), engine.py:166-186, rows cut into chunks
//
// The logits are exact bf16 products summed in fp32 by MFMA (no fp32 copy of
// the 129280 x 7168 matrix, which the reference makes every step).  Sampling
// finds the nucleus threshold by a radix search on the probability value and
// draws from the kept tokens by an inverse CDF with a counter-based
// generator: amla_argmax / amla_sample_top_p with one workgroup per row,
// amla_sample with rows x chunks workgroups and a workspace (same results).
#include <math.h>

#include <algorithm>

#include "amla_common.h"
#include "amla_internal.h"

namespace amla {

// logits[m, n] = sum_k f32(x[m, k]) * f32(w[n, k]).  A workgroup takes 16
// tokens and 64 rows of w (four tiles of 16); its four waves take interleaved
// 32-wide K steps, so one x fragment feeds four MFMAs (four accumulator
// chains), and add their partial tiles in wave order through LDS.
constexpr int LOGIT_ROWS = 64;
// Dynamic LDS the launch reserves (unused by the kernel) so that at most four
// workgroups (16 KB static + this) are resident per CU: the weight stream is
// fastest with that many loads in flight (measured at batch 8, 129280 x 7168:
// 498 us with the eight workgroups per CU the waves allow, 386 us with four,
// 546 with two, 523 with six).
constexpr int LOGIT_LDS_RESERVE = 24 * 1024;
__global__ __launch_bounds__(256) void bf16_logits_kernel(const uint16_t *__restrict__ x,
                                                          const uint16_t *__restrict__ w, int M, int K, int N,
                                                          float *__restrict__ out, int64_t ldo) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * LOGIT_ROWS, m0 = blockIdx.y * 16;
  const int r = lane & 15, kq = lane >> 4;
  const uint16_t *xp = x + (size_t)min(m0 + r, M - 1) * K + 8 * kq;
  const uint16_t *wp[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) wp[t] = w + (size_t)min(n0 + 16 * t + r, N - 1) * K + 8 * kq;
  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int steps = K / 32;
#pragma unroll 4
  for (int ks = wave; ks < steps; ks += 4) {
    const bf16x8 a = as_bf16x8(ldg16(xp + ks * 32));
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = mfma16(a, as_bf16x8(ldg16_nt(wp[t] + ks * 32)), acc[t]);
  }
  __shared__ f32x4 red[4][4][64];
#pragma unroll
  for (int t = 0; t < 4; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  // wave t sums tile t in wave order; C layout: tokens 4 (lane/16) .. +3 of row lane % 16
  const int t = wave;
  f32x4 v = red[0][t][lane];
#pragma unroll
  for (int q = 1; q < 4; ++q) v += red[q][t][lane];
  const int n = n0 + 16 * t + (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 4 * (lane >> 4) + i;
    if (m < M && n < N) out[(size_t)m * ldo + n] = v[i];
  }
}

constexpr int SAMPLE_THREADS = 1024;  // amla_argmax, amla_sample_top_p: one workgroup per row
constexpr int NS_THREADS = 256;       // amla_sample: one workgroup per row chunk
constexpr int NS_TARGET_WG = 512;     // chunk workgroups a launch aims for (two per CU)
constexpr int NS_ALIGN = 1024;        // chunk lengths are multiples of this
constexpr int NS_HIST = 3 * 2048;     // one row's three level histograms
constexpr int NS_MAX_CHUNKS = NS_TARGET_WG;

// (value, index) maximum with ties to the lower index
AMLA_DEV void argmax_merge(float &v, int &i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

template <int NT>
AMLA_DEV void block_argmax(float &v, int &i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_merge(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  __shared__ float sv[NT / 64];
  __shared__ int si[NT / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  for (int q = 1; q < NT / 64; ++q) argmax_merge(v, i, sv[q], si[q]);
  __syncthreads();
}

// Exclusive prefix over the threads of the block (thread order); `total` gets the sum.
template <int NT>
AMLA_DEV unsigned long long block_exscan_u64(unsigned long long v, unsigned long long &total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  __shared__ unsigned long long wsum[NT / 64];
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  unsigned long long before = 0, all = 0;
  for (int q = 0; q < NT / 64; ++q) {
    const unsigned long long s = wsum[q];
    if (q < wave) before += s;
    all += s;
  }
  __syncthreads();
  total = all;
  return before + inc - v;
}

// Index of the largest logit of each row (ties to the lower index).
__global__ __launch_bounds__(SAMPLE_THREADS) void argmax_kernel(const float *__restrict__ logits, int64_t n,
                                                                int64_t ld, int64_t *__restrict__ out) {
  const float *row = logits + (size_t)blockIdx.x * ld;
  float v = -INFINITY;
  int i = INT32_MAX;
  for (int64_t j = threadIdx.x; j < n; j += SAMPLE_THREADS) argmax_merge(v, i, row[j], (int)j);
  block_argmax<SAMPLE_THREADS>(v, i);
  if (threadIdx.x == 0) out[blockIdx.x] = i == INT32_MAX ? 0 : i;
}

// 64-bit counter-based generator (the SplitMix64 finaliser of seed + golden-ratio steps)
AMLA_DEV uint64_t splitmix64(uint64_t seed, uint64_t ctr) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (ctr + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Nucleus sampling, the reference's rule: p = softmax(logits / T); sorted
// descending, token k is dropped when the mass strictly before it exceeds
// top_p; the kept probabilities are renormalised and one is drawn.
// Everything works on e = exp(logits / T - max) (p = e / sum e; the
// normalisation cancels): with e1 > e2 > .. sorted and C_k their prefix sums,
// the reference keeps e_1 .. e_{K+1}, K the last k with C_k <= top_p * sum e:
// every token with e > t, t the smallest value whose strictly larger mass is
// <= top_p * sum e, and of the tokens equal to t those whose mass before them
// is still <= top_p * sum e.  The reference's sort leaves the order of equal
// values open; here it is the vocabulary order (a stable sort), so the j-th
// token equal to t (j from 0) is kept while above + j * e_t <= top_p * sum e.
// t is always the value of a token, found on the fp32 bit pattern (e >= 0:
// bit order = value order) by a three-level radix search: per level a
// histogram of the mass over the next 11 / 11 / 10 bits.  Masses are integers
// in 2^-40 fixed point, so every sum (histogram bins, kept mass, running mass
// of the draw) is independent of the order of the additions: the
// one-workgroup and the chunked kernels find the same t and draw the same
// token.  The draw takes u = floor(K * r / 2^64) (K the kept mass, r a 64-bit
// counter-based random number) and returns the first kept token in
// vocabulary order whose running kept mass exceeds u.
constexpr double NUCLEUS_FX = 1099511627776.0;  // 2^40

AMLA_DEV unsigned long long mass_fx(float e) { return (unsigned long long)((double)e * NUCLEUS_FX); }

AMLA_DEV int level_shift(int level) { return level == 0 ? 21 : (level == 1 ? 10 : 0); }

// top_p * sum e in the same fixed point, saturated (any top_p that large keeps every token)
AMLA_DEV unsigned long long top_mass_fx(float top_p, unsigned long long total) {
  const double t = (double)top_p * (double)total;
  return t >= 18446744073709549568.0 ? ~0ull : (unsigned long long)t;
}

// How many of the tokens equal to the threshold are kept (the first ones in
// vocabulary order): the j-th has mass above + j * ft before it.
AMLA_DEV unsigned long long ties_kept(unsigned long long top_fx, unsigned long long above, unsigned long long ft) {
  if (ft == 0) return ~0ull;
  const unsigned long long q = (top_fx - above) / ft;
  return q == ~0ull ? q : q + 1;
}

// One full wave, wave-uniform results: the smallest bin b of this level's
// histogram whose mass above it (the bins above b plus `above`, the mass above
// the prefix of the earlier levels) is <= top_p * total, and that mass.  At
// level 0 `total` is set to the sum of the histogram (the whole row).
AMLA_DEV int nucleus_select(const unsigned long long *hist, int level, float top_p, unsigned long long &total,
                            unsigned long long above, unsigned long long &mass_above) {
  const int lane = threadIdx.x & 63;
  const int nb = level == 2 ? 1024 : 2048, per = nb / 64;
  const int b_hi = nb - 1 - lane * per;  // this lane's bins: b_hi down to b_hi - per + 1
  unsigned long long own = 0;
  for (int q = 0; q < per; ++q) own += hist[b_hi - q];
  unsigned long long ex = own;  // inclusive prefix over lanes 0..lane (higher bins first)
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned long long v = __shfl_up(ex, o, 64);
    if (lane >= o) ex += v;
  }
  if (level == 0) total = __shfl(ex, 63, 64);
  const unsigned long long top_fx = top_mass_fx(top_p, total);
  ex -= own;
  unsigned long long run = above + ex;
  int found = -1;
  unsigned long long m = 0;
  for (int q = 0; q < per; ++q) {
    const int bb = b_hi - q;
    if (run > top_fx) break;
    found = bb;  // bins are visited downwards: keep the smallest
    m = run;
    run += hist[bb];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int ob = __shfl_xor(found, o, 64);
    const unsigned long long om = __shfl_xor(m, o, 64);
    if (ob >= 0 && (found < 0 || ob < found)) {
      found = ob;
      m = om;
    }
  }
  mass_above = m;
  return found;
}

// The draw over consecutive per-thread ranges [a0, a1) (thread order = vocabulary
// order): kept mass per thread (tokens above t, and ties of rank < tie_lim;
// tie_base = rank of the first tie of thread 0's range), then the thread whose
// range holds u walks it and sets *pick.  u = floor(K * rnd / 2^64) over the
// block's kept mass K when scale_by_total, else u_in (relative to the ranges).
template <int NT, typename EV>
AMLA_DEV void draw_ranges(EV ev, int64_t a0, int64_t a1, float tstar, unsigned long long ft,
                          unsigned long long tie_lim, unsigned long long tie_base, unsigned long long rnd,
                          bool scale_by_total, unsigned long long u_in, int *pick) {
  unsigned long long gt = 0, ties = 0;
  for (int64_t j = a0; j < a1; ++j) {
    const float e = ev(j);
    if (e > tstar)
      gt += mass_fx(e);
    else if (e == tstar)
      ++ties;
  }
  unsigned long long all_ties, kept;
  const unsigned long long tie_pre = tie_base + block_exscan_u64<NT>(ties, all_ties);
  const unsigned long long kt = tie_pre >= tie_lim ? 0 : std::min(ties, tie_lim - tie_pre);
  const unsigned long long mine = gt + kt * ft;
  const unsigned long long pre = block_exscan_u64<NT>(mine, kept);
  const unsigned long long u = scale_by_total ? __umul64hi(kept, rnd) : u_in;
  if (mine > 0 && u >= pre && u - pre < mine) {
    unsigned long long acc = pre, rank = tie_pre;
    for (int64_t j = a0; j < a1; ++j) {
      const float e = ev(j);
      unsigned long long w;
      if (e > tstar)
        w = mass_fx(e);
      else if (e == tstar && rank++ < tie_lim)
        w = ft;
      else
        continue;
      acc += w;
      if (u < acc) {
        *pick = (int)j;
        break;
      }
    }
  }
}

// One workgroup per row: the three histogram levels, then the draw.
__global__ __launch_bounds__(SAMPLE_THREADS) void top_p_kernel(const float *__restrict__ logits, int64_t n,
                                                               int64_t ld, float temp, float top_p, uint64_t seed,
                                                               int64_t *__restrict__ out) {
  const float *row = logits + (size_t)blockIdx.x * ld;
  const int tid = threadIdx.x;
  float mx = -INFINITY;
  int dummy = 0;
  for (int64_t j = tid; j < n; j += SAMPLE_THREADS) mx = fmaxf(mx, row[j] / temp);
  block_argmax<SAMPLE_THREADS>(mx, dummy);
  auto ev = [&](int64_t j) { return expf(row[j] / temp - mx); };
  __shared__ unsigned long long hist[2048];
  __shared__ unsigned long long above_s, total_s;
  __shared__ uint32_t prefix_s;
  __shared__ int pick;
  if (tid == 0) {
    above_s = 0;
    total_s = 0;
    prefix_s = 0;
    pick = -1;
  }
  for (int level = 0; level < 3; ++level) {
    const int shift = level_shift(level);
    const int nb = level == 2 ? 1024 : 2048;
    for (int i = tid; i < 2048; i += SAMPLE_THREADS) hist[i] = 0;
    __syncthreads();
    const uint32_t prefix = prefix_s;
    const int pshift = shift + (level == 2 ? 10 : 11);  // bits above this level's bins
    for (int64_t j = tid; j < n; j += SAMPLE_THREADS) {
      const float e = ev(j);
      const uint32_t key = __float_as_uint(e);
      if (level == 0 || (key >> pshift) == (prefix >> pshift)) atomicAdd(&hist[(key >> shift) & (nb - 1)], mass_fx(e));
    }
    __syncthreads();
    if (tid < 64) {
      unsigned long long total = total_s, mass_above;
      const int found = nucleus_select(hist, level, top_p, total, above_s, mass_above);
      if (tid == 0) {
        prefix_s = prefix | ((uint32_t)found << shift);
        above_s = mass_above;
        total_s = total;
      }
    }
    __syncthreads();
  }
  const float tstar = __uint_as_float(prefix_s);
  const unsigned long long ft = mass_fx(tstar);
  const unsigned long long tie_lim = ties_kept(top_mass_fx(top_p, total_s), above_s, ft);
  const int64_t chunk = (n + SAMPLE_THREADS - 1) / SAMPLE_THREADS;
  const int64_t c0 = std::min<int64_t>(n, tid * chunk), c1 = std::min<int64_t>(n, c0 + chunk);
  draw_ranges<SAMPLE_THREADS>(ev, c0, c1, tstar, ft, tie_lim, 0, splitmix64(seed, blockIdx.x), true, 0, &pick);
  __syncthreads();
  if (tid == 0) out[blockIdx.x] = pick < 0 ? 0 : pick;
}

// ------------------------------------------------ chunked sampling (amla_sample)
//
// A row of n logits is cut into `chunks` ranges of `chunk` (a multiple of
// NS_ALIGN) so that rows x chunks workgroups fill the chip; the chunk
// workgroups of a launch add their LDS histograms into the row's histogram in
// the workspace with integer atomics (order-independent).  Launches, in order
// (chunk kernels on grid rows * chunks, blockIdx.x = row * chunks + chunk):
//   ns_max_kernel        chunk maxima of logits / T; clears the row's histograms
//   ns_hist_kernel<0>    level-0 histogram
//   ns_hist_kernel<1>    level-0 selection (every workgroup of the row makes the
//                        same one from the same histogram), level-1 histogram
//   ns_hist_kernel<2>    level-1 selection, level-2 histogram
//   ns_kept_kernel       level-2 selection (the threshold t), kept mass per chunk
//   ns_draw_kernel       one workgroup per row: the chunk that holds u, then the token
// Temperature 0: ns_argmax_part_kernel (per chunk) and ns_argmax_final_kernel.

struct NucleusState {           // one row's search after a level (written by chunk 0)
  unsigned long long total;     // sum of e over the row (fixed point)
  unsigned long long above;     // mass of the values above the prefix
  uint32_t prefix;              // threshold bits found so far
  uint32_t pad[3];
};
static_assert(sizeof(NucleusState) == 32, "NucleusState layout");

struct ArgPart {
  float v;
  int i;
};

struct ChunkKept {              // one chunk after the search
  unsigned long long gt;        // mass of its tokens above t
  unsigned long long ties;      // its tokens equal to t
};

// Row maximum from the chunk maxima; every wave computes it by itself.
AMLA_DEV float chunks_max(const float *cm, int chunks) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY;
  for (int q = lane; q < chunks; q += 64) m = fmaxf(m, cm[q]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  return m;
}

__global__ __launch_bounds__(NS_THREADS) void ns_max_kernel(const float *__restrict__ logits, int64_t n, int64_t ld,
                                                            float temp, int64_t chunk, int chunks,
                                                            float *__restrict__ cmax,
                                                            unsigned long long *__restrict__ hist) {
  const int r = blockIdx.x / chunks, c = blockIdx.x % chunks;
  const float *row = logits + (size_t)r * ld;
  const int64_t j0 = (int64_t)c * chunk, j1 = std::min<int64_t>(n, j0 + chunk);
  float mx = -INFINITY;
  for (int64_t j = j0 + threadIdx.x; j < j1; j += NS_THREADS) mx = fmaxf(mx, row[j] / temp);
  int dummy = 0;
  block_argmax<NS_THREADS>(mx, dummy);
  if (threadIdx.x == 0) cmax[blockIdx.x] = mx;
  unsigned long long *h = hist + (size_t)r * NS_HIST;
  const int per = (NS_HIST + chunks - 1) / chunks;
  const int i1 = std::min(NS_HIST, (c + 1) * per);
  for (int i = c * per + threadIdx.x; i < i1; i += NS_THREADS) h[i] = 0;
}

template <int LEVEL>
__global__ __launch_bounds__(NS_THREADS) void ns_hist_kernel(const float *__restrict__ logits, int64_t n, int64_t ld,
                                                             float temp, float top_p, int64_t chunk, int chunks,
                                                             const float *__restrict__ cmax,
                                                             unsigned long long *__restrict__ hist,
                                                             NucleusState *__restrict__ state) {
  constexpr int SHIFT = LEVEL == 0 ? 21 : (LEVEL == 1 ? 10 : 0);
  constexpr int NB = LEVEL == 2 ? 1024 : 2048;
  constexpr int PSHIFT = SHIFT + (LEVEL == 2 ? 10 : 11);  // bits above this level's bins
  const int tid = threadIdx.x, r = blockIdx.x / chunks, c = blockIdx.x % chunks;
  const float *row = logits + (size_t)r * ld;
  const int64_t j0 = (int64_t)c * chunk, j1 = std::min<int64_t>(n, j0 + chunk);
  const float mx = chunks_max(cmax + (size_t)r * chunks, chunks);
  unsigned long long *hrow = hist + (size_t)r * NS_HIST;
  __shared__ unsigned long long h[2048];
  __shared__ uint32_t prefix_s;
  if constexpr (LEVEL > 0) {
    // the previous level's histogram (2048 bins) staged in LDS by coalesced loads
    for (int i = tid; i < 2048; i += NS_THREADS) h[i] = hrow[(LEVEL - 1) * 2048 + i];
    __syncthreads();
    if (tid < 64) {
      NucleusState s{};
      if constexpr (LEVEL == 2) s = state[(size_t)r * 3];
      unsigned long long mass_above;
      const int found = nucleus_select(h, LEVEL - 1, top_p, s.total, s.above, mass_above);
      s.prefix |= (uint32_t)found << level_shift(LEVEL - 1);
      s.above = mass_above;
      if (tid == 0) {
        prefix_s = s.prefix;
        if (c == 0) state[(size_t)r * 3 + LEVEL - 1] = s;
      }
    }
    __syncthreads();
  }
  for (int i = tid; i < NB; i += NS_THREADS) h[i] = 0;
  __syncthreads();
  uint32_t prefix = 0;
  if constexpr (LEVEL > 0) prefix = prefix_s;
  for (int64_t j = j0 + tid; j < j1; j += NS_THREADS) {
    const float e = expf(row[j] / temp - mx);
    const uint32_t key = __float_as_uint(e);
    bool match = true;
    if constexpr (LEVEL > 0) match = (key >> PSHIFT) == (prefix >> PSHIFT);
    if (match) atomicAdd(&h[(key >> SHIFT) & (NB - 1)], mass_fx(e));
  }
  __syncthreads();
  for (int i = tid; i < NB; i += NS_THREADS) {
    const unsigned long long v = h[i];
    if (v) atomicAdd(&hrow[LEVEL * 2048 + i], v);
  }
}

__global__ __launch_bounds__(NS_THREADS) void ns_kept_kernel(const float *__restrict__ logits, int64_t n, int64_t ld,
                                                             float temp, float top_p, int64_t chunk, int chunks,
                                                             const float *__restrict__ cmax,
                                                             const unsigned long long *__restrict__ hist,
                                                             NucleusState *__restrict__ state,
                                                             ChunkKept *__restrict__ kept) {
  const int tid = threadIdx.x, r = blockIdx.x / chunks, c = blockIdx.x % chunks;
  const float *row = logits + (size_t)r * ld;
  const int64_t j0 = (int64_t)c * chunk, j1 = std::min<int64_t>(n, j0 + chunk);
  const float mx = chunks_max(cmax + (size_t)r * chunks, chunks);
  __shared__ uint32_t tbits_s;
  __shared__ unsigned long long h[1024];
  for (int i = tid; i < 1024; i += NS_THREADS) h[i] = hist[(size_t)r * NS_HIST + 2 * 2048 + i];
  __syncthreads();
  if (tid < 64) {
    NucleusState s = state[(size_t)r * 3 + 1];
    unsigned long long mass_above;
    const int found = nucleus_select(h, 2, top_p, s.total, s.above, mass_above);
    s.prefix |= (uint32_t)found;
    s.above = mass_above;
    if (tid == 0) {
      tbits_s = s.prefix;
      if (c == 0) state[(size_t)r * 3 + 2] = s;
    }
  }
  __syncthreads();
  const float tstar = __uint_as_float(tbits_s);
  unsigned long long gt = 0, ties = 0;
  for (int64_t j = j0 + tid; j < j1; j += NS_THREADS) {
    const float e = expf(row[j] / temp - mx);
    if (e > tstar)
      gt += mass_fx(e);
    else if (e == tstar)
      ++ties;
  }
  unsigned long long gt_sum, tie_sum;
  block_exscan_u64<NS_THREADS>(gt, gt_sum);
  block_exscan_u64<NS_THREADS>(ties, tie_sum);
  if (tid == 0) kept[blockIdx.x] = ChunkKept{gt_sum, tie_sum};
}

__global__ __launch_bounds__(NS_THREADS) void ns_draw_kernel(const float *__restrict__ logits, int64_t n, int64_t ld,
                                                             float temp, float top_p, uint64_t seed, int64_t chunk,
                                                             int chunks, const float *__restrict__ cmax,
                                                             const NucleusState *__restrict__ state,
                                                             const ChunkKept *__restrict__ kept,
                                                             int64_t *__restrict__ out) {
  const int tid = threadIdx.x, lane = tid & 63, r = blockIdx.x;
  const float *row = logits + (size_t)r * ld;
  const float mx = chunks_max(cmax + (size_t)r * chunks, chunks);
  const NucleusState s = state[(size_t)r * 3 + 2];
  const float tstar = __uint_as_float(s.prefix);
  const unsigned long long ft = mass_fx(tstar);
  const unsigned long long tie_lim = ties_kept(top_mass_fx(top_p, s.total), s.above, ft);
  const ChunkKept *kr = kept + (size_t)r * chunks;
  __shared__ int chunk_s, pick;
  __shared__ unsigned long long u_s, tb_s;
  if (tid < 64) {
    // kept mass of 64 chunks from q0 on (the ties counted from tbase, advanced past them);
    // tie_before: rank of the chunk's first tie
    auto group = [&](int q0, unsigned long long &tbase, unsigned long long &tie_before) {
      const bool in = q0 + lane < chunks;
      const unsigned long long gt = in ? kr[q0 + lane].gt : 0, ties = in ? kr[q0 + lane].ties : 0;
      unsigned long long inc = ties;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
      }
      tie_before = tbase + inc - ties;
      tbase += __shfl(inc, 63, 64);
      const unsigned long long kt = tie_before >= tie_lim ? 0 : std::min(ties, tie_lim - tie_before);
      return gt + kt * ft;
    };
    unsigned long long total = 0, tb = 0, tbf;
    for (int q0 = 0; q0 < chunks; q0 += 64) {
      unsigned long long v = group(q0, tb, tbf);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
      total += v;
    }
    const unsigned long long u = __umul64hi(total, splitmix64(seed, r));
    // the first chunk whose running kept mass exceeds u
    unsigned long long base = 0, lo_found = 0, tb_found = 0;
    int cfound = -1;
    tb = 0;
    for (int q0 = 0; q0 < chunks && cfound < 0; q0 += 64) {
      const unsigned long long v = group(q0, tb, tbf);
      unsigned long long inc = v;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
      }
      const unsigned long long lo = base + inc - v;
      const unsigned long long hit = __ballot(v > 0 && u >= lo && u - lo < v);
      if (hit) {
        const int l = __builtin_ctzll(hit);
        cfound = q0 + l;
        lo_found = __shfl(lo, l, 64);
        tb_found = __shfl(tbf, l, 64);
      }
      base += __shfl(inc, 63, 64);
    }
    if (tid == 0) {
      chunk_s = cfound;
      u_s = u - lo_found;
      tb_s = tb_found;
      pick = -1;
    }
  }
  __syncthreads();
  const int cc = chunk_s;
  if (cc >= 0) {  // block-uniform
    const int64_t j0 = (int64_t)cc * chunk, j1 = std::min<int64_t>(n, j0 + chunk);
    const int64_t per = (j1 - j0 + NS_THREADS - 1) / NS_THREADS;
    const int64_t a0 = std::min<int64_t>(j1, j0 + tid * per), a1 = std::min<int64_t>(j1, a0 + per);
    auto ev = [&](int64_t j) { return expf(row[j] / temp - mx); };
    draw_ranges<NS_THREADS>(ev, a0, a1, tstar, ft, tie_lim, tb_s, 0, false, u_s, &pick);
  }
  __syncthreads();
  if (tid == 0) out[r] = pick < 0 ? 0 : pick;
}

__global__ __launch_bounds__(NS_THREADS) void ns_argmax_part_kernel(const float *__restrict__ logits, int64_t n,
                                                                    int64_t ld, int64_t chunk, int chunks,
                                                                    ArgPart *__restrict__ part) {
  const int r = blockIdx.x / chunks, c = blockIdx.x % chunks;
  const float *row = logits + (size_t)r * ld;
  const int64_t j0 = (int64_t)c * chunk, j1 = std::min<int64_t>(n, j0 + chunk);
  float v = -INFINITY;
  int i = INT32_MAX;
  for (int64_t j = j0 + threadIdx.x; j < j1; j += NS_THREADS) argmax_merge(v, i, row[j], (int)j);
  block_argmax<NS_THREADS>(v, i);
  if (threadIdx.x == 0) part[blockIdx.x] = ArgPart{v, i};
}

__global__ __launch_bounds__(64) void ns_argmax_final_kernel(const ArgPart *__restrict__ part, int chunks,
                                                             int64_t *__restrict__ out) {
  const ArgPart *p = part + (size_t)blockIdx.x * chunks;
  float v = -INFINITY;
  int i = INT32_MAX;
  for (int q = threadIdx.x; q < chunks; q += 64) argmax_merge(v, i, p[q].v, p[q].i);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_merge(v, i, __shfl_xor(v, o, 64), __shfl_xor(i, o, 64));
  if (threadIdx.x == 0) out[blockIdx.x] = i == INT32_MAX ? 0 : i;
}

struct SamplePlan {
  int64_t chunk;
  int chunks;
  size_t cmax, hist, state, kept, bytes;
};

// Chunks of a multiple of NS_ALIGN, about NS_TARGET_WG workgroups per launch
// (at most NS_MAX_CHUNKS per row); the workspace sections 256-byte aligned.
static SamplePlan sample_plan(int64_t rows, int64_t n) {
  SamplePlan p;
  const int64_t per_row = std::max<int64_t>(1, NS_TARGET_WG / rows);
  p.chunk = (int64_t)align_up((size_t)((n + per_row - 1) / per_row), NS_ALIGN);
  p.chunks = (int)((n + p.chunk - 1) / p.chunk);
  size_t off = 0;
  p.cmax = off;  // float maxima, or (value, index) pairs at temperature 0
  off = align_up(off + (size_t)rows * p.chunks * sizeof(ArgPart), 256);
  p.hist = off;
  off = align_up(off + (size_t)rows * NS_HIST * sizeof(unsigned long long), 256);
  p.state = off;
  off = align_up(off + (size_t)rows * 3 * sizeof(NucleusState), 256);
  p.kept = off;
  off = align_up(off + (size_t)rows * p.chunks * sizeof(ChunkKept), 256);
  p.bytes = off;
  return p;
}

}  // namespace amla

using namespace amla;

extern "C" {

int amla_bf16_logits(const void *x, int64_t m, int64_t k, const void *weight, int64_t n, float *logits,
                     int64_t ld_logits, void *stream) {
  if (!x || !weight || !logits) return fail(AMLA_EINVAL, "bf16_logits: null pointer");
  if (m < 0 || k <= 0 || n <= 0 || ld_logits < n) return fail(AMLA_EINVAL, "bf16_logits: bad sizes");
  if (m == 0) return AMLA_OK;
  if (k % 32 || !aligned16(x) || !aligned16(weight) || k > INT32_MAX || n > INT32_MAX || m > (int64_t)65535 * 16)
    return fail(AMLA_EUNSUPPORTED, "bf16_logits: needs k %% 32 == 0 and 16-byte aligned x and weight");
  bf16_logits_kernel<<<dim3((unsigned)((n + LOGIT_ROWS - 1) / LOGIT_ROWS), (unsigned)((m + 15) / 16)), 256, LOGIT_LDS_RESERVE,
                       reinterpret_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t *>(x),
                                                                static_cast<const uint16_t *>(weight), (int)m, (int)k,
                                                                (int)n, logits, ld_logits);
  return check_launch("bf16_logits");
}

int amla_argmax(const float *logits, int64_t rows, int64_t n, int64_t ld, int64_t *out, void *stream) {
  if (!logits || !out) return fail(AMLA_EINVAL, "argmax: null pointer");
  if (rows < 0 || n <= 0 || ld < n || n > INT32_MAX - 1) return fail(AMLA_EINVAL, "argmax: bad sizes");
  if (rows == 0) return AMLA_OK;
  argmax_kernel<<<dim3((unsigned)rows), SAMPLE_THREADS, 0, reinterpret_cast<hipStream_t>(stream)>>>(logits, n, ld,
                                                                                                    out);
  return check_launch("argmax");
}

int amla_sample_top_p(const float *logits, int64_t rows, int64_t n, int64_t ld, float temperature, float top_p,
                      uint64_t seed, int64_t *out, void *stream) {
  if (!logits || !out) return fail(AMLA_EINVAL, "sample_top_p: null pointer");
  if (rows < 0 || n <= 0 || ld < n || n > INT32_MAX - 1) return fail(AMLA_EINVAL, "sample_top_p: bad sizes");
  if (!(temperature > 0.f) || !(top_p >= 0.f)) return fail(AMLA_EINVAL, "sample_top_p: needs temperature > 0");
  if (rows == 0) return AMLA_OK;
  top_p_kernel<<<dim3((unsigned)rows), SAMPLE_THREADS, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      logits, n, ld, temperature, top_p, seed, out);
  return check_launch("sample_top_p");
}

size_t amla_sample_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0 || n > INT32_MAX - 1 || rows > INT32_MAX / NS_MAX_CHUNKS) return 0;
  return sample_plan(rows, n).bytes;
}

int amla_sample(const float *logits, int64_t rows, int64_t n, int64_t ld, float temperature, float top_p,
                uint64_t seed, int64_t *out, void *workspace, size_t workspace_bytes, void *stream) {
  if (!logits || !out) return fail(AMLA_EINVAL, "sample: null pointer");
  if (rows < 0 || n <= 0 || ld < n || n > INT32_MAX - 1) return fail(AMLA_EINVAL, "sample: bad sizes");
  if (!(temperature >= 0.f) || !(top_p >= 0.f))
    return fail(AMLA_EINVAL, "sample: needs temperature >= 0 and top_p >= 0");
  if (rows == 0) return AMLA_OK;
  if (rows > INT32_MAX / NS_MAX_CHUNKS) return fail(AMLA_EUNSUPPORTED, "sample: rows > %d", INT32_MAX / NS_MAX_CHUNKS);
  const SamplePlan p = sample_plan(rows, n);
  if (!workspace || workspace_bytes < p.bytes)
    return fail(AMLA_EWORKSPACE, "sample: workspace of %zu bytes needed, %zu given", p.bytes,
                workspace ? workspace_bytes : (size_t)0);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(AMLA_EINVAL, "sample: workspace must be 256-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char *ws = static_cast<char *>(workspace);
  float *cmax = reinterpret_cast<float *>(ws + p.cmax);
  unsigned long long *hist = reinterpret_cast<unsigned long long *>(ws + p.hist);
  NucleusState *state = reinterpret_cast<NucleusState *>(ws + p.state);
  ChunkKept *kept = reinterpret_cast<ChunkKept *>(ws + p.kept);
  const unsigned grid = (unsigned)(rows * p.chunks);
  if (temperature == 0.f) {
    ArgPart *part = reinterpret_cast<ArgPart *>(ws + p.cmax);
    ns_argmax_part_kernel<<<grid, NS_THREADS, 0, st>>>(logits, n, ld, p.chunk, p.chunks, part);
    ns_argmax_final_kernel<<<(unsigned)rows, 64, 0, st>>>(part, p.chunks, out);
    return check_launch("sample (temperature 0)");
  }
  ns_max_kernel<<<grid, NS_THREADS, 0, st>>>(logits, n, ld, temperature, p.chunk, p.chunks, cmax, hist);
  ns_hist_kernel<0><<<grid, NS_THREADS, 0, st>>>(logits, n, ld, temperature, top_p, p.chunk, p.chunks, cmax, hist, state);
  ns_hist_kernel<1><<<grid, NS_THREADS, 0, st>>>(logits, n, ld, temperature, top_p, p.chunk, p.chunks, cmax, hist, state);
  ns_hist_kernel<2><<<grid, NS_THREADS, 0, st>>>(logits, n, ld, temperature, top_p, p.chunk, p.chunks, cmax, hist, state);
  ns_kept_kernel<<<grid, NS_THREADS, 0, st>>>(logits, n, ld, temperature, top_p, p.chunk, p.chunks, cmax, hist, state,
                                              kept);
  ns_draw_kernel<<<(unsigned)rows, NS_THREADS, 0, st>>>(logits, n, ld, temperature, top_p, seed, p.chunk, p.chunks,
                                                        cmax, state, kept, out);
  return check_launch("sample");
}

}  // extern "C"
