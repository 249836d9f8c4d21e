// Output head for gfx950:
//
//   amla_bf16_logits  <- hidden.float() @ lm_head_w.float().T, inference/forward.py:70-72
//   amla_argmax       <- sample(..., temperature=0), inference/engine.py:172-173
//   amla_sample_top_p <- sample(...) with temperature and nucleus filtering, engine.py:175-186
//
// The logits are exact bf16 products summed in fp32 by MFMA (no fp32 copy of
// the 129280 x 7168 matrix, which the reference makes every step).  Sampling
// is one workgroup per row: softmax statistics, a radix search on the
// probability value for the nucleus threshold, and an inverse-CDF draw over
// the kept tokens from a counter-based generator.
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

constexpr int SAMPLE_THREADS = 1024;

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

template <int NT>
AMLA_DEV float block_sum(float s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  __shared__ float ss[NT / 64];
  if ((threadIdx.x & 63) == 0) ss[threadIdx.x >> 6] = s;
  __syncthreads();
  float t = 0.f;
  for (int q = 0; q < NT / 64; ++q) t += ss[q];
  __syncthreads();
  return t;
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

// 64-bit counter-based generator (SplitMix64 finaliser) -> uniform [0, 1)
AMLA_DEV float uniform01(uint64_t seed, uint64_t ctr) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (ctr + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(z >> 40) * (1.0f / 16777216.0f);
}

// Nucleus sampling of one row, the reference's rule: p = softmax(logits / T);
// sorted descending, token k is dropped when the mass strictly before it
// exceeds top_p; the kept probabilities are renormalised and one is drawn.
// Everything works on e = exp(logits / T - max) (p = e / sum e; the
// normalisation cancels): with e1 > e2 > .. sorted and C_k their prefix sums,
// the reference keeps e_1 .. e_{K+1}, K the last k with C_k <= top_p * sum e,
// i.e. every token with e >= t, t the smallest value whose strictly larger
// mass is <= top_p * sum e.  t is always the value of a token (or 0), found on
// the fp32 bit pattern (e >= 0: bit order = value order) by a three-level
// radix search: per level a histogram of the mass over the next 11 / 11 / 10
// bits in 2^-40 fixed point (integer sums: independent of the atomics' order).
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
  constexpr double FX = 1099511627776.0;  // 2^40
  __shared__ unsigned long long hist[2048];
  __shared__ unsigned long long above_s, total_s;
  __shared__ uint32_t prefix_s;
  if (tid == 0) {
    above_s = 0;
    prefix_s = 0;
  }
  for (int level = 0; level < 3; ++level) {
    const int shift = level == 0 ? 21 : (level == 1 ? 10 : 0);
    const int nb = level == 2 ? 1024 : 2048;
    for (int i = tid; i < 2048; i += SAMPLE_THREADS) hist[i] = 0;
    __syncthreads();
    const uint32_t prefix = prefix_s;
    const int pshift = shift + (level == 2 ? 10 : 11);  // bits above this level's bins
    for (int64_t j = tid; j < n; j += SAMPLE_THREADS) {
      const float e = ev(j);
      const uint32_t key = __float_as_uint(e);
      if (level == 0 || (key >> pshift) == (prefix >> pshift))
        atomicAdd(&hist[(key >> shift) & (nb - 1)], (unsigned long long)((double)e * FX));
    }
    __syncthreads();
    if (level == 0 && tid < 64) {
      unsigned long long t = 0;
      for (int q = tid; q < 2048; q += 64) t += hist[q];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
      if (tid == 0) total_s = t;
    }
    __syncthreads();
    const unsigned long long top_fx = (unsigned long long)((double)top_p * (double)total_s);
    // smallest bin b whose mass above (bins > b, plus everything above this
    // level's prefix) is <= top_p * sum: wave 0, nb / 64 bins per lane from the top
    if (tid < 64) {
      const int per = nb / 64;
      const int b_hi = nb - 1 - tid * per;  // this lane's bins: b_hi down to b_hi - per + 1
      unsigned long long own = 0;
      for (int q = 0; q < per; ++q) own += hist[b_hi - q];
      unsigned long long ex = own;  // inclusive prefix over lanes 0..tid (higher bins first)
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long v = __shfl_up(ex, o, 64);
        if (tid >= o) ex += v;
      }
      ex -= own;
      const unsigned long long base = above_s;
      unsigned long long run = base + ex;
      int found = -1;
      unsigned long long mass_above = 0;
      for (int q = 0; q < per; ++q) {
        const int bb = b_hi - q;
        if (run > top_fx) break;
        found = bb;  // bins are visited downwards: keep the smallest
        mass_above = run;
        run += hist[bb];
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const int ob = __shfl_xor(found, o, 64);
        const unsigned long long om = __shfl_xor(mass_above, o, 64);
        if (ob >= 0 && (found < 0 || ob < found)) {
          found = ob;
          mass_above = om;
        }
      }
      if (tid == 0) {
        prefix_s = prefix | ((uint32_t)found << shift);
        above_s = mass_above;
      }
    }
    __syncthreads();
  }
  const float tstar = __uint_as_float(prefix_s);  // keep e >= t*
  // kept mass, then an inverse-CDF draw in vocabulary order over contiguous chunks
  const int64_t chunk = (n + SAMPLE_THREADS - 1) / SAMPLE_THREADS;
  const int64_t c0 = std::min<int64_t>(n, tid * chunk), c1 = std::min<int64_t>(n, c0 + chunk);
  float mine = 0.f;
  for (int64_t j = c0; j < c1; ++j) {
    const float e = ev(j);
    if (e >= tstar) mine += e;
  }
  // exclusive prefix of the per-thread kept mass
  __shared__ float pre[SAMPLE_THREADS];
  pre[tid] = mine;
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int q = 0; q < SAMPLE_THREADS; ++q) {
      const float v = pre[q];
      pre[q] = acc;
      acc += v;
    }
  }
  __syncthreads();
  __shared__ float tot_s;
  if (tid == SAMPLE_THREADS - 1) tot_s = pre[tid] + mine;
  __syncthreads();
  const float u = uniform01(seed, blockIdx.x) * tot_s;
  __shared__ int pick;
  if (tid == 0) pick = -1;
  __syncthreads();
  if (u >= pre[tid] && u < pre[tid] + mine) {
    float acc = pre[tid];
    int64_t last = -1;
    for (int64_t j = c0; j < c1; ++j) {
      const float e = ev(j);
      if (e < tstar) continue;
      last = j;
      acc += e;
      if (u < acc) break;
    }
    atomicMax(&pick, (int)last);
  }
  __syncthreads();
  if (tid == 0) {
    int r = pick;
    if (r < 0) {  // u fell on the rounding edge of the last chunk: take the last kept token
      for (int64_t j = n - 1; j >= 0; --j)
        if (ev(j) >= tstar) {
          r = (int)j;
          break;
        }
    }
    out[blockIdx.x] = r;
  }
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

}  // extern "C"
