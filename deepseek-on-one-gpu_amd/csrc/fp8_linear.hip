// Block-FP8 linear kernels for gfx950 and their C entry points.
//
//   amla_fp8_block_dequant  <- inference/ops.py:30-43 (dequant, bit-exact fp32)
//   amla_fp8_linear         <- inference/ops.py:15-44 (dequant + fp32 GEMM -> bf16)
//   amla_rms_norm           <- inference/ops.py:10-12
//   amla_apply_rope         <- inference/ops.py:86-97
//
// Skinny GEMM (M <= 64, the decode projections): HBM-bound on the fp8 weight
// stream.  Each wave owns RT tiles of 16 weight rows and walks 128-wide K
// blocks; per block a lane loads 32 contiguous fp8 bytes of one row (4 lanes
// cover the block's 128 bytes), converts them exactly to bf16 and issues four
// v_mfma_f32_16x16x32_bf16 against x^T (batch rows as the MFMA N dimension).
// The block's partial product is scaled by its fp32 scale_inv (wave-uniform:
// a 16-row tile never straddles a 128-row scale block) and added to an fp32
// accumulator, so the weight is never materialised.  The 4-16 waves of a
// workgroup split the K blocks and reduce through LDS in a fixed order, so
// results are deterministic and no workgroup waits on another (a split of K
// across workgroups would need device-scope release fences, which write back
// the per-XCD L2s and cost more than they save).
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "amla_common.h"
#include "amla_internal.h"

namespace amla {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return AMLA_OK;
}

// ---------------------------------------------------------------- K1 dequant

__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w,
                                                      const float *__restrict__ scale, int64_t n,
                                                      int64_t k, float *__restrict__ out) {
  const int64_t kb = (k + 127) >> 7;
  const int64_t chunks_per_row = k >> 4;  // fast path: k % 16 == 0
  const int64_t total = n * chunks_per_row;
  for (int64_t c = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = c / chunks_per_row;
    const int64_t j = (c - i * chunks_per_row) << 4;
    const float s = scale[(i >> 7) * kb + (j >> 7)];
    const u32x4 raw = ldg16(w + i * k + j);
    f32x4 o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x2 a = fp8x2_to_f32<false>(raw[q]);
      const f32x2 b = fp8x2_to_f32<true>(raw[q]);
      o[q] = f32x4{a.x * s, a.y * s, b.x * s, b.y * s};
    }
    f32x4 *dst = reinterpret_cast<f32x4 *>(out + i * k + j);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = o[q];
  }
}

__global__ __launch_bounds__(256) void dequant_scalar_kernel(const uint8_t *__restrict__ w,
                                                             const float *__restrict__ scale,
                                                             int64_t n, int64_t k,
                                                             float *__restrict__ out) {
  const int64_t kb = (k + 127) >> 7;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n * k;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / k, j = e - i * k;
    const f32x2 v = fp8x2_to_f32<false>((uint32_t)w[e]);
    out[e] = v.x * scale[(i >> 7) * kb + (j >> 7)];
  }
}

// ---------------------------------------------------------------- epilogue

AMLA_DEV int row_position(const GemvParams &p, int m) {
  return p.pos[m / p.seq_len] + m % p.seq_len;
}

// Stores 4 consecutive outputs n .. n+3 of row m (fp32, fully reduced).
template <int MODE>
AMLA_DEV void store4(const GemvParams &p, int m, int n, f32x4 v) {
  if (MODE == GEMV_PLAIN) {
    u32x2 o = {pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
    *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
  } else if (MODE == GEMV_RESID) {
    const u32x2 r = *reinterpret_cast<const u32x2 *>(p.res + (size_t)m * p.ldr + n);
    u32x2 o = {pack_bf16(lo_bf(r.x) + round_bf16(v.x), hi_bf(r.x) + round_bf16(v.y)),
               pack_bf16(lo_bf(r.y) + round_bf16(v.z), hi_bf(r.y) + round_bf16(v.w))};
    *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
  } else if (MODE == GEMV_QKVA) {
    u32x2 o = {pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
    if (n < p.n_split) {
      *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
    } else {
      const int b = m / p.seq_len;
      const int64_t row = row_position(p, m);
      const int nn = n - p.n_split;
      uint16_t *dst = nn < p.kv_lora
                          ? p.ckv + b * p.ckv_bstride + row * p.kv_lora + nn
                          : p.kpe + b * p.kpe_bstride + row * p.rope + (nn - p.kv_lora);
      *reinterpret_cast<u32x2 *>(dst) = o;
    }
  } else {  // GEMV_QROPE
    float a0 = round_bf16(v.x), a1 = round_bf16(v.y), a2 = round_bf16(v.z), a3 = round_bf16(v.w);
    const int d = n % p.head_dim;
    if (d >= p.nope) {
      const int i = (d - p.nope) >> 1;
      const int64_t row = row_position(p, m);
      const f32x4 cs = *reinterpret_cast<const f32x4 *>(p.rope_table + (row * (p.rope >> 1) + i) * 2);
      // (x0 + i x1) * (c + i s), each product rounded, no fused multiply-add
      const float r0 = __fsub_rn(__fmul_rn(a0, cs.x), __fmul_rn(a1, cs.y));
      const float r1 = __fadd_rn(__fmul_rn(a0, cs.y), __fmul_rn(a1, cs.x));
      const float r2 = __fsub_rn(__fmul_rn(a2, cs.z), __fmul_rn(a3, cs.w));
      const float r3 = __fadd_rn(__fmul_rn(a2, cs.w), __fmul_rn(a3, cs.z));
      a0 = r0; a1 = r1; a2 = r2; a3 = r3;
    }
    u32x2 o = {pack_bf16(a0, a1), pack_bf16(a2, a3)};
    *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
  }
}

// ---------------------------------------------------------------- skinny GEMM

// Workgroup = NW waves over one group of RT 16-row tiles; wave w takes the
// K blocks kb = w, w + NW, ...; partials reduce through LDS in wave order, so
// results are deterministic and no workgroup depends on another.
template <int RT, int MT, int NW, int MODE>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(GemvParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int tile0 = blockIdx.x * RT;
  const int KB = p.K >> 7;

  const uint8_t *wrow[RT];
  const float *srow[RT];
  bool rvalid[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int nt = (tile0 + r) * 16;
    rvalid[r] = nt < p.N;
    const bool seg1 = (MODE == GEMV_QKVA) && nt >= p.n_split;
    const int ntl = seg1 ? nt - p.n_split : nt;
    const uint8_t *wb = seg1 ? p.w1 : p.w0;
    const float *sb = seg1 ? p.s1 : p.s0;
    wrow[r] = wb + (size_t)(rvalid[r] ? ntl + li : 0) * p.K + lg * 32;
    srow[r] = sb + (size_t)(rvalid[r] ? (ntl >> 7) : 0) * KB;
  }
  const uint16_t *xrow[MT];
  bool mvalid[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = t * 16 + li;
    mvalid[t] = m < p.M;
    xrow[t] = p.x + (size_t)(mvalid[t] ? m : 0) * p.ldx + lg * 32;
  }

  f32x4 acc[RT][MT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // block kb + NW is loaded while block kb is computed (a wave otherwise sits
  // out one memory latency per 2 KB of weights)
  u32x4 a0[2][RT], a1[2][RT];
  bf16x8 xb[2][MT][4];
  auto load_block = [&](int kb, int buf) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      if (rvalid[r]) {
        a0[buf][r] = ldg16_nt(wrow[r] + (size_t)kb * 128);
        a1[buf][r] = ldg16_nt(wrow[r] + (size_t)kb * 128 + 16);
      } else {
        a0[buf][r] = u32x4{0, 0, 0, 0};
        a1[buf][r] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        xb[buf][t][u] = mvalid[t] ? as_bf16x8(ldg16(xrow[t] + kb * 128 + u * 8)) : as_bf16x8(u32x4{0, 0, 0, 0});
  };
  auto compute_block = [&](int kb, int buf) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const float s = rvalid[r] ? srow[r][kb] : 0.f;
      bf16x8 w0, w1, w2, w3;
      fp8x16_to_bf16x16(a0[buf][r], w0, w1);
      fp8x16_to_bf16x16(a1[buf][r], w2, w3);
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
        c = mfma16(w0, xb[buf][t][0], c);
        c = mfma16(w1, xb[buf][t][1], c);
        c = mfma16(w2, xb[buf][t][2], c);
        c = mfma16(w3, xb[buf][t][3], c);
        acc[r][t] += s * c;
      }
    }
  };
  if (wave < KB) load_block(wave, 0);
  int kb = wave;
  for (; kb + NW < KB; kb += 2 * NW) {
    load_block(kb + NW, 1);
    compute_block(kb, 0);
    if (kb + 2 * NW < KB) load_block(kb + 2 * NW, 0);
    compute_block(kb + NW, 1);
  }
  if (kb < KB) compute_block(kb, 0);

  __shared__ f32x4 red[NW][RT * MT][64];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][r * MT + t][lane] = acc[r][t];
  __syncthreads();
  for (int idx = threadIdx.x; idx < RT * MT * 64; idx += NW * 64) {
    const int rt = idx >> 6, ln = idx & 63;
    const int r = rt / MT, t = rt % MT;
    const int m = t * 16 + (ln & 15);
    const int n = (tile0 + r) * 16 + 4 * (ln >> 4);
    if (m >= p.M || n >= p.N) continue;
    f32x4 v = red[0][rt][ln];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][rt][ln];
    store4<MODE>(p, m, n, v);
  }
}

GemvPlan plan_gemv(int M, int N, int K) {
  GemvPlan pl;
  const int tiles = (N + 15) / 16;
  const int KB = K / 128;
  const int MT = (M + 15) / 16;
  // two row tiles per wave halve the x traffic once there are enough rows
  pl.rt = (M > 4 && tiles >= 2 * 256) ? 2 : 1;
  pl.groups = (tiles + pl.rt - 1) / pl.rt;
  // waves per workgroup: enough waves in flight to cover the memory latency
  // (~24 resident waves per CU at this kernel's register count) while every
  // workgroup stays resident, and at least two K blocks per wave
  int nw = 16;
  while (nw > 4 && ((int64_t)pl.groups * nw > 256 * 24 || KB < 2 * nw)) nw /= 2;
  while (nw > 4 && nw * pl.rt * (MT > 2 ? 4 : MT) > 64) nw /= 2;
  pl.nw = nw;
  return pl;
}

template <int RT, int MT, int NW>
static void launch_cfg(const GemvParams &p, int mode, const GemvPlan &pl, hipStream_t st) {
  dim3 grid(pl.groups);
  switch (mode) {
    case GEMV_PLAIN: gemv_kernel<RT, MT, NW, GEMV_PLAIN><<<grid, NW * 64, 0, st>>>(p); break;
    case GEMV_RESID: gemv_kernel<RT, MT, NW, GEMV_RESID><<<grid, NW * 64, 0, st>>>(p); break;
    case GEMV_QKVA: gemv_kernel<RT, MT, NW, GEMV_QKVA><<<grid, NW * 64, 0, st>>>(p); break;
    default: gemv_kernel<RT, MT, NW, GEMV_QROPE><<<grid, NW * 64, 0, st>>>(p); break;
  }
}

template <int RT, int MT>
static void launch_rt_mt(const GemvParams &p, int mode, const GemvPlan &pl, hipStream_t st) {
  if (pl.nw == 16) launch_cfg<RT, MT, 16>(p, mode, pl, st);
  else if (pl.nw == 8) launch_cfg<RT, MT, 8>(p, mode, pl, st);
  else launch_cfg<RT, MT, 4>(p, mode, pl, st);
}

template <int RT>
static void launch_rt(const GemvParams &p, int mode, const GemvPlan &pl, hipStream_t st) {
  const int MT = (p.M + 15) / 16;
  if (MT == 1) launch_rt_mt<RT, 1>(p, mode, pl, st);
  else if (MT == 2) launch_rt_mt<RT, 2>(p, mode, pl, st);
  else launch_rt_mt<RT, 4>(p, mode, pl, st);
}

int launch_gemv(const GemvParams &p0, int mode, const GemvPlan &pl, hipStream_t st) {
  if (p0.M < 1 || p0.M > 64) return fail(AMLA_EINVAL, "skinny fp8 GEMM needs 1 <= M <= 64 (got %d)", p0.M);
  if (p0.N % 16 || p0.K % 128)
    return fail(AMLA_EUNSUPPORTED, "skinny fp8 GEMM needs N %% 16 == 0 and K %% 128 == 0 (N=%d K=%d)", p0.N, p0.K);
  if (pl.rt == 1) launch_rt<1>(p0, mode, pl, st);
  else launch_rt<2>(p0, mode, pl, st);
  return check_launch("fp8 skinny GEMM");
}

// ---------------------------------------------------------------- rms_norm

// One workgroup per row: fp32 sum of squares, r = rsqrt(mean + eps),
// y = bf16(bf16(x * r) * gamma)  (the two roundings of inference/ops.py:12).
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t *__restrict__ x, int64_t dim,
                                                       int64_t ldx, const uint16_t *__restrict__ gamma,
                                                       float eps, uint16_t *__restrict__ y,
                                                       int64_t ldy) {
  const uint16_t *xr = x + blockIdx.x * ldx;
  uint16_t *yr = y + blockIdx.x * ldy;
  float ss = 0.f;
  for (int64_t j = threadIdx.x; j < dim; j += 256) {
    const float v = bf2f(xr[j]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float r = rsqrtf(tot / (float)dim + eps);
  for (int64_t j = threadIdx.x; j < dim; j += 256) {
    const float nv = round_bf16(bf2f(xr[j]) * r);
    yr[j] = f2bf(nv * bf2f(gamma[j]));
  }
}

int launch_rms_norm(const uint16_t *x, int64_t rows, int64_t dim, int64_t ldx, const uint16_t *gamma,
                    float eps, uint16_t *y, int64_t ldy, hipStream_t st) {
  if (rows == 0) return AMLA_OK;
  rms_norm_kernel<<<dim3((unsigned)rows), 256, 0, st>>>(x, dim, ldx, gamma, eps, y, ldy);
  return check_launch("rms_norm");
}

// ---------------------------------------------------------------- apply_rope

__global__ __launch_bounds__(256) void rope_kernel(const uint16_t *__restrict__ x, int64_t groups,
                                                   int64_t s, int64_t half,
                                                   const float *__restrict__ freqs,
                                                   uint16_t *__restrict__ y) {
  const int64_t total = groups * s * half;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e % half;
    const int64_t t = (e / half) % s;
    const uint32_t xv = reinterpret_cast<const uint32_t *>(x)[e];
    const float a = lo_bf(xv), b = hi_bf(xv);
    const float c = freqs[(t * half + i) * 2], sn = freqs[(t * half + i) * 2 + 1];
    const float re = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, sn));
    const float im = __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, c));
    reinterpret_cast<uint32_t *>(y)[e] = pack_bf16(re, im);
  }
}

}  // namespace amla

using namespace amla;

extern "C" {

int amla_abi_version(void) { return 100; }

const char *amla_last_error(void) { return g_last_error.c_str(); }

int amla_fp8_block_dequant(const void *weight, const float *scale_inv, int64_t n, int64_t k,
                           float *out, void *stream) {
  if (!weight || !scale_inv || !out) return fail(AMLA_EINVAL, "fp8_block_dequant: null pointer");
  if (n < 0 || k < 0) return fail(AMLA_EINVAL, "fp8_block_dequant: negative shape");
  if (n == 0 || k == 0) return AMLA_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint8_t *w = reinterpret_cast<const uint8_t *>(weight);
  if (k % 16 == 0 && aligned16(w) && aligned16(out)) {
    const int64_t chunks = n * (k / 16);
    const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 65536);
    dequant_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(w, scale_inv, n, k, out);
  } else {
    const int64_t blocks = std::min<int64_t>((n * k + 255) / 256, 65536);
    dequant_scalar_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(w, scale_inv, n, k, out);
  }
  return check_launch("fp8_block_dequant");
}

size_t amla_fp8_linear_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  (void)m; (void)n; (void)k;
  return 0;
}

int amla_fp8_linear(const void *x, int64_t m, int64_t k, int64_t ldx, const void *weight,
                    const float *scale_inv, int64_t n, void *y, int64_t ldy, void *workspace,
                    size_t workspace_bytes, void *stream) {
  if (!x || !weight || !scale_inv || !y) return fail(AMLA_EINVAL, "fp8_linear: null pointer");
  if (m < 0 || n <= 0 || k <= 0) return fail(AMLA_EINVAL, "fp8_linear: bad shape m=%lld n=%lld k=%lld",
                                             (long long)m, (long long)n, (long long)k);
  if (ldx < k || ldy < n) return fail(AMLA_EINVAL, "fp8_linear: row stride smaller than the row");
  if (m == 0) return AMLA_OK;
  if (n % 16 || k % 128 || ldx % 8 || ldy % 4 || !aligned16(x) || !aligned16(weight))
    return fail(AMLA_EUNSUPPORTED,
                "fp8_linear: needs n %% 16 == 0, k %% 128 == 0, ldx %% 8 == 0, ldy %% 4 == 0 and 16-byte "
                "aligned x/weight (n=%lld k=%lld)",
                (long long)n, (long long)k);
  GemvParams p = {};
  p.x = reinterpret_cast<const uint16_t *>(x);
  p.M = (int)m;
  p.ldx = (int)ldx;
  p.w0 = reinterpret_cast<const uint8_t *>(weight);
  p.s0 = scale_inv;
  p.N = (int)n;
  p.K = (int)k;
  p.n_split = (int)n;
  p.y = reinterpret_cast<uint16_t *>(y);
  p.ldy = (int)ldy;
  p.seq_len = 1;
  (void)workspace;
  (void)workspace_bytes;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (m > 64) return launch_gemm(p, GEMV_PLAIN, st);
  return launch_gemv(p, GEMV_PLAIN, plan_gemv((int)m, (int)n, (int)k), st);
}

int amla_rms_norm(const void *x, int64_t rows, int64_t dim, int64_t ldx, const void *gamma, float eps,
                  void *y, int64_t ldy, void *stream) {
  if (!x || !gamma || !y) return fail(AMLA_EINVAL, "rms_norm: null pointer");
  if (rows < 0 || dim <= 0 || ldx < dim || ldy < dim) return fail(AMLA_EINVAL, "rms_norm: bad shape");
  if (rows > 0x7fffffff) return fail(AMLA_EUNSUPPORTED, "rms_norm: too many rows");
  return launch_rms_norm(reinterpret_cast<const uint16_t *>(x), rows, dim, ldx,
                         reinterpret_cast<const uint16_t *>(gamma), eps, reinterpret_cast<uint16_t *>(y),
                         ldy, reinterpret_cast<hipStream_t>(stream));
}

int amla_apply_rope(const void *x, int64_t groups, int64_t s, int64_t dim, const float *freqs, void *y,
                    void *stream) {
  if (!x || !freqs || !y) return fail(AMLA_EINVAL, "apply_rope: null pointer");
  if (groups < 0 || s < 0 || dim <= 0 || dim % 2) return fail(AMLA_EINVAL, "apply_rope: bad shape");
  const int64_t total = groups * s * (dim / 2);
  if (total == 0) return AMLA_OK;
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
  rope_kernel<<<dim3((unsigned)blocks), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint16_t *>(x), groups, s, dim / 2, freqs, reinterpret_cast<uint16_t *>(y));
  return check_launch("apply_rope");
}

}  // extern "C"
