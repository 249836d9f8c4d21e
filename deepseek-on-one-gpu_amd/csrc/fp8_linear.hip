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

// Streaming skinny GEMM for M <= 64 (decode projections).  The weight matrix
// is cut into units of RG consecutive 16-row tiles x one K part of 4*BW
// 128-wide blocks; a workgroup (4 waves) owns one unit and wave w the blocks
// BW*w .. BW*w+BW-1 of the part.  A wave holds the x fragments of its blocks
// in registers for the whole unit and streams the weight rows tile after tile
// (the next tile's loads are in flight while the current one is converted and
// multiplied): 2*BW KB of weights per tile and wave, no x traffic per tile.
// The four waves' partial tiles are summed through LDS in wave order; with
// one K part the sum goes through the epilogue, otherwise into fp32 partials
// [part][M][N] that gemv_finish sums in part order (deterministic, no atomics
// and no workgroup depends on another).
//
// Within a block, lane (row l%16, group g = l/16) holds weight bytes
// 16g .. 16g+15 and 64+16g .. 64+16g+15 of its row: each 16 B load covers
// whole 64 B sectors of 16 rows.  The MFMA K order is permuted accordingly
// and the x fragments follow the same order.
constexpr int GEMV_MAX_PARTS = 32;  // K parts summed by gemv_finish
constexpr int GEMV_MAX_RG = 16;     // 16-row tiles per workgroup

template <int MT, int BW, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p, int rg, int kparts) {
  // wave index in a scalar register: block ranges, scale loads and the
  // per-block branches below stay scalar (a vector scale load would make the
  // compiler wait for every weight load in flight)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int KB = p.K >> 7;
  const int ntiles = p.N >> 4;
  const int part = blockIdx.x % kparts;
  const int tile_begin = (blockIdx.x / kparts) * rg;
  const int tile_end = min(tile_begin + rg, ntiles);
  const int kb0 = part * 4 * BW + wave * BW;            // first block of this wave
  const int nb = max(0, min(BW, KB - kb0));              // blocks of this wave (wave-uniform)

  // x fragments of the wave's blocks: [block][m tile][MFMA of the block]
  bf16x8 xf[BW][MT][4];
#pragma unroll
  for (int j = 0; j < BW; ++j)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 16 + li;
      const bool ok = j < nb && m < p.M;
      const uint16_t *xr = p.x + (size_t)(ok ? m : 0) * p.ldx + (size_t)(kb0 + (ok ? j : 0)) * 128 + lg * 16;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        xf[j][t][u] = ok ? as_bf16x8(ldg16(xr + (u >> 1) * 64 + (u & 1) * 8)) : as_bf16x8(u32x4{0, 0, 0, 0});
    }

  __shared__ f32x4 red[2][4][MT][64];
  // reduced tiles of the unit, epilogue deferred to the end (one round of
  // epilogue loads - rope table, residual - instead of one per tile)
  __shared__ f32x4 done[GEMV_MAX_RG][MT][64];
  // a tile's weights and block scales are loaded together, one tile ahead,
  // unconditionally (the last trip and absent blocks re-read valid data that
  // is not used): with no load under a branch the compiler's wait for the
  // current tile never waits for the next one's loads
  constexpr int NBUF = 3;  // tiles in flight: the current one and two ahead
  u32x4 wv[NBUF][BW][2];
  float sv[NBUF][BW];
  const uint32_t woff = (uint32_t)(li * p.K + lg * 16);
  auto load_tile = [&](int tile, int buf) {
    const int nt = min(tile, tile_end - 1) * 16;
    const bool seg1 = (MODE == GEMV_QKVA) && nt >= p.n_split;
    const uint8_t *wb = seg1 ? p.w1 : p.w0;
    const int nl = seg1 ? nt - p.n_split : nt;
    // uniform tile base + unsigned 32-bit lane offset: scalar-base loads, no
    // per-tile address registers
    const uint8_t *tb = wb + (size_t)nl * p.K;
    const float *sr = (seg1 ? p.s1 : p.s0) + (size_t)(nl >> 7) * KB;
#pragma unroll
    for (int j = 0; j < BW; ++j) {
      const int kb = min(kb0 + j, KB - 1);
      sv[buf][j] = sr[kb];
      wv[buf][j][0] = ldg16_nt(tb + (size_t)kb * 128 + woff);
      wv[buf][j][1] = ldg16_nt(tb + (size_t)kb * 128 + 64 + woff);
    }
  };
  auto do_tile = [&](int tile, int buf) {
    load_tile(tile + NBUF - 1, (buf + NBUF - 1) % NBUF);
    const int nt = tile * 16;
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BW; ++j) {
      if (j < nb) {
        const float sc = sv[buf][j];
        bf16x8 w0, w1, w2, w3;
        fp8x16_to_bf16x16(wv[buf][j][0], w0, w1);
        fp8x16_to_bf16x16(wv[buf][j][1], w2, w3);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
          c = mfma16(w0, xf[j][t][0], c);
          c = mfma16(w1, xf[j][t][1], c);
          c = mfma16(w2, xf[j][t][2], c);
          c = mfma16(w3, xf[j][t][3], c);
          acc[t] += sc * c;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) red[tile & 1][wave][t][lane] = acc[t];
    __syncthreads();
    // MT * 64 lanes of results (4 outputs each) per tile; thread idx sums the
    // four waves in order
    for (int idx = threadIdx.x; idx < MT * 64; idx += 256) {
      const int t = idx >> 6, ln = idx & 63;
      const int m = t * 16 + (ln & 15);
      const int n = nt + 4 * (ln >> 4);
      if (m >= p.M) continue;
      f32x4 v = red[tile & 1][0][t][ln];
      v += red[tile & 1][1][t][ln];
      v += red[tile & 1][2][t][ln];
      v += red[tile & 1][3][t][ln];
      if (kparts == 1) done[tile - tile_begin][t][ln] = v;
      else *reinterpret_cast<f32x4 *>(p.part + ((size_t)part * p.M + m) * p.N + n) = v;
    }
    // red[tile & 1] is rewritten two tiles later, after the next barrier
  };
  // NBUF tiles per trip: the register buffer index stays a constant
  if (tile_begin < tile_end) {
#pragma unroll
    for (int b = 0; b < NBUF - 1; ++b) load_tile(tile_begin + b, b);
  }
  for (int tile = tile_begin; tile < tile_end; tile += NBUF) {
    do_tile(tile, 0);
    if (tile + 1 < tile_end) do_tile(tile + 1, 1);
    if (tile + 2 < tile_end) do_tile(tile + 2, 2);
  }
  if (kparts == 1) {
    __syncthreads();
    const int nitems = (tile_end - tile_begin) * MT * 64;
    for (int idx = threadIdx.x; idx < nitems; idx += 256) {
      const int tl = idx / (MT * 64), t = (idx >> 6) % MT, ln = idx & 63;
      const int m = t * 16 + (ln & 15);
      const int n = (tile_begin + tl) * 16 + 4 * (ln >> 4);
      if (m < p.M) store4<MODE>(p, m, n, done[tl][t][ln]);
    }
  }
}

// Sums the K parts of gemv_kernel in part order and applies the epilogue.
// All parts are loaded before the first add (independent loads in flight).
template <int MODE>
__global__ __launch_bounds__(64) void gemv_finish(GemvParams p, int kparts) {
  const int64_t total = (int64_t)p.M * (p.N >> 2);
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (i >= total) return;
  const int m = (int)(i / (p.N >> 2));
  const int n = (int)(i % (p.N >> 2)) * 4;
  f32x4 v[GEMV_MAX_PARTS];
#pragma unroll
  for (int q = 0; q < GEMV_MAX_PARTS; ++q)
    if (q < kparts) v[q] = *reinterpret_cast<const f32x4 *>(p.part + ((size_t)q * p.M + m) * p.N + n);
  f32x4 s = v[0];
#pragma unroll
  for (int q = 1; q < GEMV_MAX_PARTS; ++q)
    if (q < kparts) s += v[q];
  store4<MODE>(p, m, n, s);
}

GemvPlan plan_gemv(int M, int N, int K) {
  GemvPlan pl;
  const int tiles = N / 16;
  const int KB = K / 128;
  const int MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  // blocks per wave: x fragments take 16 * BW * MT registers (<= 64).  One K
  // part when it fits (no finishing pass), else the BW wasting the fewest
  // wave-blocks, larger BW on ties
  const int bw_max = MT == 1 ? 4 : (MT == 2 ? 2 : 1);
  int bw = bw_max;
  if (KB <= 4 * bw_max) {
    while (bw > 1 && 4 * (bw / 2) >= KB) bw /= 2;
  } else {
    int best_waste = 1 << 30;
    for (int b = bw_max; b >= 1; b /= 2) {
      const int waste = ((KB + 4 * b - 1) / (4 * b)) * 4 * b - KB;
      if (waste < best_waste) {
        best_waste = waste;
        bw = b;
      }
    }
  }
  pl.bw = bw;
  pl.kparts = (KB + 4 * bw - 1) / (4 * bw);  // launch_gemv rejects more than GEMV_MAX_PARTS
  // tiles per unit: fewest rounds of 256 workgroups x tiles per unit, then
  // the largest unit (fewer x reloads); <= 16 tiles
  int best_rg = 1;
  int64_t best_cost = INT64_MAX;
  for (int rg = 1; rg <= GEMV_MAX_RG; ++rg) {
    const int64_t units = (int64_t)((tiles + rg - 1) / rg) * pl.kparts;
    const int64_t cost = ((units + 255) / 256) * rg;
    if (cost <= best_cost) {
      best_cost = cost;
      best_rg = rg;
    }
  }
  pl.rg = best_rg;
  pl.groups = ((tiles + pl.rg - 1) / pl.rg) * pl.kparts;
  pl.part_bytes = pl.kparts > 1 ? (size_t)pl.kparts * M * N * 4 : 0;
  return pl;
}

template <int MT, int BW>
static void launch_cfg(const GemvParams &p, int mode, const GemvPlan &pl, hipStream_t st) {
  dim3 grid(pl.groups);
  switch (mode) {
    case GEMV_PLAIN: gemv_kernel<MT, BW, GEMV_PLAIN><<<grid, 256, 0, st>>>(p, pl.rg, pl.kparts); break;
    case GEMV_RESID: gemv_kernel<MT, BW, GEMV_RESID><<<grid, 256, 0, st>>>(p, pl.rg, pl.kparts); break;
    case GEMV_QKVA: gemv_kernel<MT, BW, GEMV_QKVA><<<grid, 256, 0, st>>>(p, pl.rg, pl.kparts); break;
    default: gemv_kernel<MT, BW, GEMV_QROPE><<<grid, 256, 0, st>>>(p, pl.rg, pl.kparts); break;
  }
}

int launch_gemv(const GemvParams &p0, int mode, const GemvPlan &pl, hipStream_t st) {
  if (p0.M < 1 || p0.M > 64) return fail(AMLA_EINVAL, "skinny fp8 GEMM needs 1 <= M <= 64 (got %d)", p0.M);
  if (p0.N % 16 || p0.K % 128)
    return fail(AMLA_EUNSUPPORTED, "skinny fp8 GEMM needs N %% 16 == 0 and K %% 128 == 0 (N=%d K=%d)", p0.N, p0.K);
  if (pl.kparts > GEMV_MAX_PARTS)
    return fail(AMLA_EUNSUPPORTED, "skinny fp8 GEMM: K=%d is too long for M=%d (more than %d K parts)", p0.K, p0.M,
                GEMV_MAX_PARTS);
  if (pl.kparts > 1 && !p0.part) return fail(AMLA_EWORKSPACE, "skinny fp8 GEMM: missing partial-sum workspace");
  const int MT = p0.M <= 16 ? 1 : (p0.M <= 32 ? 2 : 4);
  if (MT == 1) {
    if (pl.bw == 4) launch_cfg<1, 4>(p0, mode, pl, st);
    else if (pl.bw == 2) launch_cfg<1, 2>(p0, mode, pl, st);
    else launch_cfg<1, 1>(p0, mode, pl, st);
  } else if (MT == 2) {
    if (pl.bw == 2) launch_cfg<2, 2>(p0, mode, pl, st);
    else launch_cfg<2, 1>(p0, mode, pl, st);
  } else {
    launch_cfg<4, 1>(p0, mode, pl, st);
  }
  if (pl.kparts > 1) {
    const int64_t total = (int64_t)p0.M * (p0.N / 4);
    const unsigned blocks = (unsigned)((total + 63) / 64);
    switch (mode) {
      case GEMV_PLAIN: gemv_finish<GEMV_PLAIN><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      case GEMV_RESID: gemv_finish<GEMV_RESID><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      case GEMV_QKVA: gemv_finish<GEMV_QKVA><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      default: gemv_finish<GEMV_QROPE><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
    }
  }
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
  if (m < 1 || m > 64 || n <= 0 || k <= 0 || n % 16 || k % 128 || n > INT32_MAX || k > INT32_MAX) return 0;
  return plan_gemv((int)m, (int)n, (int)k).part_bytes;
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
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (m > 64) return launch_gemm(p, GEMV_PLAIN, st);
  const GemvPlan pl = plan_gemv((int)m, (int)n, (int)k);
  if (pl.part_bytes) {
    if (!workspace || workspace_bytes < pl.part_bytes || !aligned16(workspace))
      return fail(AMLA_EWORKSPACE, "fp8_linear: needs %zu bytes of 16-byte aligned workspace (got %zu)", pl.part_bytes,
                  workspace ? workspace_bytes : (size_t)0);
    p.part = reinterpret_cast<float *>(workspace);
  }
  return launch_gemv(p, GEMV_PLAIN, pl, st);
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
