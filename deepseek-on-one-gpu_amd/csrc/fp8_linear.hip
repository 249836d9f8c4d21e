// Block-FP8 linear kernels for gfx950 and their C entry points.
//
//   amla_fp8_block_dequant  <- inference/ops.py:30-43 (dequant, bit-exact fp32)
//   amla_fp8_linear         <- inference/ops.py:15-44 (dequant + fp32 GEMM -> bf16)
//   amla_rms_norm           <- inference/ops.py:10-12
//   amla_apply_rope         <- inference/ops.py:86-97
//
// Skinny GEMM (M <= 64, the decode projections): HBM-bound on the fp8 weight
// stream.  Weight tiles of 16 rows stream HBM -> LDS by LDS-DMA; the 4 waves
// of a workgroup split a tile's 128-wide K blocks, convert the fp8 bytes
// exactly to bf16 and issue v_mfma_f32_16x16x32_bf16 against x^T (batch rows
// as the MFMA N dimension).  A block's partial product is scaled by its fp32
// scale_inv (wave-uniform: a 16-row tile never straddles a 128-row scale
// block) and added to an fp32 accumulator, so the weight is never
// materialised; the waves' partial tiles are summed through LDS in wave
// order.  A long K is split into K parts over workgroups: their fp32 sums go
// to the workspace and a finishing pass (gemv_finish, or the consumer's own
// finish) adds them in part order.  Results are deterministic, and no
// workgroup waits on another: an in-kernel finish would need device-scope
// release fences, which write back the per-XCD L2s and cost more than the
// separate pass.  M > 64 takes the tiled GEMM (gemm_kernel, mla_prefill.hip).
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>

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

// Operands the epilogue of outputs (m, n .. n+3) reads besides the sums: the
// residual (RESID), the position of row m (QKVA, QROPE) and the (cos, sin)
// pairs of that position for columns n .. n+3 (QROPE; loaded for every column,
// used by the rope columns).  The streaming GEMVs load them at the start
// (epi_load1, then epi_load2, which depends on the position, once the stream
// is issued), so that their tail waits for no further round trip.
struct EpiOps {
  int pos;
  u32x2 res;
  f32x4 cs;
};

template <int MODE>
AMLA_DEV void epi_load1(const GemvParams &p, int m, int n, EpiOps &e) {
  if constexpr (MODE == GEMV_RESID) e.res = *reinterpret_cast<const u32x2 *>(p.res + (size_t)m * p.ldr + n);
  if constexpr (MODE == GEMV_QKVA || MODE == GEMV_QROPE) e.pos = p.pos[m / p.seq_len];
}

template <int MODE>
AMLA_DEV void epi_load2(const GemvParams &p, int m, int n, EpiOps &e) {
  if constexpr (MODE == GEMV_QROPE) {
    const int i = max(n % p.head_dim - p.nope, 0) >> 1;
    const int64_t row = min(e.pos + m % p.seq_len, p.rope_rows - 1);  // in bounds for any device position
    e.cs = *reinterpret_cast<const f32x4 *>(p.rope_table + (row * (p.rope >> 1) + i) * 2);
  }
}

// Stores 4 consecutive outputs n .. n+3 of row m (fp32, fully reduced), its
// other operands from e.
template <int MODE>
AMLA_DEV void store4e(const GemvParams &p, int m, int n, f32x4 v, const EpiOps &e) {
  if (MODE == GEMV_PLAIN) {
    u32x2 o = {pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
    *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
  } else if (MODE == GEMV_F32) {
    *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.y) + (size_t)m * p.ldy + n) = v;
  } else if (MODE == GEMV_RESID) {
    const u32x2 r = e.res;
    u32x2 o = {pack_bf16(lo_bf(r.x) + round_bf16(v.x), hi_bf(r.x) + round_bf16(v.y)),
               pack_bf16(lo_bf(r.y) + round_bf16(v.z), hi_bf(r.y) + round_bf16(v.w))};
    *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
  } else if (MODE == GEMV_QKVA) {
    u32x2 o = {pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
    if (n < p.n_split) {
      *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
    } else {
      const int b = m / p.seq_len;
      const int64_t row = e.pos + m % p.seq_len;
      if (row >= p.max_rows) return;  // a device position past the cache: nothing is written
      const int nn = n - p.n_split;
      uint16_t *dst = nn < p.kv_lora
                          ? p.ckv + b * p.ckv_bstride + row * p.kv_lora + nn
                          : p.kpe + b * p.kpe_bstride + row * p.rope + (nn - p.kv_lora);
      *reinterpret_cast<u32x2 *>(dst) = o;
    }
  } else {  // GEMV_QROPE
    float a0 = round_bf16(v.x), a1 = round_bf16(v.y), a2 = round_bf16(v.z), a3 = round_bf16(v.w);
    if (n % p.head_dim >= p.nope) {
      const f32x4 cs = e.cs;
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

// store4e with its operands loaded here.
template <int MODE>
AMLA_DEV void store4(const GemvParams &p, int m, int n, f32x4 v) {
  EpiOps e = {};
  epi_load1<MODE>(p, m, n, e);
  epi_load2<MODE>(p, m, n, e);
  store4e<MODE>(p, m, n, v, e);
}

// ---------------------------------------------------------------- skinny GEMM

// Streaming skinny GEMM for M <= 64 (decode projections).  The weight matrix
// is cut into units of RG consecutive 16-row tiles x one K part of KPB
// 128-wide blocks; a workgroup (4 waves) owns one unit.
//   * x[:, part] is staged in LDS once per workgroup (bf16, 16 B padded rows);
//   * weight tiles stream HBM -> LDS with LDS-DMA (global_load_lds, no
//     registers), nbuf - 1 tiles ahead; one copy moves 512 contiguous bytes of
//     two rows, so every row is read in long runs;
//   * the 4 waves split the part's blocks of a tile (block b -> wave b % 4),
//     read the MFMA fragments from LDS, convert fp8 -> bf16 in registers and
//     sum their partial tiles through LDS in wave order.
// With one K part the sums go through the epilogue (deferred to the end of the
// unit: one round of epilogue loads), otherwise into fp32 partials
// [part][M][N] that gemv_finish sums in part order (deterministic, no atomics,
// no workgroup depends on another).
//
// Weight tile layout in LDS: segment s (512 B of K) of row pair i (rows 2i,
// 2i+1) is one 1 KB DMA copy at ((s * 8 + i) * 1024); row 2i+j's half at +512j;
// inside a row's 512 B, 16 B chunk c sits at (c & ~7) | ((c ^ row) & 7), so the
// 16 rows of a fragment read hit distinct banks.
// MFMA K order inside a 128-wide block: lane (row l%16, group g = l/16) holds
// weight chunks g and 4+g (bytes 16g.., 64+16g..) = K slots 0-7, 8-15 (first
// chunk) and 64.., 72.. (second); x fragments follow the same order.
constexpr int GEMV_MAX_RG = 16;     // 16-row tiles per workgroup
constexpr int GEMV_KPB = 16;        // max 128-wide blocks per K part (2 KB of a row)
// Weight tiles resident: nbuf (current + nbuf - 1 in flight).  Measured on
// MI355X (decode shapes at M = 8, the FFN and MoE blocks): keeping about
// 32 KB of copies in flight per workgroup is fastest, deeper rings are
// slower (o_proj 32 KB tiles: ring 3 31.1 us, 4 32.2; q_b 24 KB tiles: ring 2
// 14.2, 3 15.0, 4 15.5; q_a | kv_a 16 KB tiles: 15.6 / 16.6 / 16.9; the MoE
// block 16 % faster with 2 or 3 than with 4).
__host__ __device__ inline int gemv_nbuf(int tile_bytes) { return tile_bytes >= 32 * 1024 ? 3 : 2; }

// LDS: [nbuf][16 rows][ceil4(kpb) * 128] weights |
//      [2][4 waves][MT][64] f32x4 partial tiles | [rg][MT][64] f32x4 results
// (not for 64-row x with K parts: there every thread of the workgroup holds
// one fp32 sum of a reduced tile and stores it at once, so long units take no
// more LDS).
// x is held in registers: each wave's fragments of the MT 16-row tiles,
// loaded once per workgroup (16 VGPRs per tile and 128-wide block of the
// wave: a K part of up to 16 blocks for MT <= 2 (128 VGPRs), 12 for MT = 4
// (192 VGPRs, so that K = 1536 needs no K parts at 64 rows)).
__host__ __device__ constexpr int gemv_kpb_max(int MT) { return MT == 4 ? 12 : GEMV_KPB; }
__host__ __device__ inline int gemv_kpb4(int kpb) { return (kpb + 3) & ~3; }

template <int MT, int MODE>
AMLA_DEV void gemv_body(const GemvParams &p, int unit, int rg, int kparts, int kpb) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int KB = p.K >> 7;
  const int ntiles = p.N >> 4;
  const int part = unit % kparts;
  const int tile_begin = (unit / kparts) * rg;
  const int tile_end = min(tile_begin + rg, ntiles);
  const int kb_begin = part * kpb;
  const int nbp = min(kpb, KB - kb_begin);  // blocks of this part
  const int nseg = (nbp + 3) >> 2;          // 512 B segments per row
  const int TILE_BYTES = 16 * gemv_kpb4(kpb) * 128;
  const int nbuf = gemv_nbuf(TILE_BYTES);

  extern __shared__ __align__(16) uint8_t gsm[];
  uint8_t *const wbuf = gsm;
  f32x4 *const red = reinterpret_cast<f32x4 *>(gsm + nbuf * TILE_BYTES);
  f32x4 *const done = red + 2 * 4 * MT * 64;

  // weight copies of one tile: row pairs i = 2*wave, 2*wave+1, every segment
  auto dma_tile = [&](int tile, int buf) {
    const int nt = min(tile, tile_end - 1) * 16;
    const bool seg1 = (MODE == GEMV_QKVA || p.w1) && nt >= p.n_split;
    const uint8_t *wb = (seg1 ? p.w1 : p.w0) + (size_t)(seg1 ? nt - p.n_split : nt) * p.K;
    uint8_t *tb = wbuf + buf * TILE_BYTES;
    for (int s = 0; s < nseg; ++s) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const int i = wave * 2 + ii;
        const int row = 2 * i + (lane >> 5);
        const int cl = lane & 31;                                 // LDS chunk in the row's 512 B
        const int cg = (cl & ~7) | ((cl ^ row) & 7);              // global chunk stored there
        const int kb = min(kb_begin + s * 4 + (cg >> 3), KB - 1);  // 128 B block (clamped: unused)
        const uint32_t off = (uint32_t)(row * p.K + kb * 128 + (cg & 7) * 16);
        // non-temporal (aux 2): each weight byte is read once per call
        __builtin_amdgcn_global_load_lds(wb + off, (__attribute__((address_space(3))) void *)(tb + (s * 8 + i) * 1024),
                                         16, 0, 2);
      }
    }
  };
  // LDS-only barrier: __syncthreads would also wait for every copy in flight
  auto lds_barrier = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // the first weight tiles are in flight while x is read
  if (tile_begin < tile_end) {
#pragma unroll
    for (int b = 0; b < nbuf - 1; ++b) dma_tile(tile_begin + b, b);
  }

  // this wave's x fragments (blocks wave + 4j of the part, rows 16t + li;
  // rows >= M are zeros), in the MFMA K order of the weight fragments below
  constexpr int NJ = gemv_kpb_max(MT) / 4;
  u32x4 xr[MT][NJ][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bl = wave + 4 * j, m = 16 * t + li;
      const bool ok = bl < nbp && m < p.M;
      const uint16_t *xp = p.x + (size_t)m * p.ldx + (size_t)(kb_begin + bl) * 128 + lg * 16;
#pragma unroll
      for (int q = 0; q < 4; ++q) xr[t][j][q] = ok ? ldg16(xp + (q & 1) * 8 + (q >> 1) * 64) : u32x4{0, 0, 0, 0};
    }
  if (p.xg) {  // input bf16(x * g) per column (the input RMSNorm's gamma; its row factor is applied by the finish)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bl = wave + 4 * j;
      if (bl < nbp) {
        const uint16_t *gp = p.xg + (size_t)(kb_begin + bl) * 128 + lg * 16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 g = ldg16(gp + (q & 1) * 8 + (q >> 1) * 64);
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              xr[t][j][q][e] = pack_bf16(lo_bf(xr[t][j][q][e]) * lo_bf(g[e]), hi_bf(xr[t][j][q][e]) * hi_bf(g[e]));
        }
      }
    }
  }

  for (int tile = tile_begin, it = 0, buf = 0; tile < tile_end; ++tile, ++it, buf = buf == nbuf - 1 ? 0 : buf + 1) {
    const int nt = tile * 16;
    // block scales of this wave's blocks through the scalar cache (constant
    // address space: the scales are never written here), so waiting for them
    // is not waiting for the weight copies in flight
    const bool seg1 = (MODE == GEMV_QKVA || p.w1) && nt >= p.n_split;
    const __attribute__((address_space(4))) float *srow =
        (const __attribute__((address_space(4))) float *)((seg1 ? p.s1 : p.s0) +
                                                          (size_t)((seg1 ? nt - p.n_split : nt) >> 7) * KB + kb_begin);
    float scw[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) scw[j] = srow[min(wave + 4 * j, nbp - 1)];
    // this tile's copies landed (the next nbuf - 2 tiles' may stay in flight:
    // 2 * nseg copies per wave per tile), then every wave's part of it is visible
    if (nbuf == 3) {
      if (nseg == 4) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else if (nseg == 3) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
      else if (nseg == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    lds_barrier();
    dma_tile(tile + nbuf - 1, buf == 0 ? nbuf - 1 : buf - 1);  // into the buffer read last trip

    const uint8_t *tb = wbuf + buf * TILE_BYTES;
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bl = wave + 4 * j;
      if (bl < nbp) {
        const int s = bl >> 2, bq = bl & 3;  // segment, block inside it
        const uint8_t *rp = tb + (s * 8 + (li >> 1)) * 1024 + (li & 1) * 512;
        const u32x4 w0 = *reinterpret_cast<const u32x4 *>(rp + ((bq * 8) | ((lg ^ li) & 7)) * 16);
        const u32x4 w1 = *reinterpret_cast<const u32x4 *>(rp + ((bq * 8) | (((4 + lg) ^ li) & 7)) * 16);
        bf16x8 a0, a1, a2, a3;
        fp8x16_to_bf16x16(w0, a0, a1);
        fp8x16_to_bf16x16(w1, a2, a3);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
          c = mfma16(a0, as_bf16x8(xr[t][j][0]), c);
          c = mfma16(a1, as_bf16x8(xr[t][j][1]), c);
          c = mfma16(a2, as_bf16x8(xr[t][j][2]), c);
          c = mfma16(a3, as_bf16x8(xr[t][j][3]), c);
          acc[t] += scw[j] * c;
        }
      }
    }
    f32x4 *rb = red + (it & 1) * 4 * MT * 64;
#pragma unroll
    for (int t = 0; t < MT; ++t) rb[(wave * MT + t) * 64 + lane] = acc[t];
    lds_barrier();
    for (int idx = tid; idx < MT * 64; idx += 256) {
      const int t = idx >> 6, ln = idx & 63;
      f32x4 v = rb[(0 * MT + t) * 64 + ln];
      v += rb[(1 * MT + t) * 64 + ln];
      v += rb[(2 * MT + t) * 64 + ln];
      v += rb[(3 * MT + t) * 64 + ln];
      if (MT < 4 || kparts == 1) {
        done[(it * MT + t) * 64 + ln] = v;
      } else {  // 64-row x, K parts: every thread holds one fp32 sum of the tile, stored at once (no LDS held)
        const int m = t * 16 + (ln & 15);
        if (m < p.M) *reinterpret_cast<f32x4 *>(p.part + ((size_t)part * p.M + m) * p.N + nt + 4 * (ln >> 4)) = v;
      }
    }
    // red[it & 1] is rewritten two tiles later, after the next two barriers
  }
  lds_barrier();
  // results of the unit: epilogue (one K part) or fp32 partial sums (64-row
  // x with K parts stored them per tile)
  const int nitems = MT < 4 || kparts == 1 ? (tile_end - tile_begin) * MT * 64 : 0;
  for (int idx = tid; idx < nitems; idx += 256) {
    const int tl = idx / (MT * 64), t = (idx >> 6) % MT, ln = idx & 63;
    const int m = t * 16 + (ln & 15);
    const int n = (tile_begin + tl) * 16 + 4 * (ln >> 4);
    if (m >= p.M) continue;
    const f32x4 v = done[(tl * MT + t) * 64 + ln];
    if (kparts == 1) store4<MODE>(p, m, n, v);
    else *reinterpret_cast<f32x4 *>(p.part + ((size_t)part * p.M + m) * p.N + n) = v;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last trips' (unused) copies land before exit
}

template <int MT, int MODE>
__global__ __launch_bounds__(256, 2) void gemv_kernel(GemvParams p, int rg, int kparts, int kpb) {
  gemv_body<MT, MODE>(p, blockIdx.x, rg, kparts, kpb);
}

// Several independent skinny GEMMs of one shape (N, K) in one launch: group g
// takes workgroups [g * units, (g + 1) * units) with its own x, weights, M,
// output and partial-sum buffer (routed experts of a MoE layer).
template <int MT>
__global__ __launch_bounds__(256, 2) void gemv_grouped_kernel(GemvParams p, GemvGroups gr, int rg, int kparts, int kpb) {
  const int g = blockIdx.x / gr.units;
  GemvParams q = p;
  q.x = gr.g[g].x;
  q.w0 = gr.g[g].w0;
  q.s0 = gr.g[g].s0;
  q.w1 = gr.g[g].w1;
  q.s1 = gr.g[g].s1;
  q.y = gr.g[g].y;
  q.part = gr.g[g].part;
  q.M = gr.g[g].M;
  gemv_body<MT, GEMV_PLAIN>(q, blockIdx.x % gr.units, rg, kparts, kpb);
}

size_t gemv_lds_bytes(int MT, int kpb, int rg, int kparts) {
  const int tile = 16 * gemv_kpb4(kpb) * 128;
  return (size_t)gemv_nbuf(tile) * tile + 2 * 4 * MT * 64 * 16 +
         (MT < 4 || kparts == 1 ? (size_t)rg * MT * 64 * 16 : 0);
}

// Sums the K parts of gemv_kernel in part order and applies the epilogue.
// All parts are loaded before the first add (independent loads in flight).
template <int MODE>
AMLA_DEV void gemv_finish_body(const GemvParams &p, int64_t i, int kparts) {
  const int64_t total = (int64_t)p.M * (p.N >> 2);
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

template <int MODE>
__global__ __launch_bounds__(64) void gemv_finish(GemvParams p, int kparts) {
  gemv_finish_body<MODE>(p, (int64_t)blockIdx.x * 64 + threadIdx.x, kparts);
}

// gemv_finish for the groups of gemv_grouped_kernel: gr.units blocks per group.
__global__ __launch_bounds__(64) void gemv_finish_grouped(GemvParams p, GemvGroups gr, int kparts) {
  const int g = blockIdx.x / gr.units;
  GemvParams q = p;
  q.y = gr.g[g].y;
  q.part = gr.g[g].part;
  q.M = gr.g[g].M;
  gemv_finish_body<GEMV_PLAIN>(q, (int64_t)(blockIdx.x % gr.units) * 64 + threadIdx.x, kparts);
}

// Skinny GEMMs of a device schedule (routed experts): entry g = blockIdx.x /
// units; entries past the device count return at once (uniform per workgroup).
template <int MT>
__global__ __launch_bounds__(256, 2) void gemv_sched_kernel(GemvParams p, MoeSched s, int units, int rg, int kparts,
                                                         int kpb) {
  const int g = blockIdx.x / units;
  if (g >= *s.count) return;
  const int32_t *en = s.ent + 4 * g;
  const int e = en[0], r0 = en[1];
  p.M = en[2];
  p.x += (size_t)r0 * p.ldx;
  p.y += (size_t)r0 * p.ldy;
  p.part += (size_t)kparts * r0 * p.N;
  moe_sched_weights(p, s, e);
  gemv_body<MT, GEMV_PLAIN>(p, blockIdx.x % units, rg, kparts, kpb);
}

// gemv_finish for the entries of gemv_sched_kernel: units blocks of 64 per entry.
__global__ __launch_bounds__(64) void gemv_finish_sched(GemvParams p, MoeSched s, int units, int kparts) {
  const int g = blockIdx.x / units;
  if (g >= *s.count) return;
  const int32_t *en = s.ent + 4 * g;
  const int r0 = en[1];
  p.M = en[2];
  p.y += (size_t)r0 * p.ldy;
  p.part += (size_t)kparts * r0 * p.N;
  gemv_finish_body<GEMV_PLAIN>(p, (int64_t)(blockIdx.x % units) * 64 + threadIdx.x, kparts);
}

// One workgroup per row m: sums the K parts of every output of the row in
// part order, stores the kv_a columns (n >= n_split) into the caches, and
// normalises the bf16 q_a columns: r = rsqrt(mean(q_a^2) + eps),
// y = bf16(bf16(q_a * r) * gamma)  (inference/ops.py:10-12, :130).
constexpr int QKVA_FIN_MAXG = 3;  // float4 groups per thread: N <= 3 * 4 * 256
constexpr int QKVA_FIN_MAXX = 4;  // 16-byte chunks of the raw input row per thread: K <= 4 * 8 * 256
__global__ __launch_bounds__(256) void qkva_finish_norm_kernel(GemvParams p, int kparts, const uint16_t *gamma,
                                                               float eps, const uint16_t *x_raw, float eps_in) {
  const int m = blockIdx.x, tid = threadIdx.x;
  const int ng = p.N >> 2;
  f32x4 v[QKVA_FIN_MAXG];
  float ss = 0.f;
  // the raw input row's sum of squares (input RMSNorm, inference/forward.py:92): its loads go out first
  u32x4 xv[QKVA_FIN_MAXX];
  if (x_raw) {
#pragma unroll
    for (int i = 0; i < QKVA_FIN_MAXX; ++i) {
      const int c = tid + 256 * i;
      xv[i] = c < (p.K >> 3) ? ldg16(x_raw + (size_t)m * p.ldx + c * 8) : u32x4{0, 0, 0, 0};
    }
  }
  // every part of every group in flight before the first add (parts in
  // batches of 8)
  f32x4 s[QKVA_FIN_MAXG];
#pragma unroll
  for (int i = 0; i < QKVA_FIN_MAXG; ++i) s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int q0 = 0; q0 < kparts; q0 += 8) {
    f32x4 t[QKVA_FIN_MAXG][8];
#pragma unroll
    for (int i = 0; i < QKVA_FIN_MAXG; ++i) {
      const int g = tid + 256 * i;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        t[i][q] = (g < ng && q0 + q < kparts)
                      ? *reinterpret_cast<const f32x4 *>(p.part + ((size_t)(q0 + q) * p.M + m) * p.N + 4 * g)
                      : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < QKVA_FIN_MAXG; ++i)
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (q0 + q < kparts) s[i] += t[i][q];  // part order
  }
  __shared__ float part[4];
  __shared__ float partx[4];
  if (x_raw) {
    // r_in = rsqrt(mean(x^2) + eps_in): the GEMM summed W . bf16(x * gamma_in), so each sum times r_in
    // is the projection of the normed input (rounded once, to bf16(x * gamma_in), instead of twice)
    float sx = 0.f;
#pragma unroll
    for (int i = 0; i < QKVA_FIN_MAXX; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) sx += lo_bf(xv[i][e]) * lo_bf(xv[i][e]) + hi_bf(xv[i][e]) * hi_bf(xv[i][e]);
    sx = wave_sum(sx);
    if ((tid & 63) == 0) partx[tid >> 6] = sx;
    __syncthreads();
    const float rin = rsqrtf(((partx[0] + partx[1]) + (partx[2] + partx[3])) / (float)p.K + eps_in);
#pragma unroll
    for (int i = 0; i < QKVA_FIN_MAXG; ++i) s[i] *= rin;
  }
#pragma unroll
  for (int i = 0; i < QKVA_FIN_MAXG; ++i) {
    const int g = tid + 256 * i;
    v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (g < ng) {
      if (4 * g >= p.n_split) {
        store4<GEMV_QKVA>(p, m, 4 * g, s[i]);
      } else {
        v[i] = f32x4{round_bf16(s[i].x), round_bf16(s[i].y), round_bf16(s[i].z), round_bf16(s[i].w)};  // q_a as stored (bf16)
        ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
      }
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float r = __builtin_amdgcn_rsqf(((part[0] + part[1]) + (part[2] + part[3])) / (float)p.n_split + eps);
#pragma unroll
  for (int i = 0; i < QKVA_FIN_MAXG; ++i) {
    const int n = 4 * (tid + 256 * i);
    if (n < p.n_split) {
      const u32x2 gm = *reinterpret_cast<const u32x2 *>(gamma + n);
      const u32x2 o = {pack_bf16(round_bf16(v[i].x * r) * lo_bf(gm.x), round_bf16(v[i].y * r) * hi_bf(gm.x)),
                       pack_bf16(round_bf16(v[i].z * r) * lo_bf(gm.y), round_bf16(v[i].w * r) * hi_bf(gm.y))};
      *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
    }
  }
}

int launch_qkva_finish_norm(const GemvParams &p, int kparts, const uint16_t *gamma, float eps, hipStream_t st,
                            const uint16_t *x_raw, float eps_in) {
  if (p.N > QKVA_FIN_MAXG * 4 * 256 || p.N % 4 || p.n_split % 4)
    return fail(AMLA_EUNSUPPORTED, "q_a/kv_a finish: N=%d exceeds %d or is not a multiple of 4", p.N,
                QKVA_FIN_MAXG * 4 * 256);
  if (x_raw && (p.K > QKVA_FIN_MAXX * 8 * 256 || p.K % 8 || p.ldx % 8 || !aligned16(x_raw)))
    return fail(AMLA_EUNSUPPORTED, "q_a/kv_a finish: input row of %d is not foldable", p.K);
  qkva_finish_norm_kernel<<<dim3((unsigned)p.M), 256, 0, st>>>(p, kparts, gamma, eps, x_raw, eps_in);
  return check_launch("q_a/kv_a finish");
}

GemvPlan plan_gemv(int M, int N, int K) {
  GemvPlan pl = {};
  const int tiles = N / 16;
  const int KB = K / 128;
  const int MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  // K part: whole K when it fits (no finishing pass), else the largest block
  // count <= gemv_kpb_max(MT) (multiple of 4) that splits K into equal parts;
  // both within the LDS budget with one tile per unit
  constexpr size_t LDS_MAX = 160 * 1024;
  // rows of K >= 2048 (o_proj, the FFN and expert projections) take 16 KB
  // tiles (more K parts, two workgroups per CU): measured faster than 32 KB
  int kmax = K >= 2048 && MT < 4 ? 8 : gemv_kpb_max(MT);
  while (kmax > 4 && gemv_lds_bytes(MT, kmax, 1, 1) > LDS_MAX) kmax -= 4;
  int kpb = KB <= kmax ? KB : 0;
  if (!kpb) {
    for (int c = kmax; c >= 4; c -= 4)
      if (KB % c == 0) { kpb = c; break; }
    if (!kpb) kpb = kmax;
  }
  pl.kpb = kpb;
  pl.kparts = (KB + kpb - 1) / kpb;
  // tiles per unit: fewest rounds of the workgroups the machine holds (256,
  // or 512 when two fit one CU's LDS: measured faster for q_a | kv_a and q_b,
  // whose units then run two per CU) x (tiles per unit + the per-workgroup
  // start-up: one tile's worth, four for 64-row x, whose fragments are eight
  // weight tiles' worth of bytes), then the largest unit (fewer x stagings),
  // within the LDS budget
  const int startup = MT == 4 ? 4 : 1;
  int best_rg = 1;
  int64_t best_cost = INT64_MAX;
  for (int rg = 1; rg <= GEMV_MAX_RG; ++rg) {
    if (gemv_lds_bytes(MT, kpb, rg, pl.kparts) > LDS_MAX) break;
    const int64_t units = (int64_t)((tiles + rg - 1) / rg) * pl.kparts;
    const int64_t slots = 256 * std::min<int64_t>(2, LDS_MAX / gemv_lds_bytes(MT, kpb, rg, pl.kparts));
    const int64_t cost = ((units + slots - 1) / slots) * (rg + startup);
    if (cost <= best_cost) {
      best_cost = cost;
      best_rg = rg;
    }
  }
  pl.rg = best_rg;
  pl.groups = ((tiles + pl.rg - 1) / pl.rg) * pl.kparts;
  pl.lds = gemv_lds_bytes(MT, kpb, pl.rg, pl.kparts);
  pl.part_bytes = pl.kparts > 1 ? (size_t)pl.kparts * M * N * 4 : 0;
  return pl;
}

GemvPlan plan_gemv_grouped(int M, int N, int K) {
  // many groups fill the machine by themselves: take the longest row run per
  // workgroup the LDS allows (fewer, longer weight streams)
  GemvPlan pl = plan_gemv(M, N, K);
  const int MT = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int tiles = N / 16;
  int rg = std::min(GEMV_MAX_RG, tiles);
  while (rg > pl.rg && gemv_lds_bytes(MT, pl.kpb, rg, pl.kparts) > 160 * 1024) --rg;
  if (rg > pl.rg) {
    pl.rg = rg;
    pl.groups = ((tiles + rg - 1) / rg) * pl.kparts;
    pl.lds = gemv_lds_bytes(MT, pl.kpb, rg, pl.kparts);
  }
  return pl;
}

// ---------------------------------------------------------------- streaming GEMV, one row of x

// With one row of x the MFMA tiles above use 1/16 of their columns and the
// weight stream pays for LDS staging, barriers and K-part partial sums.  Here
// a workgroup (256 threads) owns a run of rpw consecutive weight rows over the
// whole K and streams them straight into registers, VG_R rows at a time:
//   * thread t takes the 16-byte fp8 chunks t, t + 256, .. (NCH of them) of
//     every row (one contiguous 1 KB span per wave and row);
//   * two groups of VG_R rows are in flight: the loads of the next group are
//     issued before the current one is computed (a register double buffer,
//     the loop unrolled by two so that both buffers are named statically and
//     the compiler's load counters stay exact);
//   * the loads carry the non-temporal hint: every weight byte is read once
//     per call, and streaming it past the caches measured 10 % faster;
//   * each chunk is converted exactly to bf16 pairs and dotted with the
//     thread's x chunk in fp32 (v_dot2_f32_bf16), then scaled by its 128x128
//     block's scale_inv (a chunk never straddles a block), like the MFMA path;
//   * every row reduces over its wave by lane swaps; the four waves' sums meet
//     in LDS once at the end, and rpw / 4 threads store four rows each through
//     the GEMV epilogue (store4), so no finishing pass is needed.
// A persistent grid of about 512 workgroups (two per CU) keeps the stream
// going: the one-shot form (a workgroup per 8 rows, 1.75 rounds of the
// machine for o_proj) measured 26.2 us against 19.4 for this one (M = 1,
// N = 7168, K = 16384) and 7.0 against 5.2 us for q_a | kv_a (N = 2112,
// K = 7168), bit-identical results (same chunks, same order per row).
// Optional input RMSNorm (p.xnorm): the workgroup holds the whole x row, so
// it normalises it exactly as rms_norm does (bf16(bf16(x * r) * xg), r =
// rsqrt(mean(x^2) + eps_in), one LDS-only barrier) while the first weight
// group is in flight.
constexpr int VG_R = 2;          // rows per group (a divisor of 128: a group never straddles a scale block)
constexpr int VG_MAX_RPW = 64;   // rows per workgroup (the LDS reduction buffer)
constexpr int VG_GRID = 512;     // target workgroups

template <int CTRL>
AMLA_DEV float vg_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// sum over the 64 lanes of a wave, in every lane
AMLA_DEV float vg_sum64(float v) {
  v += vg_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += vg_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += vg_dpp<0x141>(v);  // row_half_mirror
  v += vg_dpp<0x140>(v);  // row_mirror
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// rows [blockIdx.x * rpw, + rpw) (rpw a multiple of 2 VG_R and of 4); rows
// past N re-read the last group of the matrix (in bounds) and are not stored
template <int NCH, int MODE>
__global__ __launch_bounds__(256, 2) void vgemv_kernel(GemvParams p, int rpw) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = blockIdx.x * rpw;
  const int C = p.K >> 4;  // 16-byte chunks per weight row
  const int KB = p.K >> 7;
  // epilogue operands of this thread's four rows (threads past them load the
  // run's last four, in bounds)
  const int en = min(nb + min(4 * tid, rpw - 4), p.N - 4);
  EpiOps eo = {};
  epi_load1<MODE>(p, 0, en, eo);

  // this thread's chunks of x (16 bf16 each) and of xg, loaded before the
  // weights so that waiting for them does not wait for the weight loads
  u32x4 xa[NCH][2], ga[NCH][2];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = tid + 256 * j;
    const bool ok = c < C;
    xa[j][0] = ok ? ldg16(p.x + c * 16) : u32x4{0, 0, 0, 0};
    xa[j][1] = ok ? ldg16(p.x + c * 16 + 8) : u32x4{0, 0, 0, 0};
    ga[j][0] = ok && p.xg ? ldg16(p.xg + c * 16) : u32x4{0, 0, 0, 0};
    ga[j][1] = ok && p.xg ? ldg16(p.xg + c * 16 + 8) : u32x4{0, 0, 0, 0};
  }

  __shared__ float red[4][VG_MAX_RPW];
  __shared__ float xss[4];
  u32x4 wa[VG_R][NCH], wb[VG_R][NCH];
  float sa[NCH], sb[NCH];
  // the weight chunks and block scales of the group at row n0
  auto load = [&](u32x4 (&W)[VG_R][NCH], float (&S)[NCH], int n0) __attribute__((always_inline)) {
    const int n = min(n0, p.N - VG_R);
    const bool seg1 = (MODE == GEMV_QKVA || p.w1) && n >= p.n_split;
    const int r0 = seg1 ? n - p.n_split : n;
    const uint8_t *wp = (seg1 ? p.w1 : p.w0) + (size_t)r0 * p.K;
    const float *sp = (seg1 ? p.s1 : p.s0) + (size_t)(r0 >> 7) * KB;
#pragma unroll
    for (int r = 0; r < VG_R; ++r)
#pragma unroll
      for (int j = 0; j < NCH; ++j) W[r][j] = ldg16_nt(wp + (size_t)r * p.K + min(tid + 256 * j, C - 1) * 16);
#pragma unroll
    for (int j = 0; j < NCH; ++j) S[j] = sp[min(tid + 256 * j, C - 1) >> 3];
  };
  // this wave's sums of the group's rows into red[wave][row - nb]
  auto compute = [&](const u32x4 (&W)[VG_R][NCH], const float (&S)[NCH], int i0) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < VG_R; ++r) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        if (tid + 256 * j >= C) continue;  // past the row (x chunks are zero there too)
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16x2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(W[r][j][e], 1.f, false);
          const bf16x2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(W[r][j][e], 1.f, true);
          // bytes 4e .. 4e+3 of the chunk are elements 4e .. 4e+3: x pairs (4e, 4e+1), (4e+2, 4e+3)
          const uint32_t x01 = xa[j][e >> 1][(e & 1) * 2], x23 = xa[j][e >> 1][(e & 1) * 2 + 1];
          d = __builtin_amdgcn_fdot2_f32_bf16(w01, __builtin_bit_cast(bf16x2_t, x01), d, false);
          d = __builtin_amdgcn_fdot2_f32_bf16(w23, __builtin_bit_cast(bf16x2_t, x23), d, false);
        }
        a = __builtin_fmaf(S[j], d, a);
      }
      a = vg_sum64(a);
      if (lane == 0) red[wave][i0 + r] = a;
    }
  };
  const int ng = rpw / VG_R;  // even, >= 2
  load(wa, sa, nb);  // in flight while x is prepared
  epi_load2<MODE>(p, 0, en, eo);
  if (p.xnorm) {
    // rms_norm(x, xg, eps_in) of the whole row (inference/ops.py:10-12), as
    // the row-norm kernel computes it; the barrier is LDS-only, so the weight
    // loads above stay in flight
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ss += lo_bf(xa[j][h][e]) * lo_bf(xa[j][h][e]) + hi_bf(xa[j][h][e]) * hi_bf(xa[j][h][e]);
    ss = vg_sum64(ss);
    if (lane == 0) xss[wave] = ss;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const float r = rsqrtf(((xss[0] + xss[1]) + (xss[2] + xss[3])) / (float)p.K + p.eps_in);
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xa[j][h][e] = pack_bf16(round_bf16(lo_bf(xa[j][h][e]) * r) * lo_bf(ga[j][h][e]),
                                  round_bf16(hi_bf(xa[j][h][e]) * r) * hi_bf(ga[j][h][e]));
  } else if (p.xg) {  // the GEMM takes bf16(x * xg)
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xa[j][h][e] = pack_bf16(lo_bf(xa[j][h][e]) * lo_bf(ga[j][h][e]), hi_bf(xa[j][h][e]) * hi_bf(ga[j][h][e]));
  }
  for (int g = 0; g < ng - 2; g += 2) {
    load(wb, sb, nb + (g + 1) * VG_R);
    compute(wa, sa, g * VG_R);
    load(wa, sa, nb + (g + 2) * VG_R);
    compute(wb, sb, (g + 1) * VG_R);
  }
  load(wb, sb, nb + (ng - 1) * VG_R);
  compute(wa, sa, (ng - 2) * VG_R);
  compute(wb, sb, (ng - 1) * VG_R);

  __syncthreads();
  if (4 * tid < rpw && nb + 4 * tid < p.N) {  // N % 8 == 0: four rows are all in range or all past N
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * tid + i;
      v[i] = (red[0][r] + red[1][r]) + (red[2][r] + red[3][r]);
    }
    store4e<MODE>(p, 0, nb + 4 * tid, v, eo);
  }
}

// Short rows (K = 1536, the q_b projection: 96 chunks of 16 bytes, too few
// for 256 threads per row): each wave streams its own rows, VGS_S = 2 rows
// (192 chunks, 3 KB contiguous) per span, lane l taking the span's chunks
// l, l + 64, l + 128, and VGS_G spans per group, two groups in flight; the
// rows reduce inside the wave and meet in LDS only for the epilogue's
// four-row stores.  Each span's rows share one 128-row scale block.
constexpr int VGS_C = 96;                    // chunks per row (K = 1536)
constexpr int VGS_S = 2;                     // rows per span
constexpr int VGS_CPL = VGS_S * VGS_C / 64;  // chunks per lane per span
constexpr int VGS_G = 3;                     // spans per group
constexpr int VGS_RPW = 4 * 2 * VGS_G * VGS_S;  // rows per workgroup: 4 waves x 2 groups

template <int MODE>
__global__ __launch_bounds__(256, 2) void vgemv_short_kernel(GemvParams p) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = blockIdx.x * VGS_RPW + wave * (VGS_RPW / 4);  // this wave's first row
  const int KB = p.K >> 7;
  // epilogue operands of this thread's four rows (threads past them load the
  // workgroup's last four, in bounds)
  const int en = min(blockIdx.x * VGS_RPW + min(4 * tid, VGS_RPW - 4), p.N - 4);
  EpiOps eo = {};
  epi_load1<MODE>(p, 0, en, eo);
  // span chunk i of this lane: row ri[i] of the span, column chunk ci[i]
  int ri[VGS_CPL], ci[VGS_CPL];
#pragma unroll
  for (int i = 0; i < VGS_CPL; ++i) {
    ri[i] = (lane + 64 * i) / VGS_C;
    ci[i] = (lane + 64 * i) % VGS_C;
  }
  u32x4 xa[VGS_CPL][2], ga[VGS_CPL][2];  // x and xg chunks, loaded before the weights
#pragma unroll
  for (int i = 0; i < VGS_CPL; ++i) {
    xa[i][0] = ldg16(p.x + ci[i] * 16);
    xa[i][1] = ldg16(p.x + ci[i] * 16 + 8);
    ga[i][0] = p.xg ? ldg16(p.xg + ci[i] * 16) : u32x4{0, 0, 0, 0};
    ga[i][1] = p.xg ? ldg16(p.xg + ci[i] * 16 + 8) : u32x4{0, 0, 0, 0};
  }
  // block scales of the lane's columns in the (at most two) 128-row blocks of the wave's rows
  const int blk0 = nw >> 7;
  float sc0[VGS_CPL], sc1[VGS_CPL];
  {
    const int blk1 = min((nw + VGS_RPW / 4 - 1) >> 7, (p.N - 1) >> 7);
#pragma unroll
    for (int i = 0; i < VGS_CPL; ++i) {
      sc0[i] = p.s0[(size_t)min(blk0, (p.N - 1) >> 7) * KB + (ci[i] >> 3)];
      sc1[i] = p.s0[(size_t)blk1 * KB + (ci[i] >> 3)];
    }
  }

  __shared__ float red[VGS_RPW];
  u32x4 wa[VGS_G][VGS_CPL], wb[VGS_G][VGS_CPL];
  auto load = [&](u32x4 (&W)[VGS_G][VGS_CPL], int n0) __attribute__((always_inline)) {
#pragma unroll
    for (int sp = 0; sp < VGS_G; ++sp) {
      const int n = min(n0 + sp * VGS_S, p.N - VGS_S);  // rows past N re-read the last span (not stored)
      const uint8_t *wp = p.w0 + (size_t)n * p.K;
#pragma unroll
      for (int i = 0; i < VGS_CPL; ++i) W[sp][i] = ldg16_nt(wp + (lane + 64 * i) * 16);
    }
  };
  auto compute = [&](const u32x4 (&W)[VGS_G][VGS_CPL], int n0) __attribute__((always_inline)) {
#pragma unroll
    for (int sp = 0; sp < VGS_G; ++sp) {
      const bool second = ((n0 + sp * VGS_S) >> 7) != blk0;  // wave-uniform
      float a[VGS_S] = {};
#pragma unroll
      for (int i = 0; i < VGS_CPL; ++i) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16x2_t w01 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(W[sp][i][e], 1.f, false);
          const bf16x2_t w23 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(W[sp][i][e], 1.f, true);
          const uint32_t x01 = xa[i][e >> 1][(e & 1) * 2], x23 = xa[i][e >> 1][(e & 1) * 2 + 1];
          d = __builtin_amdgcn_fdot2_f32_bf16(w01, __builtin_bit_cast(bf16x2_t, x01), d, false);
          d = __builtin_amdgcn_fdot2_f32_bf16(w23, __builtin_bit_cast(bf16x2_t, x23), d, false);
        }
        const float v = (second ? sc1[i] : sc0[i]) * d;
#pragma unroll
        for (int r = 0; r < VGS_S; ++r) a[r] += ri[i] == r ? v : 0.f;
      }
#pragma unroll
      for (int r = 0; r < VGS_S; ++r) {
        const float t = vg_sum64(a[r]);
        if (lane == 0) red[n0 + sp * VGS_S + r - blockIdx.x * VGS_RPW] = t;
      }
    }
  };
  load(wa, nw);
  load(wb, nw + VGS_G * VGS_S);
  epi_load2<MODE>(p, 0, en, eo);
  // x prepared while the weights are in flight: rms_norm(x, xg, eps_in) of
  // the whole row (inference/ops.py:10-12; each wave holds every column
  // chunk, the span's first row once), or bf16(x * xg)
  if (p.xnorm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VGS_CPL; ++i)
      if (ri[i] == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            ss += lo_bf(xa[i][h][e]) * lo_bf(xa[i][h][e]) + hi_bf(xa[i][h][e]) * hi_bf(xa[i][h][e]);
      }
    const float r = rsqrtf(vg_sum64(ss) / (float)p.K + p.eps_in);
#pragma unroll
    for (int i = 0; i < VGS_CPL; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xa[i][h][e] = pack_bf16(round_bf16(lo_bf(xa[i][h][e]) * r) * lo_bf(ga[i][h][e]),
                                  round_bf16(hi_bf(xa[i][h][e]) * r) * hi_bf(ga[i][h][e]));
  } else if (p.xg) {
#pragma unroll
    for (int i = 0; i < VGS_CPL; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xa[i][h][e] = pack_bf16(lo_bf(xa[i][h][e]) * lo_bf(ga[i][h][e]), hi_bf(xa[i][h][e]) * hi_bf(ga[i][h][e]));
  }
  compute(wa, nw);
  compute(wb, nw + VGS_G * VGS_S);
  __syncthreads();
  const int nb = blockIdx.x * VGS_RPW;
  if (4 * tid < VGS_RPW && nb + 4 * tid < p.N) {
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = red[4 * tid + i];
    store4e<MODE>(p, 0, nb + 4 * tid, v, eo);
  }
}

// ---------------------------------------------------------------- streaming GEMV, 2 .. 8 rows of x

// With a few rows of x (decode batches of 2 .. 8) the skinny GEMM above stages
// the weights through LDS and holds x in registers, which bounds a K part to
// 1024 columns and needs a finishing pass over fp32 partial sums.  Here the
// roles swap: x sits in LDS and the weights stream straight into registers in
// MFMA fragment order, so every workgroup covers the whole K of its rows.
//   * one workgroup per CU (8 waves) owns a run of rpw rows (a multiple of 4,
//     about N / 256): 16-row MFMA tiles, the last one partial (its missing
//     rows are not loaded and not stored);
//   * x is copied into LDS (one padded bf16 row per row of x) whole, or in
//     chunks of KC columns when it does not fit: then each wave stages only
//     the columns it reads, in two buffers of its own (the next chunk's loads
//     in flight while the current one is used), so no barrier is needed;
//   * wave (wt, wk) takes tiles wt, wt + WT, .. (TPW of them) and a contiguous
//     run of IPW 128-wide K blocks of every chunk; the weights are read in
//     whole 128-byte lines (eight rows per load, non-temporal: each weight
//     byte is read once per call) and one lane swap puts them in the MFMA
//     fragment order, lane (row l%16, group g = l/16) holding bytes 16g ..
//     16g+15 and 64+16g .. of the block; the first 8 bytes of each feed one
//     MFMA and the next 8 another, x fragments in the same K order, so one x
//     fragment read serves all TPW tiles;
//   * each 128-wide block's sum is scaled by its scale_inv (the D lanes' four
//     rows share a 128-row scale block), like the other paths;
//   * the WK waves of a tile meet in LDS once at the end, in wave order, and
//     the GEMV epilogue stores four rows per lane: no K parts, no finish.
// Optional input RMSNorm (p.xnorm, one chunk only): wave m normalises row m
// of x in LDS exactly as rms_norm does (bf16(bf16(x * r) * xg)) while the
// first weight items are in flight; with xg and no xnorm the GEMV takes
// bf16(x * xg).
constexpr int XG_WAVES = 8;
constexpr int XG_MAXM = 8;

template <int TPW, int WT, int IPW, int NCH>
struct XgShape {
  static constexpr int WK = XG_WAVES / WT;
  static constexpr int KC = IPW * WK * 128;  // columns of one x chunk
  static constexpr int PITCH = KC * 2 + 16;  // bytes per x row in LDS: the 16 rows of a fragment read differ in bits 4-7
  static constexpr int NXB = NCH > 1 ? 2 : 1;
  static constexpr int NIT = NCH * IPW;      // 128-wide blocks per wave
  static constexpr int XPT = KC / 512;       // 16-byte x pieces per thread and chunk (8 rows)
  // several chunks with one tile group: each wave reads only its own columns
  // of x (IPW blocks per chunk), so each stages them itself in its own two
  // buffers and no barrier is needed between chunks
  static constexpr bool XWAVE = NCH > 1 && WT == 1;
  static constexpr int WSLICE = IPW * 128;       // columns of a wave's slice of a chunk
  static constexpr int WPITCH = WSLICE * 2 + 16;  // bytes per x row of a slice
  static constexpr int XWP = WSLICE / 64;         // 16-byte pieces per lane and slice (8 rows)
  static constexpr size_t XLDS = XWAVE ? (size_t)XG_WAVES * 2 * XG_MAXM * WPITCH : (size_t)NXB * XG_MAXM * PITCH;
  static constexpr size_t GAM = NCH == 1 ? (size_t)KC * 4 : 0;  // the norm weight as fp32 (one chunk only)
  static constexpr size_t LDS = XLDS + GAM + (size_t)XG_WAVES * TPW * 64 * 16;
};

template <int TPW, int WT, int IPW, int NCH, int D, int MODE>
__global__ __launch_bounds__(512, 1) void xgemv_kernel(GemvParams p, int rpw) {
  typedef XgShape<TPW, WT, IPW, NCH> S;
  static_assert(D >= 1 && D <= S::NIT && TPW * WT <= 8, "items in flight within the wave's items; tiles fit one pass");
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  constexpr int WK = S::WK, KC = S::KC, PITCH = S::PITCH, NIT = S::NIT, XPT = S::XPT;
  extern __shared__ __align__(16) uint8_t xsm[];
  const int M = p.M;
  uint8_t *const gsm = xsm + S::XLDS;  // norm weight, fp32
  f32x4 *const red = reinterpret_cast<f32x4 *>(gsm + S::GAM);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wt = wave % WT, wk = wave / WT;
  const int li = lane & 15, lg = lane >> 4;
  const int r0 = blockIdx.x * rpw;
  const int rend = min(r0 + rpw, p.N);
  const int KB = p.K >> 7;
  const bool two = MODE == GEMV_QKVA || p.w1 != nullptr;
  // epilogue operands of the outputs this thread stores (tile tid / 64, x row
  // lane % 16, rows 4 (lane / 16) ..; threads past them load in-bounds ones)
  const int em = min(lane & 15, M - 1), en = min(r0 + 16 * (tid >> 6) + 4 * (lane >> 4), rend - 4);
  EpiOps eo = {};
  epi_load1<MODE>(p, em, en, eo);

  // Weight loads read whole 128-byte lines: for each tile and 128-wide block
  // one load covers rows 0-7 and one rows 8-15, lane l taking row l & 7 and
  // 16-byte chunk cl = ((l >> 4) & 1) + 2 (l >> 5) + 4 ((l >> 3) & 1) of the
  // block (eight lanes per row).  One lane swap (lanes l and l ^ 8, selected
  // by bit 3) turns the pair into the MFMA fragment order: lane (row l % 16,
  // group l / 16) with chunks g and 4 + g.  Rows past the run re-read its last
  // row (the same addresses: no extra traffic; their results are not stored).
  // The scale row is that of the output rows (D: rows 4 lg .. 4 lg + 3 of each
  // tile).  Every load of the stream is unconditional, so the compiler's waits
  // count exactly the items in flight.
  const int cl = ((lane >> 4) & 1) + 2 * (lane >> 5) + 4 * ((lane >> 3) & 1);
  const bool hi8 = (lane >> 3) & 1;
  const uint8_t *wrow[TPW][2];
  const float *srow[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t0 = r0 + 16 * (wt + WT * j);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int rc = min(t0 + 8 * hf + (lane & 7), rend - 1);
      const bool s1 = two && rc >= p.n_split;
      wrow[j][hf] = (s1 ? p.w1 : p.w0) + (size_t)(s1 ? rc - p.n_split : rc) * p.K + 16 * cl;
    }
    const int rd = min(t0 + 4 * lg, p.N - 1);
    const bool d1 = two && rd >= p.n_split;
    srow[j] = (d1 ? p.s1 : p.s0) + (size_t)((d1 ? rd - p.n_split : rd) >> 7) * KB;
  }

  // x chunk c -> registers (piece q of this thread: row q / (KC / 8), 16-byte
  // column piece q % (KC / 8); rows past M re-read row M - 1 and are not stored)
  u32x4 xs[XPT];
  auto load_x = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int q = tid + 512 * i, m = min(q / (KC / 8), M - 1), c8 = q % (KC / 8);
      xs[i] = ldg16(p.x + (size_t)m * p.ldx + (size_t)c * KC + c8 * 8);
    }
  };
  auto store_x = [&](int buf) __attribute__((always_inline)) {
    uint8_t *xb = xsm + (size_t)buf * XG_MAXM * PITCH;
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int q = tid + 512 * i, m = q / (KC / 8), c8 = q % (KC / 8);
      *reinterpret_cast<u32x4 *>(xb + m * PITCH + c8 * 16) = xs[i];
    }
  };
  // a wave's own slice of chunk c (XWAVE): rows past M re-read row M - 1
  constexpr int WSLICE = S::WSLICE, WPITCH = S::WPITCH, XWP = S::XWP;
  u32x4 xw[S::XWAVE ? XWP : 1];
  auto load_xw = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XWP; ++i) {
      const int q = lane + 64 * i, m = min(q / (WSLICE / 8), M - 1), c8 = q % (WSLICE / 8);
      xw[i] = ldg16(p.x + (size_t)m * p.ldx + (size_t)c * KC + wk * WSLICE + c8 * 8);
    }
  };
  auto store_xw = [&](int buf) __attribute__((always_inline)) {
    uint8_t *xb = xsm + (size_t)((wave * 2 + buf) * XG_MAXM) * WPITCH;
#pragma unroll
    for (int i = 0; i < XWP; ++i) {
      const int q = lane + 64 * i, m = q / (WSLICE / 8), c8 = q % (WSLICE / 8);
      *reinterpret_cast<u32x4 *>(xb + m * WPITCH + c8 * 16) = xw[i];
    }
  };
  // LDS-only barrier: the weight loads in flight are not waited for
  auto lds_barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // weight items: item i = block ii of chunk c, both 64-byte steps of each tile
  u32x4 W[NIT][TPW][2];
  float SC[NIT][TPW];
  auto load_w = [&](int i) __attribute__((always_inline)) {
    const int c = i / IPW, ii = i % IPW;
    const int kb = c * (IPW * WK) + wk * IPW + ii;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) W[i][j][hf] = ldg16_nt(wrow[j][hf] + (size_t)kb * 128);
      SC[i][j] = srow[j][kb];
    }
  };

  // The scheduler barriers keep every load where it is written: loads complete
  // in issue order, so a load moved later would make the wait for an earlier
  // one (the compiler's or the x chunk's) wait for it too.
  // x first, then the norm weight (one chunk only; unconditional, from x when
  // there is none; staged in LDS), then the weights: waiting for x and xg does
  // not wait for the weights
  constexpr int PL = KC / 512;                    // 16-byte pieces per lane of a row
  constexpr int GPT = (KC / 8 + 511) / 512;       // 16-byte norm weight pieces per thread
  u32x4 gs[GPT];
  if constexpr (S::XWAVE) load_xw(0);
  else load_x(0);
  if (NCH == 1) {
    const uint16_t *gp = p.xg ? p.xg : p.x;
#pragma unroll
    for (int i = 0; i < GPT; ++i) gs[i] = ldg16(gp + min(tid + 512 * i, KC / 8 - 1) * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < D; ++i) load_w(i);
  epi_load2<MODE>(p, em, en, eo);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (S::XWAVE) store_xw(0);  // this wave's own reads follow in order: no barrier
  else store_x(0);
  if (NCH == 1) {
    // unpacked once here: every row's pass below reads it as fp32
#pragma unroll
    for (int i = 0; i < GPT; ++i)
      if (tid + 512 * i < KC / 8) {
        f32x4 *gd = reinterpret_cast<f32x4 *>(gsm + (tid + 512 * i) * 32);
        gd[0] = f32x4{lo_bf(gs[i].x), hi_bf(gs[i].x), lo_bf(gs[i].y), hi_bf(gs[i].y)};
        gd[1] = f32x4{lo_bf(gs[i].z), hi_bf(gs[i].z), lo_bf(gs[i].w), hi_bf(gs[i].w)};
      }
  }
  if (NCH == 1 && p.xg) {
    // rms_norm(x, xg, eps_in) of each row (inference/ops.py:10-12) in place,
    // wave m on row m, or bf16(x * xg)
    lds_barrier();
    if (wave < M) {
      uint8_t *xr = xsm + wave * PITCH;
      // two passes over the row in LDS (few registers while the weights are
      // in flight): the sum of squares, then bf16(bf16(x * r) * xg); without
      // the norm r = 1 and bf16(x * 1) = x
      float r = 1.f;
      if (p.xnorm) {
        // squares of a bf16 pair in one v_dot2_f32_bf16 (exact products,
        // fp32 sum), two chains
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
          const u32x4 v = *reinterpret_cast<const u32x4 *>(xr + (lane + 64 * i) * 16);
          // named components: a subscripted element cast to bf16x2 was
          // compiled as element 0
          const uint32_t d0 = v.x, d1 = v.y, d2 = v.z, d3 = v.w;
          s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, d0), __builtin_bit_cast(bf16x2, d0), s0, false);
          s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, d1), __builtin_bit_cast(bf16x2, d1), s1, false);
          s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, d2), __builtin_bit_cast(bf16x2, d2), s0, false);
          s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, d3), __builtin_bit_cast(bf16x2, d3), s1, false);
        }
        r = rsqrtf(vg_sum64(s0 + s1) / (float)p.K + p.eps_in);
      }
      // bf16(bf16(x r) g): one packed conversion rounds both halves of a
      // pair after each product
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(xr + (lane + 64 * i) * 16);
        const f32x4 g0 = *reinterpret_cast<const f32x4 *>(gsm + (lane + 64 * i) * 32);
        const f32x4 g1 = *reinterpret_cast<const f32x4 *>(gsm + (lane + 64 * i) * 32 + 16);
        const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        u32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t t = pack_bf16(lo_bf(v[e]) * r, hi_bf(v[e]) * r);
          y[e] = pack_bf16(lo_bf(t) * g[2 * e], hi_bf(t) * g[2 * e + 1]);
        }
        *reinterpret_cast<u32x4 *>(xr + (lane + 64 * i) * 16) = y;
      }
    }
  }
  if constexpr (S::XWAVE) {
    load_xw(1);
  } else {
    lds_barrier();
    if (NCH > 1) load_x(1);
  }
  __builtin_amdgcn_sched_barrier(0);

  // B operand column li holds x row li % M: the columns past M repeat real
  // rows (no conditional reads) and their sums are not stored
  const int xrow = li % M;
  f32x4 acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NIT; ++i) {
    const int c = i / IPW, ii = i % IPW;
    if (i + D < NIT) load_w(i + D);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t *xb = S::XWAVE ? xsm + (size_t)((wave * 2 + c % 2) * XG_MAXM + xrow) * WPITCH + (ii * 128 + 16 * lg) * 2
                                 : xsm + (size_t)(c % S::NXB) * XG_MAXM * PITCH + xrow * PITCH +
                                       ((wk * IPW + ii) * 128 + 16 * lg) * 2;
    bf16x8 xf[2][2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int h = 0; h < 2; ++h) xf[st][h] = as_bf16x8(*reinterpret_cast<const u32x4 *>(xb + 128 * st + 16 * h));
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      // rows 0-7 | rows 8-15 -> fragment order: step 0 (chunks 0-3), step 1 (4-7)
      u32x4 wf[2];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x0 = W[i][j][0][e], x1 = W[i][j][1][e];
        const uint32_t r0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x0, 0x128, 0xf, 0xf, false);  // row_ror:8
        const uint32_t r1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x1, 0x128, 0xf, 0xf, false);
        wf[0][e] = hi8 ? r1 : x0;
        wf[1][e] = hi8 ? x1 : r0;
      }
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const u32x4 w = wf[st];
        bf16x2_t q[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          q[2 * e] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[e], 1.f, false);
          q[2 * e + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[e], 1.f, true);
        }
        const bf16x8 a0 = {q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
        const bf16x8 a1 = {q[4][0], q[4][1], q[5][0], q[5][1], q[6][0], q[6][1], q[7][0], q[7][1]};
        s = mfma16(a0, xf[st][0], s);
        s = mfma16(a1, xf[st][1], s);
      }
      acc[j] += SC[i][j] * s;
    }
    if (NCH > 1 && ii == IPW - 1 && c + 1 < NCH) {
      // chunk c done: the next one into the other buffer (free since the last
      // barrier), then the one after that on its way
      if constexpr (S::XWAVE) {
        store_xw((c + 1) % 2);  // the buffer of chunk c - 1, which this wave has finished
        if (c + 2 < NCH) load_xw(c + 2);
      } else {
        store_x((c + 1) % 2);
        lds_barrier();
        if (c + 2 < NCH) load_x(c + 2);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

#pragma unroll
  for (int j = 0; j < TPW; ++j) red[(wave * TPW + j) * 64 + lane] = acc[j];
  lds_barrier();
  const int ntile = (rend - r0 + 15) >> 4;
  if (tid < ntile * 64) {
    const int tw = tid >> 6, ln = tid & 63;
    const int wtt = tw % WT, j = tw / WT;
    f32x4 v = red[(wtt * TPW + j) * 64 + ln];
#pragma unroll
    for (int k = 1; k < WK; ++k) v += red[((k * WT + wtt) * TPW + j) * 64 + ln];
    const int m = ln & 15, n = r0 + 16 * tw + 4 * (ln >> 4);
    if (m < M && n < rend) store4e<MODE>(p, m, n, v, eo);  // (m, n) = (em, en) here
  }
}

// The shapes with an instantiation: K, tiles per wave, wave rows WT, blocks per
// wave and chunk, chunks, items in flight; rows per workgroup fall in
// (16 (TPW WT - 1) .. 16 TPW WT] (1 .. 16 for one tile).
struct XgCfg {
  int K, tpw, wt, ipw, nch, d;
};
constexpr XgCfg XG_CFGS[] = {
    {16384, 2, 1, 4, 4, 4},  // o_proj (7168 x 16384): 28 rows per workgroup
    {7168, 1, 1, 7, 1, 7},   // q_a | kv_a (2112 x 7168), q_a, kv_a: up to 16 rows
    {1536, 3, 2, 3, 1, 3},   // q_b (24576 x 1536): 96 rows
    {512, 1, 8, 4, 1, 4},    // kv_b (32768 x 512): 128 rows
};
constexpr int XG_NCFG = sizeof(XG_CFGS) / sizeof(XG_CFGS[0]);

static int xgemv_rpw(int N) { return std::max(4, ((N + 255) / 256 + 3) & ~3); }

static int xgemv_cfg(int M, int N, int K) {
  if (M < 2 || M > XG_MAXM || N % 4 || K % 128) return -1;
  const int rpw = xgemv_rpw(N);
  for (int c = 0; c < XG_NCFG; ++c) {
    const XgCfg &g = XG_CFGS[c];
    const int cap = 16 * g.tpw * g.wt;
    if (g.K == K && rpw <= cap && rpw > cap - 16 * g.wt) return c;
  }
  return -1;
}

template <int TPW, int WT, int IPW, int NCH, int D, int MODE>
static void launch_xg(const GemvParams &p, int rpw, unsigned groups, hipStream_t st) {
  static bool attr_set = false;  // raise the dynamic LDS limit once per process
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)xgemv_kernel<TPW, WT, IPW, NCH, D, MODE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr_set = true;
  }
  xgemv_kernel<TPW, WT, IPW, NCH, D, MODE>
      <<<groups, 512, XgShape<TPW, WT, IPW, NCH>::LDS, st>>>(p, rpw);
}

template <int TPW, int WT, int IPW, int NCH, int D>
static void launch_xg_mode(const GemvParams &p, int mode, int rpw, unsigned groups, hipStream_t st) {
  switch (mode) {
    case GEMV_PLAIN: launch_xg<TPW, WT, IPW, NCH, D, GEMV_PLAIN>(p, rpw, groups, st); break;
    case GEMV_RESID: launch_xg<TPW, WT, IPW, NCH, D, GEMV_RESID>(p, rpw, groups, st); break;
    case GEMV_QKVA: launch_xg<TPW, WT, IPW, NCH, D, GEMV_QKVA>(p, rpw, groups, st); break;
    case GEMV_F32: launch_xg<TPW, WT, IPW, NCH, D, GEMV_F32>(p, rpw, groups, st); break;
    default: launch_xg<TPW, WT, IPW, NCH, D, GEMV_QROPE>(p, rpw, groups, st); break;
  }
}

static int launch_xgemv(const GemvParams &p, int mode, hipStream_t st) {
  const int c = xgemv_cfg(p.M, p.N, p.K);
  if (c < 0) return fail(AMLA_EINVAL, "fp8 GEMV (x in LDS): plan for another shape (M=%d N=%d K=%d)", p.M, p.N, p.K);
  if (p.ldx < p.K || p.ldx % 8 || !aligned16(p.x) || (p.xg && !aligned16(p.xg)))
    return fail(AMLA_EINVAL, "fp8 GEMV (x in LDS): x must be 16-byte aligned rows of at least K elements");
  if (p.xg && XG_CFGS[c].nch != 1)
    return fail(AMLA_EUNSUPPORTED, "fp8 GEMV (x in LDS): an input norm needs K <= %d", XG_CFGS[1].K);
  if ((mode == GEMV_QKVA || p.w1) && p.n_split % 4)
    return fail(AMLA_EUNSUPPORTED, "fp8 GEMV (x in LDS): the first weight segment must be a multiple of 4 rows");
  const int rpw = xgemv_rpw(p.N);
  const unsigned groups = (unsigned)((p.N + rpw - 1) / rpw);
  switch (c) {
    case 0: launch_xg_mode<2, 1, 4, 4, 4>(p, mode, rpw, groups, st); break;
    case 1: launch_xg_mode<1, 1, 7, 1, 7>(p, mode, rpw, groups, st); break;
    case 2: launch_xg_mode<3, 2, 3, 1, 3>(p, mode, rpw, groups, st); break;
    default: launch_xg_mode<1, 8, 4, 1, 4>(p, mode, rpw, groups, st); break;
  }
  return check_launch("fp8 GEMV (x in LDS)");
}

// ---------------------------------------------------------------- streaming GEMV, 9 .. 64 rows of x
//
// The form of xgemv_kernel for more rows of x: NCT column tiles of 16 rows
// (MP = 16 NCT), so each weight fragment feeds NCT MFMAs.  A workgroup (8
// waves = WT tile groups x WK K groups) owns R = 16 TPW WT consecutive weight
// rows and one of KP equal K parts (grid y); x of the part moves through LDS
// in NCH chunks of KC = 128 IPW WK columns (all MP rows, double buffered,
// staged through registers one chunk ahead; rows past M repeat row M - 1);
// the weights stream straight into registers as whole 128-byte lines, D
// 128-wide blocks ahead, converted and swapped into fragment order as in
// xgemv_kernel.  Each block's TPW x NCT sums are scaled by its scale_inv; the
// WK waves of a tile meet in LDS at the end (in wave order) and the workgroup
// stores either the GEMV epilogue (KP = 1) or its fp32 K-part sums in the
// [part][M][N] layout that gemv_finish (or the q_a | kv_a finish) sums in
// part order.  With p.xg the GEMM takes bf16(x * xg) (the folded input norm).
template <int NCT, int TPW, int WT, int IPW, int NCH>
struct MgShape {
  static constexpr int MP = 16 * NCT;
  static constexpr int WK = XG_WAVES / WT;
  static constexpr int KC = IPW * WK * 128;
  static constexpr int PITCH = KC * 2 + 16;  // the 16 rows of a fragment read differ in bits 4-7
  static constexpr int NXB = NCH > 1 ? 2 : 1;
  static constexpr int XPT = MP * KC / 4096;  // 16-byte x pieces per thread and chunk
  static constexpr int RING = 2;              // chunks of weights in registers
  static constexpr size_t XLDS = (size_t)NXB * MP * PITCH;
  static constexpr size_t RED = (size_t)XG_WAVES * TPW * NCT * 64 * 16;  // aliases the x buffers at the end
  static constexpr size_t LDS = XLDS > RED ? XLDS : RED;
  static_assert(XPT >= 1 && MP * KC % 4096 == 0, "whole x pieces per thread");
};

template <int NCT, int TPW, int WT, int IPW, int NCH, int MODE, bool PART>
__global__ __launch_bounds__(512, 1) void mgemv_kernel(GemvParams p, int rpw) {
  typedef MgShape<NCT, TPW, WT, IPW, NCH> S;
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  constexpr int WK = S::WK, KC = S::KC, PITCH = S::PITCH, XPT = S::XPT, MP = S::MP;
  extern __shared__ __align__(16) uint8_t xsm[];
  f32x4 *const red = reinterpret_cast<f32x4 *>(xsm);  // after the last chunk
  const int M = p.M;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wt = wave % WT, wk = wave / WT;
  const int li = lane & 15, lg = lane >> 4;
  const int r0 = blockIdx.x * rpw;
  const int rend = min(r0 + rpw, p.N);
  const int KB = p.K >> 7;
  const int kb0 = blockIdx.y * (NCH * IPW * WK);  // first 128-wide block of this K part
  const bool two = MODE == GEMV_QKVA || p.w1 != nullptr;

  // whole-line weight loads (xgemv_kernel's layout): lane l takes row l & 7
  // (+8 for the second load) and 16-byte chunk cl of the block
  const int cl = ((lane >> 4) & 1) + 2 * (lane >> 5) + 4 * ((lane >> 3) & 1);
  const bool hi8 = (lane >> 3) & 1;
  const uint8_t *wrow[TPW][2];
  const float *srow[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t0 = r0 + 16 * (wt + WT * j);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int rc = min(t0 + 8 * hf + (lane & 7), rend - 1);
      const bool s1 = two && rc >= p.n_split;
      wrow[j][hf] = (s1 ? p.w1 : p.w0) + (size_t)(s1 ? rc - p.n_split : rc) * p.K + 16 * cl;
    }
    const int rd = min(t0 + 4 * lg, p.N - 1);
    const bool d1 = two && rd >= p.n_split;
    srow[j] = (d1 ? p.s1 : p.s0) + (size_t)((d1 ? rd - p.n_split : rd) >> 7) * KB;
  }

  // x chunk c of the part -> registers (piece q: row q / (KC / 8), 16-byte
  // column piece q % (KC / 8)), times xg when set
  u32x4 xs[XPT];
  auto load_x = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int q = tid + 512 * i, m = min(q / (KC / 8), M - 1), c8 = q % (KC / 8);
      xs[i] = ldg16(p.x + (size_t)m * p.ldx + (size_t)kb0 * 128 + (size_t)c * KC + c8 * 8);
    }
  };
  auto store_x = [&](int c) __attribute__((always_inline)) {
    uint8_t *xb = xsm + (size_t)(c % S::NXB) * MP * PITCH;
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int q = tid + 512 * i, m = q / (KC / 8), c8 = q % (KC / 8);
      u32x4 v = xs[i];
      if (p.xg) {
        const u32x4 g = ldg16(p.xg + (size_t)kb0 * 128 + (size_t)c * KC + c8 * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = pack_bf16(lo_bf(v[e]) * lo_bf(g[e]), hi_bf(v[e]) * hi_bf(g[e]));
      }
      *reinterpret_cast<u32x4 *>(xb + m * PITCH + c8 * 16) = v;
    }
  };
  auto lds_barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // weights of RING chunks in registers: buffer c % RING holds chunk c's IPW
  // blocks; chunk c + RING is loaded into it as soon as chunk c is consumed.
  // Past the part's end the last chunk is read again (the same lines: no
  // extra traffic), so every load is unconditional and the compiler's waits
  // count exactly the loads in flight.
  constexpr int RING = S::RING;
  u32x4 W[RING][IPW][TPW][2];
  float SC[RING][IPW][TPW];
  auto load_w = [&](int buf, int c, int ii) __attribute__((always_inline)) {
    const int kb = kb0 + min(c, NCH - 1) * (IPW * WK) + wk * IPW + ii;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) W[buf][ii][j][hf] = ldg16_nt(wrow[j][hf] + (size_t)kb * 128);
      SC[buf][ii][j] = srow[j][kb];
    }
  };

  // x first, then the weights (waiting for x does not wait for the weights)
  load_x(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < RING; ++r)
#pragma unroll
    for (int ii = 0; ii < IPW; ++ii) load_w(r, r, ii);
  __builtin_amdgcn_sched_barrier(0);
  store_x(0);
  lds_barrier();
  load_x(min(1, NCH - 1));
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[TPW][NCT];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[j][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  // chunk c from weight buffer buf; B operand of column tile ct: x row
  // 16 ct + li (rows past M hold row M - 1)
  auto chunk = [&](int c, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int ii = 0; ii < IPW; ++ii) {
      const uint8_t *xb = xsm + (size_t)(c % S::NXB) * MP * PITCH + li * PITCH + ((wk * IPW + ii) * 128 + 16 * lg) * 2;
      f32x4 sm[TPW][NCT];
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) sm[j][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        bf16x8 xf[NCT][2];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            xf[ct][h] = as_bf16x8(*reinterpret_cast<const u32x4 *>(xb + (size_t)16 * ct * PITCH + 128 * st + 16 * h));
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          // rows 0-7 | rows 8-15 -> fragment order of step st
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t x0 = W[buf][ii][j][0][e], x1 = W[buf][ii][j][1][e];
            if (st == 0) {
              const uint32_t r1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x1, 0x128, 0xf, 0xf, false);  // row_ror:8
              w[e] = hi8 ? r1 : x0;
            } else {
              const uint32_t r0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x0, 0x128, 0xf, 0xf, false);
              w[e] = hi8 ? x1 : r0;
            }
          }
          bf16x2_t q[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            q[2 * e] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[e], 1.f, false);
            q[2 * e + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[e], 1.f, true);
          }
          const bf16x8 a0 = {q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
          const bf16x8 a1 = {q[4][0], q[4][1], q[5][0], q[5][1], q[6][0], q[6][1], q[7][0], q[7][1]};
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            sm[j][ct] = mfma16(a0, xf[ct][0], sm[j][ct]);
            sm[j][ct] = mfma16(a1, xf[ct][1], sm[j][ct]);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[j][ct] += SC[buf][ii][j] * sm[j][ct];
      load_w(buf, c + RING, ii);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (NCH > 1 && c + 1 < NCH) {
      // every wave is done with chunk c - 1, whose buffer takes chunk c + 1
      // (loaded during chunk c - 1); then chunk c + 2 on its way
      store_x(c + 1);
      lds_barrier();
      load_x(min(c + 2, NCH - 1));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  static_assert(NCH <= 4, "the chunk loop is unrolled");
#pragma unroll
  for (int c = 0; c < NCH; ++c) chunk(c, c % RING);

  // the x buffers become the reduction buffer: every wave is past its last read
  lds_barrier();
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) red[((wave * TPW + j) * NCT + ct) * 64 + lane] = acc[j][ct];
  lds_barrier();
  const int ntile = (rend - r0 + 15) >> 4;
  for (int u = tid; u < ntile * NCT * 64; u += 512) {
    const int ln = u & 63, ct = (u >> 6) % NCT, tw = (u >> 6) / NCT;
    const int wtt = tw % WT, j = tw / WT;
    f32x4 v = red[((wtt * TPW + j) * NCT + ct) * 64 + ln];
#pragma unroll
    for (int k = 1; k < WK; ++k) v += red[(((k * WT + wtt) * TPW + j) * NCT + ct) * 64 + ln];
    const int m = 16 * ct + (ln & 15), n = r0 + 16 * tw + 4 * (ln >> 4);
    if (m < M && n < rend) {
      if constexpr (PART)
        *reinterpret_cast<f32x4 *>(p.part + ((size_t)blockIdx.y * M + m) * p.N + n) = v;
      else
        store4<MODE>(p, m, n, v);
    }
  }
}

// Shapes with an instantiation (the MLA projections): K, N, tile groups, K
// parts; rows per workgroup R = 16 TPW WT.
struct MgCfg {
  int K, N, tpw, wt, ipw, nch, kp;
};
// Measured against the skinny MFMA GEMM (gemv_kernel + finish) at M = 16, 32
// and 64 (kernel trace, one box): q_b 12.0 / 14.9 / 19.0 -> 10.7 / 12.1 /
// 15.2 us, q_a | kv_a 11.4 / 13.8 / 18.6 -> 9.4 / 10.6 / 13.7, q_a 11.8 /
// 13.4 / 18.2 -> 9.4 / 10.2 / 13.5, kv_b 7.3 / 8.7 / 11.5 -> 6.3 / 6.8 / 8.7.
// o_proj (128 rows x 4 parts of 4096: 30.5 / 35.4 / 44.5 -> 36.2 / 39.2 /
// 44.9) and kv_a alone (63 workgroups) stay on the skinny GEMM.
constexpr MgCfg MG_CFGS[] = {
    {1536, 24576, 3, 2, 1, 3, 1},  // q_b: 96 rows, whole K (256 workgroups)
    {7168, 2112, 2, 2, 1, 2, 7},   // q_a | kv_a: 64 rows x 7 parts of 1024 (231 workgroups)
    {7168, 1536, 2, 2, 1, 2, 7},   // q_a
    {512, 32768, 2, 4, 2, 1, 1},   // kv_b: 128 rows, whole K (256 workgroups)
};
constexpr int MG_NCFG = sizeof(MG_CFGS) / sizeof(MG_CFGS[0]);

static int mgemv_cfg(int M, int N, int K) {
  if (M <= XG_MAXM || M > 64) return -1;
  for (int c = 0; c < MG_NCFG; ++c)
    if (MG_CFGS[c].K == K && MG_CFGS[c].N == N) return c;
  return -1;
}

template <int NCT, int TPW, int WT, int IPW, int NCH, int MODE, bool PART>
static void launch_mg(const GemvParams &p, int rpw, dim3 grid, hipStream_t st) {
  typedef MgShape<NCT, TPW, WT, IPW, NCH> S;
  static bool attr_set = false;  // raise the dynamic LDS limit once per process
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)mgemv_kernel<NCT, TPW, WT, IPW, NCH, MODE, PART>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr_set = true;
  }
  static_assert(S::LDS <= 160 * 1024, "LDS budget");
  mgemv_kernel<NCT, TPW, WT, IPW, NCH, MODE, PART><<<grid, 512, S::LDS, st>>>(p, rpw);
}

template <int NCT, int TPW, int WT, int IPW, int NCH, bool PART>
static void launch_mg_mode(const GemvParams &p, int mode, int rpw, dim3 grid, hipStream_t st) {
  if constexpr (PART) {
    launch_mg<NCT, TPW, WT, IPW, NCH, GEMV_F32, true>(p, rpw, grid, st);
  } else {
    switch (mode) {
      case GEMV_PLAIN: launch_mg<NCT, TPW, WT, IPW, NCH, GEMV_PLAIN, false>(p, rpw, grid, st); break;
      case GEMV_RESID: launch_mg<NCT, TPW, WT, IPW, NCH, GEMV_RESID, false>(p, rpw, grid, st); break;
      case GEMV_QKVA: launch_mg<NCT, TPW, WT, IPW, NCH, GEMV_QKVA, false>(p, rpw, grid, st); break;
      case GEMV_F32: launch_mg<NCT, TPW, WT, IPW, NCH, GEMV_F32, false>(p, rpw, grid, st); break;
      default: launch_mg<NCT, TPW, WT, IPW, NCH, GEMV_QROPE, false>(p, rpw, grid, st); break;
    }
  }
}

// configurations with K parts store fp32 part sums (PART), the others the
// GEMV epilogue
template <int NCT>
static void launch_mg_cfg(const GemvParams &p, int mode, int c, int rpw, dim3 grid, hipStream_t st) {
  switch (c) {
    case 0: launch_mg_mode<NCT, 3, 2, 1, 3, false>(p, mode, rpw, grid, st); break;
    case 1:
    case 2: launch_mg_mode<NCT, 2, 2, 1, 2, true>(p, mode, rpw, grid, st); break;
    default: launch_mg_mode<NCT, 2, 4, 2, 1, false>(p, mode, rpw, grid, st); break;
  }
}

static int launch_mgemv(const GemvParams &p, int mode, const GemvPlan &pl, hipStream_t st, bool finish) {
  const int c = mgemv_cfg(p.M, p.N, p.K);
  if (c < 0) return fail(AMLA_EINVAL, "fp8 GEMV (9 .. 64 rows of x): plan for another shape (M=%d N=%d K=%d)", p.M, p.N, p.K);
  const MgCfg &g = MG_CFGS[c];
  if (p.ldx < p.K || p.ldx % 8 || !aligned16(p.x) || (p.xg && !aligned16(p.xg)))
    return fail(AMLA_EINVAL, "fp8 GEMV (9 .. 64 rows of x): x must be 16-byte aligned rows of at least K elements");
  if ((mode == GEMV_QKVA || p.w1) && p.n_split % 4)
    return fail(AMLA_EUNSUPPORTED, "fp8 GEMV (9 .. 64 rows of x): the first weight segment must be a multiple of 4 rows");
  if (g.kp > 1 && !p.part) return fail(AMLA_EWORKSPACE, "fp8 GEMV (9 .. 64 rows of x): missing partial-sum workspace");
  const int rpw = 16 * g.tpw * g.wt;
  const dim3 grid((unsigned)((p.N + rpw - 1) / rpw), (unsigned)g.kp);
  if (p.M <= 16) launch_mg_cfg<1>(p, mode, c, rpw, grid, st);
  else if (p.M <= 32) launch_mg_cfg<2>(p, mode, c, rpw, grid, st);
  else launch_mg_cfg<4>(p, mode, c, rpw, grid, st);
  int rc = check_launch("fp8 GEMV (9 .. 64 rows of x)");
  if (rc) return rc;
  if (g.kp > 1 && finish) {
    const int64_t total = (int64_t)p.M * (p.N / 4);
    const unsigned blocks = (unsigned)((total + 63) / 64);
    switch (mode) {
      case GEMV_PLAIN: gemv_finish<GEMV_PLAIN><<<blocks, 64, 0, st>>>(p, g.kp); break;
      case GEMV_RESID: gemv_finish<GEMV_RESID><<<blocks, 64, 0, st>>>(p, g.kp); break;
      case GEMV_QKVA: gemv_finish<GEMV_QKVA><<<blocks, 64, 0, st>>>(p, g.kp); break;
      case GEMV_F32: gemv_finish<GEMV_F32><<<blocks, 64, 0, st>>>(p, g.kp); break;
      default: gemv_finish<GEMV_QROPE><<<blocks, 64, 0, st>>>(p, g.kp); break;
    }
    return check_launch("fp8 GEMV finish (9 .. 64 rows of x)");
  }
  (void)pl;
  return AMLA_OK;
}

static GemvPlan plan_mgemv(int M, int N, int K) {
  GemvPlan pl = {};
  const MgCfg &g = MG_CFGS[mgemv_cfg(M, N, K)];
  const int rpw = 16 * g.tpw * g.wt;
  pl.kparts = g.kp;
  pl.kpb = K / 128 / g.kp;
  pl.rg = g.tpw * g.wt;
  pl.groups = ((N + rpw - 1) / rpw) * g.kp;
  pl.part_bytes = g.kp > 1 ? (size_t)g.kp * M * N * 4 : 0;
  pl.vec = 4;
  return pl;
}

// rows per workgroup of the streaming GEMV: about VG_GRID workgroups
static int vgemv_rpw(int N) {
  const int r = (N + VG_GRID - 1) / VG_GRID;
  return std::min(VG_MAX_RPW, std::max(2 * VG_R, (r + 3) & ~3));
}

template <int NCH>
static void launch_vgemv_mode(const GemvParams &p, int mode, hipStream_t st) {
  const int rpw = vgemv_rpw(p.N);
  const unsigned groups = (unsigned)((p.N + rpw - 1) / rpw);
  switch (mode) {
    case GEMV_PLAIN: vgemv_kernel<NCH, GEMV_PLAIN><<<groups, 256, 0, st>>>(p, rpw); break;
    case GEMV_RESID: vgemv_kernel<NCH, GEMV_RESID><<<groups, 256, 0, st>>>(p, rpw); break;
    case GEMV_QKVA: vgemv_kernel<NCH, GEMV_QKVA><<<groups, 256, 0, st>>>(p, rpw); break;
    case GEMV_F32: vgemv_kernel<NCH, GEMV_F32><<<groups, 256, 0, st>>>(p, rpw); break;
    default: vgemv_kernel<NCH, GEMV_QROPE><<<groups, 256, 0, st>>>(p, rpw); break;
  }
}

static bool vgemv_applies(int M, int N, int K) { return M == 1 && K % 128 == 0 && K >= 4096 && K <= 16384 && N % 8 == 0; }
static bool vgemv_short_applies(int M, int N, int K) { return M == 1 && K == VGS_C * 16 && N % 8 == 0; }

GemvPlan plan_linear(int M, int N, int K) {
  GemvPlan pl = {};
  if (vgemv_applies(M, N, K)) {
    pl.groups = (N + vgemv_rpw(N) - 1) / vgemv_rpw(N);
    pl.vec = 1;
  } else if (vgemv_short_applies(M, N, K)) {
    pl.groups = (N + VGS_RPW - 1) / VGS_RPW;
    pl.vec = 2;
  } else if (xgemv_cfg(M, N, K) >= 0) {
    pl.groups = (N + xgemv_rpw(N) - 1) / xgemv_rpw(N);
    pl.vec = 3;
  } else if (mgemv_cfg(M, N, K) >= 0) {
    return plan_mgemv(M, N, K);
  } else {
    return plan_gemv(M, N, K);
  }
  pl.kpb = K / 128;
  pl.kparts = 1;
  pl.rg = 1;
  return pl;
}

static int launch_vgemv(const GemvParams &p, int mode, int vec, hipStream_t st) {
  if (vec == 3) return launch_xgemv(p, mode, st);
  if (p.ldx < p.K || !aligned16(p.x) || (p.xg && !aligned16(p.xg)))
    return fail(AMLA_EINVAL, "streaming fp8 GEMV: x must be 16-byte aligned rows of at least K elements");
  if (vec == 2) {
    // one weight segment (the row-segment and cache epilogues take the long-row kernel)
    if (!vgemv_short_applies(p.M, p.N, p.K) || p.w1 || mode == GEMV_QKVA)
      return fail(AMLA_EINVAL, "streaming fp8 GEMV: plan for another shape (M=%d N=%d K=%d)", p.M, p.N, p.K);
    const unsigned groups = (unsigned)((p.N + VGS_RPW - 1) / VGS_RPW);
    switch (mode) {
      case GEMV_PLAIN: vgemv_short_kernel<GEMV_PLAIN><<<groups, 256, 0, st>>>(p); break;
      case GEMV_RESID: vgemv_short_kernel<GEMV_RESID><<<groups, 256, 0, st>>>(p); break;
      case GEMV_F32: vgemv_short_kernel<GEMV_F32><<<groups, 256, 0, st>>>(p); break;
      default: vgemv_short_kernel<GEMV_QROPE><<<groups, 256, 0, st>>>(p); break;
    }
    return check_launch("fp8 streaming GEMV (short rows)");
  }
  if (!vgemv_applies(p.M, p.N, p.K) || (p.w1 || mode == GEMV_QKVA ? p.n_split % 128 : 0))
    return fail(AMLA_EINVAL, "streaming fp8 GEMV: plan for another shape (M=%d N=%d K=%d)", p.M, p.N, p.K);
  const int C = p.K >> 4;
  if (C <= 256) launch_vgemv_mode<1>(p, mode, st);
  else if (C <= 512) launch_vgemv_mode<2>(p, mode, st);
  else launch_vgemv_mode<4>(p, mode, st);
  return check_launch("fp8 streaming GEMV");
}

template <int MT, int MODE>
static int launch_cfg(const GemvParams &p, const GemvPlan &pl, hipStream_t st) {
  static bool attr_set = false;  // raise the dynamic LDS limit once per process
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)gemv_kernel<MT, MODE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    attr_set = true;
  }
  gemv_kernel<MT, MODE><<<dim3(pl.groups), 256, pl.lds, st>>>(p, pl.rg, pl.kparts, pl.kpb);
  return 0;
}

template <int MT>
static void launch_mt(const GemvParams &p, int mode, const GemvPlan &pl, hipStream_t st) {
  switch (mode) {
    case GEMV_PLAIN: launch_cfg<MT, GEMV_PLAIN>(p, pl, st); break;
    case GEMV_RESID: launch_cfg<MT, GEMV_RESID>(p, pl, st); break;
    case GEMV_QKVA: launch_cfg<MT, GEMV_QKVA>(p, pl, st); break;
    case GEMV_F32: launch_cfg<MT, GEMV_F32>(p, pl, st); break;
    default: launch_cfg<MT, GEMV_QROPE>(p, pl, st); break;
  }
}

int launch_gemv(const GemvParams &p0, int mode, const GemvPlan &pl, hipStream_t st, bool finish) {
  if (pl.vec == 4) return launch_mgemv(p0, mode, pl, st, finish);
  if (pl.vec) return launch_vgemv(p0, mode, pl.vec, st);
  if (p0.M < 1 || p0.M > 64) return fail(AMLA_EINVAL, "skinny fp8 GEMM needs 1 <= M <= 64 (got %d)", p0.M);
  if (p0.N % 16 || p0.K % 128)
    return fail(AMLA_EUNSUPPORTED, "skinny fp8 GEMM needs N %% 16 == 0 and K %% 128 == 0 (N=%d K=%d)", p0.N, p0.K);
  if (pl.kparts > GEMV_MAX_PARTS)
    return fail(AMLA_EUNSUPPORTED, "skinny fp8 GEMM: K=%d is too long for M=%d (more than %d K parts)", p0.K, p0.M,
                GEMV_MAX_PARTS);
  if (pl.kparts > 1 && !p0.part) return fail(AMLA_EWORKSPACE, "skinny fp8 GEMM: missing partial-sum workspace");
  if ((mode == GEMV_QKVA && p0.max_rows <= 0) || (mode == GEMV_QROPE && p0.rope_rows <= 0))
    return fail(AMLA_EINVAL, "skinny fp8 GEMM: cache rows / rope rows of the epilogue not set");
  if (p0.w1 && p0.n_split % 128)
    return fail(AMLA_EUNSUPPORTED, "skinny fp8 GEMM: the first weight segment must be a multiple of 128 rows");
  const int MT = p0.M <= 16 ? 1 : (p0.M <= 32 ? 2 : 4);
  if (pl.kpb > gemv_kpb_max(MT) || gemv_lds_bytes(MT, pl.kpb, pl.rg, pl.kparts) > pl.lds)
    return fail(AMLA_EINVAL, "skinny fp8 GEMM: plan for a smaller M");
  if (MT == 1) launch_mt<1>(p0, mode, pl, st);
  else if (MT == 2) launch_mt<2>(p0, mode, pl, st);
  else launch_mt<4>(p0, mode, pl, st);
  if (pl.kparts > 1 && finish) {
    const int64_t total = (int64_t)p0.M * (p0.N / 4);
    const unsigned blocks = (unsigned)((total + 63) / 64);
    switch (mode) {
      case GEMV_PLAIN: gemv_finish<GEMV_PLAIN><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      case GEMV_RESID: gemv_finish<GEMV_RESID><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      case GEMV_QKVA: gemv_finish<GEMV_QKVA><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      case GEMV_F32: gemv_finish<GEMV_F32><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
      default: gemv_finish<GEMV_QROPE><<<blocks, 64, 0, st>>>(p0, pl.kparts); break;
    }
  }
  return check_launch("fp8 skinny GEMM");
}

template <int MT>
static void launch_grouped_mt(const GemvParams &p, const GemvGroups &gr, const GemvPlan &pl, hipStream_t st) {
  static bool attr_set = false;  // raise the dynamic LDS limit once per process
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)gemv_grouped_kernel<MT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    attr_set = true;
  }
  gemv_grouped_kernel<MT><<<dim3((unsigned)(gr.n * gr.units)), 256, pl.lds, st>>>(p, gr, pl.rg, pl.kparts, pl.kpb);
}

int launch_gemv_grouped(const GemvParams &p, GemvGroups gr, const GemvPlan &pl, hipStream_t st) {
  if (gr.n < 1 || gr.n > GEMV_MAX_GROUPS) return fail(AMLA_EINVAL, "grouped skinny GEMM: %d groups", gr.n);
  int max_m = 0;
  for (int g = 0; g < gr.n; ++g) {
    if (gr.g[g].M < 1 || gr.g[g].M > 64) return fail(AMLA_EINVAL, "grouped skinny GEMM: M=%d", gr.g[g].M);
    if (pl.kparts > 1 && !gr.g[g].part) return fail(AMLA_EWORKSPACE, "grouped skinny GEMM: missing partial sums");
    max_m = std::max(max_m, gr.g[g].M);
  }
  if (p.N % 16 || p.K % 128 || pl.kparts > GEMV_MAX_PARTS || (p.w1 && p.n_split % 128))
    return fail(AMLA_EUNSUPPORTED, "grouped skinny GEMM: unsupported shape N=%d K=%d", p.N, p.K);
  const int MT = max_m <= 16 ? 1 : (max_m <= 32 ? 2 : 4);
  if (gemv_lds_bytes(MT, pl.kpb, pl.rg, pl.kparts) > pl.lds || pl.kpb > gemv_kpb_max(MT))
    return fail(AMLA_EINVAL, "grouped skinny GEMM: plan for a smaller M");
  gr.units = pl.groups;
  if (MT == 1) launch_grouped_mt<1>(p, gr, pl, st);
  else if (MT == 2) launch_grouped_mt<2>(p, gr, pl, st);
  else launch_grouped_mt<4>(p, gr, pl, st);
  if (pl.kparts > 1) {
    GemvGroups fr = gr;
    fr.units = (int)(((int64_t)max_m * (p.N / 4) + 63) / 64);
    gemv_finish_grouped<<<dim3((unsigned)(fr.n * fr.units)), 64, 0, st>>>(p, fr, pl.kparts);
  }
  return check_launch("grouped fp8 skinny GEMM");
}

template <int MT>
static void launch_sched_mt(const GemvParams &p, const MoeSched &s, int max_entries, const GemvPlan &pl,
                            hipStream_t st) {
  static bool attr_set = false;  // raise the dynamic LDS limit once per process
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)gemv_sched_kernel<MT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024);
    attr_set = true;
  }
  gemv_sched_kernel<MT><<<dim3((unsigned)(max_entries * pl.groups)), 256, pl.lds, st>>>(p, s, pl.groups, pl.rg,
                                                                                      pl.kparts, pl.kpb);
}

int launch_gemv_sched(const GemvParams &p, const MoeSched &s, int max_entries, int max_m, const GemvPlan &pl,
                      hipStream_t st) {
  if (max_entries <= 0) return AMLA_OK;
  if (max_m < 1 || max_m > 64) return fail(AMLA_EINVAL, "scheduled skinny GEMM: max rows %d", max_m);
  if (p.N % 16 || p.K % 128 || pl.kparts > GEMV_MAX_PARTS || (!s.down && p.n_split % 128))
    return fail(AMLA_EUNSUPPORTED, "scheduled skinny GEMM: unsupported shape N=%d K=%d", p.N, p.K);
  if (pl.kparts > 1 && !p.part) return fail(AMLA_EWORKSPACE, "scheduled skinny GEMM: missing partial sums");
  const int MT = max_m <= 16 ? 1 : (max_m <= 32 ? 2 : 4);
  if (gemv_lds_bytes(MT, pl.kpb, pl.rg, pl.kparts) > pl.lds || pl.kpb > gemv_kpb_max(MT))
    return fail(AMLA_EINVAL, "scheduled skinny GEMM: plan for a smaller M");
  if ((int64_t)max_entries * pl.groups > INT32_MAX) return fail(AMLA_EUNSUPPORTED, "scheduled skinny GEMM: grid");
  if (MT == 1) launch_sched_mt<1>(p, s, max_entries, pl, st);
  else if (MT == 2) launch_sched_mt<2>(p, s, max_entries, pl, st);
  else launch_sched_mt<4>(p, s, max_entries, pl, st);
  if (pl.kparts > 1) {
    const int units = (int)(((int64_t)max_m * (p.N / 4) + 63) / 64);
    gemv_finish_sched<<<dim3((unsigned)(max_entries * units)), 64, 0, st>>>(p, s, units, pl.kparts);
  }
  return check_launch("scheduled fp8 skinny GEMM");
}

// ---------------------------------------------------------------- rms_norm

// One workgroup per row: fp32 sum of squares, r = rsqrt(mean + eps),
// y = bf16(bf16(x * r) * gamma)  (the two roundings of inference/ops.py:12).
// Rows of up to RMS_VEC_MAXC * 256 16-byte chunks are read once, every load
// in flight together, and kept in registers for the output pass; other
// shapes take the element-wise loop.
constexpr int RMS_VEC_MAXC = 8;
template <bool VEC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t *__restrict__ x, int64_t dim,
                                                       int64_t ldx, const uint16_t *__restrict__ gamma,
                                                       float eps, uint16_t *__restrict__ y,
                                                       int64_t ldy) {
  const uint16_t *xr = x + blockIdx.x * ldx;
  uint16_t *yr = y + blockIdx.x * ldy;
  const int tid = threadIdx.x;
  __shared__ float part[4];
  float ss = 0.f;
  if constexpr (VEC) {
    const int nc = (int)(dim >> 3);
    u32x4 v[RMS_VEC_MAXC];
#pragma unroll
    for (int i = 0; i < RMS_VEC_MAXC; ++i) {
      const int c = tid + 256 * i;
      v[i] = c < nc ? ldg16(xr + c * 8) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < RMS_VEC_MAXC; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += lo_bf(v[i][e]) * lo_bf(v[i][e]) + hi_bf(v[i][e]) * hi_bf(v[i][e]);
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float r = rsqrtf(((part[0] + part[1]) + (part[2] + part[3])) / (float)dim + eps);
#pragma unroll
    for (int i = 0; i < RMS_VEC_MAXC; ++i) {
      const int c = tid + 256 * i;
      if (c < nc) {
        const u32x4 g = ldg16(gamma + c * 8);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = pack_bf16(round_bf16(lo_bf(v[i][e]) * r) * lo_bf(g[e]), round_bf16(hi_bf(v[i][e]) * r) * hi_bf(g[e]));
        *reinterpret_cast<u32x4 *>(yr + c * 8) = o;
      }
    }
  } else {
    for (int64_t j = tid; j < dim; j += 256) {
      const float v = bf2f(xr[j]);
      ss += v * v;
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float r = rsqrtf(((part[0] + part[1]) + (part[2] + part[3])) / (float)dim + eps);
    for (int64_t j = tid; j < dim; j += 256) {
      const float nv = round_bf16(bf2f(xr[j]) * r);
      yr[j] = f2bf(nv * bf2f(gamma[j]));
    }
  }
}

int launch_rms_norm(const uint16_t *x, int64_t rows, int64_t dim, int64_t ldx, const uint16_t *gamma,
                    float eps, uint16_t *y, int64_t ldy, hipStream_t st) {
  if (rows == 0) return AMLA_OK;
  const bool vec = dim % 8 == 0 && dim <= RMS_VEC_MAXC * 256 * 8 && ldx % 8 == 0 && ldy % 8 == 0 && aligned16(x) &&
                   aligned16(y) && aligned16(gamma);
  if (vec) rms_norm_kernel<true><<<dim3((unsigned)rows), 256, 0, st>>>(x, dim, ldx, gamma, eps, y, ldy);
  else rms_norm_kernel<false><<<dim3((unsigned)rows), 256, 0, st>>>(x, dim, ldx, gamma, eps, y, ldy);
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

int amla_abi_version(void) { return 104; }

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
  return plan_linear((int)m, (int)n, (int)k).part_bytes;
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
  const GemvPlan pl = plan_linear((int)m, (int)n, (int)k);
  if (pl.part_bytes) {
    if (!workspace || workspace_bytes < pl.part_bytes || !aligned16(workspace))
      return fail(AMLA_EWORKSPACE, "fp8_linear: needs %zu bytes of 16-byte aligned workspace (got %zu)", pl.part_bytes,
                  workspace ? workspace_bytes : (size_t)0);
    p.part = reinterpret_cast<float *>(workspace);
  }
  return launch_gemv(p, GEMV_PLAIN, pl, st);
}

int amla_fp8_linear_f32(const void *x, int64_t m, int64_t k, int64_t ldx, const void *weight,
                        const float *scale_inv, int64_t n, float *y, int64_t ldy, void *workspace,
                        size_t workspace_bytes, void *stream) {
  if (!x || !weight || !scale_inv || !y) return fail(AMLA_EINVAL, "fp8_linear_f32: null pointer");
  if (m < 0 || n <= 0 || k <= 0) return fail(AMLA_EINVAL, "fp8_linear_f32: bad shape m=%lld n=%lld k=%lld",
                                             (long long)m, (long long)n, (long long)k);
  if (ldx < k || ldy < n) return fail(AMLA_EINVAL, "fp8_linear_f32: row stride smaller than the row");
  if (m == 0) return AMLA_OK;
  if (n % 16 || k % 128 || ldx % 8 || ldy % 4 || !aligned16(x) || !aligned16(weight) || !aligned16(y))
    return fail(AMLA_EUNSUPPORTED,
                "fp8_linear_f32: needs n %% 16 == 0, k %% 128 == 0, ldx %% 8 == 0, ldy %% 4 == 0 and 16-byte "
                "aligned x/weight/y (n=%lld k=%lld)",
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
  p.y = reinterpret_cast<uint16_t *>(y);  // fp32 rows in GEMV_F32 mode
  p.ldy = (int)ldy;
  p.seq_len = 1;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (m > 64) return launch_gemm(p, GEMV_F32, st);
  const GemvPlan pl = plan_linear((int)m, (int)n, (int)k);
  if (pl.part_bytes) {
    if (!workspace || workspace_bytes < pl.part_bytes || !aligned16(workspace))
      return fail(AMLA_EWORKSPACE, "fp8_linear_f32: needs %zu bytes of 16-byte aligned workspace (got %zu)",
                  pl.part_bytes, workspace ? workspace_bytes : (size_t)0);
    p.part = reinterpret_cast<float *>(workspace);
  }
  return launch_gemv(p, GEMV_F32, pl, st);
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
