// MLA prefill for gfx950: amla_mla_prefill replaces mla_attention for S >= 1
// tokens per sequence with a causal mask (inference/ops.py:100-183, :172-177),
// and the large-M block-FP8 GEMM that amla_fp8_linear uses for M > 64.
//
// Prefill keeps the reference's non-absorbed formulation (absorption would
// cost more FLOPs at S = T): kv_b decompresses the RMS-normed latent rows once
// per call (one GEMM), and causal flash attention runs per head with
// d_qk = 128 + 64 (the rope key shared by all heads) and d_v = 128.
//
// GEMM (K3): C[m, n] = sum_k X[m, k] W[n, k] scale_inv[n/128, k/128], with
//   256 x 256 workgroup tiles, LDS-DMA staging of fp8 weights and bf16
//   activations, exact in-register fp8 -> bf16 conversion, 32x32x16 MFMAs and
//   a running-scale accumulator for the 128 x 128 block scales.
#include <math.h>

#include <algorithm>

#include "amla_common.h"
#include "amla_internal.h"

namespace amla {

// Epilogue shared with the skinny GEMM (fp8_linear.hip); same contract.
AMLA_DEV int prow_position(const GemvParams &p, int m) { return p.pos[m / p.seq_len] + m % p.seq_len; }

template <int MODE>
AMLA_DEV void pstore4(const GemvParams &p, int m, int n, f32x4 v) {
  if (MODE == GEMV_PLAIN) {
    u32x2 o = {pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
    *reinterpret_cast<u32x2 *>(p.y + (size_t)m * p.ldy + n) = o;
  } else if (MODE == GEMV_F32) {
    *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.y) + (size_t)m * p.ldy + n) = v;
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
      const int64_t row = prow_position(p, m);
      if (row >= p.max_rows) return;  // a device position past the cache: nothing is written
      const int nn = n - p.n_split;
      uint16_t *dst = nn < p.kv_lora ? p.ckv + b * p.ckv_bstride + row * p.kv_lora + nn
                                     : p.kpe + b * p.kpe_bstride + row * p.rope + (nn - p.kv_lora);
      *reinterpret_cast<u32x2 *>(dst) = o;
    }
  } else {
    float a0 = round_bf16(v.x), a1 = round_bf16(v.y), a2 = round_bf16(v.z), a3 = round_bf16(v.w);
    const int d = n % p.head_dim;
    if (d >= p.nope) {
      const int i = (d - p.nope) >> 1;
      const int64_t row = min(prow_position(p, m), p.rope_rows - 1);  // in bounds for any device position
      const f32x4 cs = *reinterpret_cast<const f32x4 *>(p.rope_table + (row * (p.rope >> 1) + i) * 2);
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

// ---------------------------------------------------------------- K3 GEMM


// Eight consecutive outputs n .. n+7 (n % 8 == 0) already rounded to bf16.
template <int MODE>
AMLA_DEV void pstore8(const GemvParams &p, int m, int n, u32x4 v) {
  if (MODE == GEMV_F32) {
    // not reached: fp32 outputs take the unstaged epilogue (launch_gemm)
  } else if (MODE == GEMV_PLAIN) {
    *reinterpret_cast<u32x4 *>(p.y + (size_t)m * p.ldy + n) = v;
  } else if (MODE == GEMV_RESID) {
    const u32x4 r = *reinterpret_cast<const u32x4 *>(p.res + (size_t)m * p.ldr + n);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16(lo_bf(r[i]) + lo_bf(v[i]), hi_bf(r[i]) + hi_bf(v[i]));
    *reinterpret_cast<u32x4 *>(p.y + (size_t)m * p.ldy + n) = o;
  } else if (MODE == GEMV_QKVA) {
    if (n < p.n_split) {
      *reinterpret_cast<u32x4 *>(p.y + (size_t)m * p.ldy + n) = v;
    } else {
      const int b = m / p.seq_len;
      const int64_t row = prow_position(p, m);
      if (row >= p.max_rows) return;  // a device position past the cache: nothing is written
      const int nn = n - p.n_split;
      uint16_t *dst = nn < p.kv_lora ? p.ckv + b * p.ckv_bstride + row * p.kv_lora + nn
                                     : p.kpe + b * p.kpe_bstride + row * p.rope + (nn - p.kv_lora);
      *reinterpret_cast<u32x4 *>(dst) = v;
    }
  } else {
    const int d = n % p.head_dim;
    u32x4 o = v;
    if (d >= p.nope) {
      const int64_t row = min(prow_position(p, m), p.rope_rows - 1);  // in bounds for any device position
      const float *tab = p.rope_table + (row * (p.rope >> 1) + ((d - p.nope) >> 1)) * 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a0 = lo_bf(v[i]), a1 = hi_bf(v[i]);
        const float c = tab[2 * i], s = tab[2 * i + 1];
        o[i] = pack_bf16(__fsub_rn(__fmul_rn(a0, c), __fmul_rn(a1, s)), __fadd_rn(__fmul_rn(a0, s), __fmul_rn(a1, c)));
      }
    }
    *reinterpret_cast<u32x4 *>(p.y + (size_t)m * p.ldy + n) = o;
  }
}

AMLA_DEV f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}


// Workgroup tile 256 weight rows (n) x 256 activation rows (m), K stage 64,
// three LDS stages filled by direct global-to-LDS copies: fp8 weight rows
// (64 B) and bf16 activation rows (128 B), 16-byte chunks swizzled per row
// (chunk c of weight row r at c ^ ((r >> 2) & 3), of activation row r at
// c ^ ((r >> 1) & 7)) so that the 16 lanes of each fragment-read group hit
// distinct banks.  Eight waves (two
// per SIMD), each 128 (n) x 64 (m) with 32x32x16 MFMAs; weight fragments are
// converted exactly from fp8 to bf16 in registers.
//
// Block scales: a wave's 128 weight rows are one scale block, so the scale of
// a 128-wide K block is one number s_kb for the whole wave tile.  The
// accumulator is kept in units of the current block's scale: entering block
// kb it is multiplied by s_{kb-1} / s_kb, and the result is acc * s_last.
// This equals sum_kb s_kb * partial_kb up to fp32 rounding of the ratios
// (~1e-5 relative over 128 blocks, far below the bf16 output rounding).  A
// block with s_kb == 0 dequantises to zero and is skipped.
constexpr int G_BN = 256, G_BM = 256, G_BK = 64, G_NST = 3, G_NW = 8;
constexpr int G_WOFF = 0, G_XOFF = G_BN * G_BK;  // fp8 weight rows, then bf16 activation rows
constexpr int G_STAGE = G_BN * G_BK + G_BM * G_BK * 2;
constexpr int G_LDS = G_NST * G_STAGE;           // 144 KB
constexpr int G_DMA = G_STAGE / 1024 / G_NW;     // copies per wave per stage
constexpr int G_EPITCH = 128 * 2 + 8;           // LDS row pitch of the staged output block
constexpr int G_WAVE_F4 = 4 * 2 * 4 * 64;        // f32x4 partial sums of one wave's 128 x 64 block
constexpr int G_TILE_F4 = G_NW * G_WAVE_F4;      // ... of one 256 x 256 tile (256 KB)
static_assert(G_NW * 64 * G_EPITCH <= G_LDS, "staged output block exceeds LDS");

// One 256 x 256 output tile at (n0, m0) over the 128-wide K blocks
// [kb_begin, kb_end).  partial != nullptr: the tile's fp32 sums (scaled) go to
// partial in the lanes' own order (gemm_finish_kernel sums the K parts),
// else through the epilogue.
template <int MODE>
AMLA_DEV void gemm_body(const GemvParams &p, bool staged_out, const int n0, const int m0, const int kb_begin,
                        const int kb_end, float *partial) {
  extern __shared__ __align__(16) uint8_t gsm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, wm = wave >> 1;
  const int j32 = lane & 31, hh = lane >> 5;
  const bool seg1 = (MODE == GEMV_QKVA || p.w1) && n0 >= p.n_split;
  const uint8_t *W = seg1 ? p.w1 : p.w0;
  const float *S = seg1 ? p.s1 : p.s0;
  const int nl0 = seg1 ? n0 - p.n_split : n0;
  const int nvalid = (seg1 ? p.N - p.n_split : p.n_split) - nl0;  // rows of this segment from nl0
  const int KB = p.K >> 7;
  const bool wave_rows = wn * 128 < nvalid;
  const __attribute__((address_space(4))) float *srow = (const __attribute__((address_space(4))) float *)(
      S + (size_t)((nl0 + min(wn * 128, nvalid - 1)) >> 7) * KB);

  // copies: wave w fills weight rows 32w .. +31 (two copies of 16 rows) and
  // activation rows 32w .. +31 (four copies of 8 rows) of each stage
  const bool wfull = nvalid >= G_BN, xfull = m0 + G_BM <= p.M;
  const uint32_t wrow = (uint32_t)(lane >> 2) * p.K, xrow = (uint32_t)(lane >> 3) * p.ldx * 2;
  auto dma = [&](int it, uint8_t *st) {
    const int k0 = it * G_BK;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r0 = 32 * wave + 16 * j;
      const uint8_t *src;
      if (wfull) {
        src = W + (size_t)(nl0 + r0) * p.K + k0 + wrow + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
      } else {
        const int r = min(r0 + (lane >> 2), nvalid - 1);
        src = W + (size_t)(nl0 + r) * p.K + k0 + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
      }
      __builtin_amdgcn_global_load_lds(src, LDS_PTR(st + G_WOFF + r0 * G_BK), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r0 = 32 * wave + 8 * j;
      const uint8_t *src;
      if (xfull) {
        src = reinterpret_cast<const uint8_t *>(p.x + (size_t)(m0 + r0) * p.ldx + k0) + xrow +
              16 * ((lane & 7) ^ ((4 * j + (lane >> 4)) & 7));
      } else {
        const int r = min(m0 + r0 + (lane >> 3), p.M - 1);
        src = reinterpret_cast<const uint8_t *>(p.x + (size_t)r * p.ldx + k0) +
              16 * ((lane & 7) ^ ((4 * j + (lane >> 4)) & 7));
      }
      __builtin_amdgcn_global_load_lds(src, LDS_PTR(st + G_XOFF + r0 * (G_BK * 2)), 16, 0, 0);
    }
  };

  // fragment offsets: weight rows wn*128 + 32 g + j32, chunk (2 pr + hh) of
  // the 64-byte row (K 32 pr + 16 hh .. +15, two MFMA steps of 8); activation
  // rows wm*64 + 32 j + j32, chunks 4 pr + 2 hh + s (K 32 pr + 16 hh + 8 s ..)
  uint32_t aoff[2], boff[2][2];
#pragma unroll
  for (int pr = 0; pr < 2; ++pr) {
    aoff[pr] = G_WOFF + (wn * 128 + j32) * G_BK + 16 * ((2 * pr + hh) ^ ((j32 >> 2) & 3));
#pragma unroll
    for (int st = 0; st < 2; ++st)
      boff[pr][st] = G_XOFF + (wm * 64 + j32) * (G_BK * 2) + 16 * ((4 * pr + 2 * hh + st) ^ ((j32 >> 1) & 7));
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[g][j][r] = 0.f;
  float s_run = 0.f;
  bool skip = false;

  const int iters = 2 * kb_end;  // 64-wide K stages, two per scale block
  dma(2 * kb_begin, gsm);
  if (2 * kb_begin + 1 < iters) dma(2 * kb_begin + 1, gsm + G_STAGE);
  int stg = 0;
  for (int it = 2 * kb_begin; it < iters; ++it) {
    if (it + 1 < iters) wait_vmcnt<G_DMA>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (it + 2 < iters) dma(it + 2, gsm + (stg == 0 ? 2 : stg - 1) * G_STAGE);
    if ((it & 1) == 0) {
      const float sk = srow[it >> 1];
      skip = sk == 0.f;
      if (!skip) {
        if (s_run != 0.f) {
          const float r = __fdiv_rn(s_run, sk);
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[g][j] *= r;
        }
        s_run = sk;
      }
    }
    if (!skip) {
      const uint8_t *st = gsm + stg * G_STAGE;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        u32x4 araw[4], bx[2][2];
#pragma unroll
        for (int g = 0; g < 4; ++g) araw[g] = *reinterpret_cast<const u32x4 *>(st + aoff[pr] + g * 32 * G_BK);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2)
            bx[j][s2] = *reinterpret_cast<const u32x4 *>(st + boff[pr][s2] + j * 32 * (G_BK * 2));
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
            const uint32_t w0 = araw[g][2 * s2], w1 = araw[g][2 * s2 + 1];
            const bf16x2_t c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, false);
            const bf16x2_t c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, true);
            const bf16x2_t c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, false);
            const bf16x2_t c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, true);
            const bf16x8 a = {c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[g][j] = mfma32(a, as_bf16x8(bx[j][s2]), acc[g][j]);
          }
      }
    }
    stg = stg == G_NST - 1 ? 0 : stg + 1;
  }

  // C[n][m]: lane holds m = 32 j + j32 of its rows, n = 32 g + 8 q + 4 hh .. +3.
  if (partial) {
    // [wave][g][j][q][lane] f32x4: every store is 1 KB contiguous per wave
    f32x4 *dst = reinterpret_cast<f32x4 *>(partial) + (size_t)wave * G_WAVE_F4;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          dst[((g * 2 + j) * 4 + q) * 64 + lane] =
              f32x4{acc[g][j][4 * q], acc[g][j][4 * q + 1], acc[g][j][4 * q + 2], acc[g][j][4 * q + 3]} * s_run;
    return;
  }
  if (!staged_out) {
    // outputs without 16-byte aligned rows: 8-byte stores straight from the accumulators
    if (wave_rows) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int m = m0 + wm * 64 + 32 * j + j32;
        if (m >= p.M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = n0 + wn * 128 + 32 * g + 8 * q + 4 * hh;
            if (n < p.N)
              pstore4<MODE>(p, m, n,
                            f32x4{acc[g][j][4 * q], acc[g][j][4 * q + 1], acc[g][j][4 * q + 2], acc[g][j][4 * q + 3]} *
                                s_run);
          }
      }
    }
    return;
  }
  // bf16(C * s) goes through LDS (this wave's 64 x 128 block, rows of m) so
  // that every global store is 16 bytes of one output row.
  __builtin_amdgcn_s_barrier();  // every wave is past its last fragment read
  asm volatile("" ::: "memory");
  uint8_t *cst = gsm + wave * (64 * G_EPITCH);
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v =
            f32x4{acc[g][j][4 * q], acc[g][j][4 * q + 1], acc[g][j][4 * q + 2], acc[g][j][4 * q + 3]} * s_run;
        *reinterpret_cast<u32x2 *>(cst + (32 * j + j32) * G_EPITCH + (32 * g + 8 * q + 4 * hh) * 2) =
            u32x2{pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
      }
  if (wave_rows) {
    const int c16 = lane & 15;
#pragma unroll 4
    for (int r4 = 0; r4 < 16; ++r4) {
      const int ml = 4 * r4 + (lane >> 4);
      const int m = m0 + wm * 64 + ml, n = n0 + wn * 128 + 8 * c16;
      const u32x4 v = *reinterpret_cast<const u32x4 *>(cst + ml * G_EPITCH + c16 * 16);
      if (m < p.M && n < p.N) pstore8<MODE>(p, m, n, v);
    }
  }
}

// Workgroup i: tile i (t = m_tile * n_tiles + n_tile) with the whole K while
// i < sp.full, else K part (i - full) % parts of tile full + (i - full) / parts.
template <int MODE>
__global__ __launch_bounds__(G_NW * 64, 1) void gemm_kernel(GemvParams p, bool staged_out, GemmSplit sp) {
  const int i = blockIdx.x, KB = p.K >> 7;
  int t = i, kb0 = 0, kb1 = KB;
  float *partial = nullptr;
  if (i >= sp.full) {
    const int st = (i - sp.full) / sp.parts, q = (i - sp.full) % sp.parts;
    t = sp.full + st;
    kb0 = q * KB / sp.parts;
    kb1 = (q + 1) * KB / sp.parts;
    partial = sp.partial + (size_t)(st * sp.parts + q) * G_TILE_F4 * 4;
  }
  gemm_body<MODE>(p, staged_out, (t % sp.n_tiles) * G_BN, (t / sp.n_tiles) * G_BM, kb0, kb1, partial);
}

// Sums the K parts of the split tiles in part order and applies the epilogue.
// Workgroup = one wave block (64 rows x 128 columns) of one split tile: the
// parts are read in the lane order they were written (coalesced), summed in
// part order, staged in LDS as rows, and stored 8 outputs per thread through
// the same epilogue as the staged tiles (16-byte row stores).
template <int MODE>
__global__ __launch_bounds__(256) void gemm_finish_kernel(GemvParams p, GemmSplit sp) {
  __shared__ float rows[64][128 + 4];
  const int tid = threadIdx.x;
  const int st = blockIdx.x / G_NW, wave = blockIdx.x % G_NW;
  const f32x4 *src = reinterpret_cast<const f32x4 *>(sp.partial) + (size_t)st * sp.parts * G_TILE_F4 +
                     (size_t)wave * G_WAVE_F4;
  constexpr int PER = G_WAVE_F4 / 256;  // f32x4 per thread
  f32x4 sum[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) sum[k] = src[k * 256 + tid];
  for (int q = 1; q < sp.parts; ++q) {
    f32x4 v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) v[k] = src[(size_t)q * G_TILE_F4 + k * 256 + tid];
#pragma unroll
    for (int k = 0; k < PER; ++k) sum[k] += v[k];
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int rr = k * 256 + tid;  // ((g * 2 + j) * 4 + q) * 64 + lane
    const int gjq = rr >> 6, lane = rr & 63;
    const int g = gjq >> 3, j = (gjq >> 2) & 1, q = gjq & 3;
    *reinterpret_cast<f32x4 *>(&rows[32 * j + (lane & 31)][32 * g + 8 * q + 4 * (lane >> 5)]) = sum[k];
  }
  __syncthreads();
  const int t = sp.full + st;
  const int m0 = (t / sp.n_tiles) * G_BM + (wave >> 1) * 64, n0 = (t % sp.n_tiles) * G_BN + (wave & 1) * 128;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = k * 256 + tid, r = e >> 4, c = (e & 15) * 8;
    const int m = m0 + r, n = n0 + c;
    if (m < p.M && n < p.N) {
      const float *v = &rows[r][c];
      pstore8<MODE>(p, m, n, u32x4{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                                   pack_bf16(v[6], v[7])});
    }
  }
}

// Tiles of the routed experts from a device schedule: workgroup (x, y) takes
// output columns 256 x of entry y (expert e, rows r0 .. r0 + rows - 1 of x and
// y, rows <= 256); entries past the count return at once.
__global__ __launch_bounds__(G_NW * 64, 1) void gemm_sched_kernel(GemvParams p, MoeSched s) {
  const int t = blockIdx.y;
  if (t >= *s.count) return;
  const int32_t *en = s.ent + 4 * t;
  const int e = en[0], r0 = en[1];
  p.M = en[2];
  p.x += (size_t)r0 * p.ldx;
  p.y += (size_t)r0 * p.ldy;
  moe_sched_weights(p, s, e);
  gemm_body<GEMV_PLAIN>(p, true, blockIdx.x * G_BN, 0, 0, p.K >> 7, nullptr);
}

// Tiles past the last full round of 256 workgroups are cut into K parts so
// that the launch ends with the machine full: time ~ (rounds of 256 work
// items) x (tile time / parts) + the partial sums written and read back (256
// KB per part); a tile's time is taken as proportional to K (~500 us at
// K = 16384 on MI355X), the partial traffic at ~5 TB/s.
GemmSplit plan_gemm_split(int M, int N, int K) {
  GemmSplit sp = {};
  sp.n_tiles = (N + G_BN - 1) / G_BN;
  const int tiles = sp.n_tiles * ((M + G_BM - 1) / G_BM);
  const int KB = K / 128;
  const int full = tiles / 256 * 256, rest = tiles - full;
  const double t_tile = 500.0 * K / 16384.0;  // us
  int best = 1;
  double best_cost = rest ? t_tile : 0.0;
  for (int s = 2; s <= std::min(GEMM_MAX_PARTS, KB) && rest; ++s) {
    const double cost = (double)((rest * s + 255) / 256) * t_tile / s + rest * s * (0.25 * 2 / 5e6 * 1e6);
    if (cost < best_cost * 0.95) {
      best_cost = cost;
      best = s;
    }
  }
  sp.full = best > 1 ? full : tiles;
  sp.parts = best;
  sp.items = sp.full + (tiles - sp.full) * best;
  sp.bytes = best > 1 ? (size_t)(tiles - sp.full) * best * G_TILE_F4 * 16 : 0;
  return sp;
}

size_t gemm_ws_bytes(int M, int N, int K) { return plan_gemm_split(M, N, K).bytes; }

int launch_gemm(const GemvParams &p, int mode, hipStream_t st, float *split_ws, size_t split_ws_bytes) {
  if (p.K % 128 || p.N % 4) return fail(AMLA_EUNSUPPORTED, "fp8 GEMM needs K %% 128 == 0 and N %% 4 == 0");
  if (p.ldx % 8) return fail(AMLA_EUNSUPPORTED, "fp8 GEMM needs 16-byte aligned activation rows");
  if ((mode == GEMV_QKVA && p.max_rows <= 0) || (mode == GEMV_QROPE && p.rope_rows <= 0))
    return fail(AMLA_EINVAL, "fp8 GEMM: cache rows / rope rows of the epilogue not set");
  if ((mode == GEMV_QKVA || p.w1) && p.n_split % G_BN)
    return fail(AMLA_EUNSUPPORTED, "fp8 GEMM: the first weight segment must be a multiple of 256 rows");
  static bool attr_set[5] = {false, false, false, false, false};  // dynamic LDS above 64 KB, once per mode
  const void *fn = mode == GEMV_PLAIN  ? (const void *)gemm_kernel<GEMV_PLAIN>
                   : mode == GEMV_RESID ? (const void *)gemm_kernel<GEMV_RESID>
                   : mode == GEMV_QKVA  ? (const void *)gemm_kernel<GEMV_QKVA>
                   : mode == GEMV_F32   ? (const void *)gemm_kernel<GEMV_F32>
                                        : (const void *)gemm_kernel<GEMV_QROPE>;
  if (mode < 0 || mode > 4) return fail(AMLA_EINVAL, "fp8 GEMM: unknown epilogue mode %d", mode);
  if (!attr_set[mode]) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, G_LDS);
    attr_set[mode] = true;
  }
  // 16-byte output stores need N, the row strides and the bases of every
  // output (and of the residual) on 8-element boundaries
  bool staged = p.N % 8 == 0 && p.ldy % 8 == 0 && aligned16(p.y);
  if (mode == GEMV_RESID) staged = staged && p.ldr % 8 == 0 && aligned16(p.res);
  if (mode == GEMV_QKVA)
    staged = staged && aligned16(p.ckv) && aligned16(p.kpe) && p.kv_lora % 8 == 0 && p.rope % 8 == 0 &&
             p.ckv_bstride % 8 == 0 && p.kpe_bstride % 8 == 0;
  if (mode == GEMV_QROPE) staged = staged && p.head_dim % 8 == 0 && p.nope % 8 == 0;
  if (mode == GEMV_F32) staged = false;  // fp32 rows: 16-byte stores of four outputs from the accumulators
  GemmSplit sp = plan_gemm_split(p.M, p.N, p.K);
  if (sp.parts > 1 && (!staged || !split_ws || split_ws_bytes < sp.bytes || !aligned16(split_ws))) {
    // no room for the partial sums (or outputs without 16-byte stores): whole tiles
    sp.full = sp.items = sp.n_tiles * ((p.M + G_BM - 1) / G_BM);
    sp.parts = 1;
  }
  sp.partial = split_ws;
  const dim3 grid(sp.items);
  switch (mode) {
    case GEMV_PLAIN: gemm_kernel<GEMV_PLAIN><<<grid, G_NW * 64, G_LDS, st>>>(p, staged, sp); break;
    case GEMV_RESID: gemm_kernel<GEMV_RESID><<<grid, G_NW * 64, G_LDS, st>>>(p, staged, sp); break;
    case GEMV_QKVA: gemm_kernel<GEMV_QKVA><<<grid, G_NW * 64, G_LDS, st>>>(p, staged, sp); break;
    case GEMV_F32: gemm_kernel<GEMV_F32><<<grid, G_NW * 64, G_LDS, st>>>(p, staged, sp); break;
    default: gemm_kernel<GEMV_QROPE><<<grid, G_NW * 64, G_LDS, st>>>(p, staged, sp); break;
  }
  int rc = check_launch("fp8 GEMM");
  if (rc || sp.parts == 1) return rc;
  const dim3 fgrid((unsigned)((sp.items - sp.full) / sp.parts * G_NW));
  switch (mode) {
    case GEMV_PLAIN: gemm_finish_kernel<GEMV_PLAIN><<<fgrid, 256, 0, st>>>(p, sp); break;
    case GEMV_RESID: gemm_finish_kernel<GEMV_RESID><<<fgrid, 256, 0, st>>>(p, sp); break;
    case GEMV_QKVA: gemm_finish_kernel<GEMV_QKVA><<<fgrid, 256, 0, st>>>(p, sp); break;
    default: gemm_finish_kernel<GEMV_QROPE><<<fgrid, 256, 0, st>>>(p, sp); break;
  }
  return check_launch("fp8 GEMM K-part finish");
}

int launch_gemm_sched(const GemvParams &p, const MoeSched &s, int max_entries, hipStream_t st) {
  if (max_entries <= 0) return AMLA_OK;
  if (p.K % 128 || p.N % 8 || p.ldx % 8 || p.ldy % 8 || !aligned16(p.x) || !aligned16(p.y))
    return fail(AMLA_EUNSUPPORTED, "scheduled fp8 GEMM needs K %% 128 == 0, N %% 8 == 0 and 16-byte aligned rows");
  if (!s.down && p.n_split % G_BN)
    return fail(AMLA_EUNSUPPORTED, "scheduled fp8 GEMM: the first weight segment must be a multiple of 256 rows");
  if (max_entries > 65535) return fail(AMLA_EUNSUPPORTED, "scheduled fp8 GEMM: %d entries", max_entries);
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void *)gemm_sched_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, G_LDS);
    attr_set = true;
  }
  gemm_sched_kernel<<<dim3((p.N + G_BN - 1) / G_BN, max_entries), G_NW * 64, G_LDS, st>>>(p, s);
  return check_launch("scheduled fp8 GEMM");
}

// ---------------------------------------------------------------- K10 causal flash attention

constexpr int P_NOPE = 128, P_ROPE = 64, P_QK = 192, P_V = 128, P_H = 128;
constexpr int P_KVROW = P_H * (P_NOPE + P_V) * 2;  // bytes per kv_b output row (all heads)
constexpr int F_KT = 64;                           // keys per tile
constexpr int F_NQG = 1;                           // groups of 32 queries per wave
constexpr int F_QW = 32 * F_NQG;                   // queries per wave
constexpr int F_NW = 8;                            // waves per workgroup (two per SIMD)
constexpr int F_QB = F_NW * F_QW;                  // queries per workgroup
constexpr int F_RPW = F_KT / F_NW;                 // key rows each wave copies per tile
constexpr int F_NST = 3;                           // LDS stages (copies run two tiles ahead)
// one stage: k_nope as two arrays of 128 B half-rows (dims 0-63 of every key,
// then dims 64-127), rope-key rows (128 B), values as two arrays of 128 B
// half-rows.  A 16-byte LDS read is served 16 consecutive lanes per pass, free
// of bank conflicts when their addresses differ in bits 4-7 (measured on
// MI355X: any two of the 16 equal there cost a second pass); a transpose read
// serves 64 lanes over a 512 B window.  So chunk c of a k_nope / rope half-row
// r sits at c ^ ((r >> 1) & 7) (the 16 key rows of a fragment read pass: two
// parities of the row x eight slots), and the 64-byte segment g of a value
// half-row at g ^ ((r >> 2) & 1) (the 8 x 64 B of a transpose read cover the
// window once).
constexpr int F_HALF = F_KT * 128;                 // one array of half-rows
constexpr int F_NOPE = 0, F_RPE = 2 * F_HALF, F_VAL = 3 * F_HALF;
constexpr int F_STAGE = F_VAL + 2 * F_HALF;        // 40 KB
constexpr int F_LDS = F_NST * F_STAGE;
constexpr int F_DMA = 5 * F_RPW / 8;               // copies per wave per tile

struct FlashParams {
  const uint16_t *q;      // (rows, H, 192): row = b*S + s, q_pe already rotated
  const uint16_t *kvb;    // (Tmax, H*256): k_nope | v per head
  const uint16_t *kpe;    // (Tmax, 64) rotated rope keys
  uint16_t *out;          // (rows, H*128)
  const int32_t *pos;
  int b, S, nqb;  // nqb: query blocks of 256 per head
  int tmax;       // key rows held (first positions are clamped to tmax - S)
  float scale_log2;
};

// Wave w copies key rows F_RPW w .. +F_RPW-1 of the tile (both k_nope halves,
// both value halves and the rope key) straight into LDS: each global_load_lds
// writes 64 lanes x 16 B contiguously (8 half-rows), so the swizzle is applied
// to the source chunk each lane fetches.  Inside the keys in use the row bases
// are scalar and each lane adds a fixed offset; the tile that crosses Tlim
// clamps rows to Tlim - 1 per lane (in bounds; their scores are masked).
struct FlashLane {
  uint32_t nope;  // lane offset of k_nope copies (row r8 of 8, swizzled chunk; + 128 B for the second half)
  uint32_t val;   // lane offset of value copies (+ 128 B for the second half)
  uint32_t rope;  // lane offset of rope-key copies
};

// chunk of a k_nope / rope half-row slot c8 of copy row r8 (key row 8 w + r8) holds
AMLA_DEV int flash_kchunk(int wave, int lane) { return (lane & 7) ^ ((4 * wave + (lane >> 4)) & 7); }
// chunk of a value half-row slot c8 holds (the 64-byte segment moves with bit 2 of the row)
AMLA_DEV int flash_vchunk(int lane) { return (lane & 7) ^ (4 * ((lane >> 5) & 1)); }

AMLA_DEV FlashLane flash_lane(int wave, int lane) {
  const int r8 = lane >> 3;
  FlashLane fl;
  fl.nope = r8 * P_KVROW + 16 * flash_kchunk(wave, lane);
  fl.val = r8 * P_KVROW + P_NOPE * 2 + 16 * flash_vchunk(lane);
  fl.rope = r8 * (P_ROPE * 2) + 16 * flash_kchunk(wave, lane);
  return fl;
}

AMLA_DEV void flash_dma(const FlashParams &p, int h, int t0, int Tlim, uint8_t *stage, int wave, int lane,
                        const FlashLane &fl) {
  static_assert(F_RPW == 8, "one copy covers the 8 rows of a wave");
  const char *kv = reinterpret_cast<const char *>(p.kvb) + h * ((P_NOPE + P_V) * 2);
  const char *kr = reinterpret_cast<const char *>(p.kpe);
  const int row = F_RPW * wave;
  if (t0 + F_KT <= Tlim) {
    const char *kvw = kv + (size_t)(t0 + row) * P_KVROW;
    const char *krw = kr + (size_t)(t0 + row) * (P_ROPE * 2);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      __builtin_amdgcn_global_load_lds(kvw + 128 * half + fl.nope, LDS_PTR(stage + F_NOPE + half * F_HALF + row * 128),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(kvw + 128 * half + fl.val, LDS_PTR(stage + F_VAL + half * F_HALF + row * 128),
                                       16, 0, 0);
    }
    __builtin_amdgcn_global_load_lds(krw + fl.rope, LDS_PTR(stage + F_RPE + row * 128), 16, 0, 0);
    return;
  }
  const int t = min(t0 + row + (lane >> 3), Tlim - 1);
  const char *src = kv + (size_t)t * P_KVROW;
  const int kc = flash_kchunk(wave, lane), vc = flash_vchunk(lane);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __builtin_amdgcn_global_load_lds(src + 128 * half + 16 * kc, LDS_PTR(stage + F_NOPE + half * F_HALF + row * 128),
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds(src + P_NOPE * 2 + 128 * half + 16 * vc,
                                     LDS_PTR(stage + F_VAL + half * F_HALF + row * 128), 16, 0, 0);
  }
  __builtin_amdgcn_global_load_lds(kr + (size_t)t * (P_ROPE * 2) + 16 * kc, LDS_PTR(stage + F_RPE + row * 128), 16,
                                   0, 0);
}

// Copy PIECE (0 .. F_DMA-1) of a tile wholly inside the keys in use: k_nope
// halves, value halves, then the rope keys.
AMLA_DEV void flash_dma_piece(const FlashParams &p, int h, int t0, uint8_t *stage, int wave, const FlashLane &fl,
                              int piece) {
  const int row = F_RPW * wave;
  const char *kvw = reinterpret_cast<const char *>(p.kvb) + h * ((P_NOPE + P_V) * 2) + (size_t)(t0 + row) * P_KVROW;
  if (piece < 2) {
    __builtin_amdgcn_global_load_lds(kvw + 128 * piece + fl.nope, LDS_PTR(stage + F_NOPE + piece * F_HALF + row * 128),
                                     16, 0, 0);
  } else if (piece < 4) {
    const int half = piece - 2;
    __builtin_amdgcn_global_load_lds(kvw + 128 * half + fl.val, LDS_PTR(stage + F_VAL + half * F_HALF + row * 128),
                                     16, 0, 0);
  } else {
    const char *krw = reinterpret_cast<const char *>(p.kpe) + (size_t)(t0 + row) * (P_ROPE * 2);
    __builtin_amdgcn_global_load_lds(krw + fl.rope, LDS_PTR(stage + F_RPE + row * 128), 16, 0, 0);
  }
}

// Grid H x (query blocks of 256), 256 threads, 120 KB of LDS: one workgroup
// per CU.  Wave w handles queries qb*256 + 64w .. +63 of head h, in two
// groups of 32.  Per 64-key tile:
//   S^T (keys x queries) = K (keys x 192) . Q^T     32x32x16 MFMAs, A = K rows
//   online softmax in registers: lane l holds 16 keys of query l%32 per
//     32-key group (the other 16 sit in lane l^32)
//   O^T (128 x queries) += V^T (128 x keys) . P^T   B = P straight from the
//     score registers, A = V^T by transpose reads
// The running max moves only when a score exceeds it by more than 2^8, so the
// O rescale is rare; exp2 arguments stay <= 8 and the final 1/l is exact.
__global__ __launch_bounds__(F_NW * 64, 1) void flash_kernel(FlashParams p) {
  extern __shared__ __align__(16) uint8_t fsm[];
  // Workgroup i runs on XCD i % 8 (round-robin dispatch): XCD x takes heads
  // x*H/8 .. +H/8-1, one head at a time with all its query blocks, heaviest
  // first, so a head's keys and values are read from HBM about once per XCD
  // and shared through that XCD's L2.
  const int nqb = p.nqb;
  const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int h = xcd * (P_H / 8) + k / nqb;
  const int qblk = nqb - 1 - k % nqb;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j32 = lane & 31, hh = lane >> 5;
  const int pos0 = min(p.pos[p.b], p.tmax - p.S);  // keys [0, pos0 + S) are in the workspace
  const int s_begin = qblk * F_QB;
  const int s_wave = s_begin + wave * F_QW;
  const int s_last_blk = min(s_begin + F_QB, p.S) - 1;
  const int Tlim = pos0 + s_last_blk + 1;  // keys needed by this block
  const int ntiles = (Tlim + F_KT - 1) / F_KT;
  const bool wave_active = s_wave < p.S;
  const int wave_last_pos = pos0 + min(s_wave + F_QW, p.S) - 1;
  const float sl2 = p.scale_log2;

  const FlashLane fl = flash_lane(wave, lane);
  flash_dma(p, h, 0, Tlim, fsm, wave, lane, fl);

  // Q^T fragments: column = query s_wave + 32 qg + j32, dims 16 ks + 8 hh .. +7
  bf16x8 qf[F_NQG][P_QK / 16];
#pragma unroll
  for (int qg = 0; qg < F_NQG; ++qg) {
    const int s = min(s_wave + 32 * qg + j32, p.S - 1);
    const uint16_t *qr = p.q + ((size_t)(p.b * p.S + s) * P_H + h) * P_QK + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < P_QK / 16; ++ks) qf[qg][ks] = as_bf16x8(ldg16(qr + 16 * ks));
  }
  if (ntiles > 1) flash_dma(p, h, F_KT, Tlim, fsm + F_STAGE, wave, lane, fl);
  f32x16 o[4][F_NQG];
  float m_run[F_NQG], l_run[F_NQG];
#pragma unroll
  for (int qg = 0; qg < F_NQG; ++qg) {
#pragma unroll
    for (int vt = 0; vt < 4; ++vt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[vt][qg][r] = 0.f;
    m_run[qg] = -INFINITY;
    l_run[qg] = 0.f;
  }

  // per-lane LDS offsets.  K fragment (A of S^T): key row 32 kg + j32, chunk
  // 2 ks + hh of half-row array ks / 4 (arrays 0, 1: k_nope; 2: rope), at slot
  // (2 ks + hh) ^ ((j32 >> 1) & 7).  V^T by ds_read_b64_tr_b16: in a 16-lane
  // group g, lane L addresses value row t + L/4 and columns c0 + 4 (L%4) .. +3
  // with c0 = 32 vt + 16 (g & 1), and receives column c0 + L of rows t .. t+3;
  // rows t = 8i + 4 hh, so the segment of column block vt sits at (vt & 1) ^ hh.
  const int L16 = lane & 15, g16 = lane >> 4;
  const int vrow = L16 >> 2;
  int koff[4];
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4) koff[k4] = F_NOPE + j32 * 128 + 16 * ((2 * k4 + hh) ^ ((j32 >> 1) & 7));
  int voff[2];  // vt even / odd
#pragma unroll
  for (int par = 0; par < 2; ++par)
    voff[par] = F_VAL + (4 * hh + vrow) * 128 + 64 * (par ^ hh) + 32 * (g16 & 1) + 8 * (L16 & 3);

  // ---- software pipeline over 32-key groups g (tile g/2, half g%2).  Step
  // A of g computes S_{g+1} while exponentiating group g; step B accumulates
  // PV_g while masking and maximising group g+1, then moves the running max
  // (rare O rescale).  Even groups live in scA, odd ones in scB.  Every wave
  // runs all groups of the block; groups past its queries are fully masked.
  const uint32_t lds0 = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t *)fsm));
  uint32_t kb[4], vb0, vb1;
  f32x16 scA[F_NQG], scB[F_NQG];
  u32x4 pb[F_NQG][2];  // [qg][16-key step]: bf16 P of the group being accumulated
  float nm[F_NQG];     // -running max (scaled) per query group
  float mx[F_NQG];
  int lim0[F_NQG];     // query position - first key of the lane's rows, for group 0
#pragma unroll
  for (int qg = 0; qg < F_NQG; ++qg) lim0[qg] = pos0 + s_wave + 32 * qg + j32 - 4 * hh;
  constexpr int FD = 4;

#define FL_KBASE(STG)                                      \
  {                                                        \
    const uint32_t sb_ = lds0 + (STG) * F_STAGE;           \
    _Pragma("unroll") for (int k4 = 0; k4 < 4; ++k4) kb[k4] = sb_ + koff[k4]; \
  }
#define FL_VBASE(STG)                                      \
  {                                                        \
    const uint32_t sb_ = lds0 + (STG) * F_STAGE;           \
    vb0 = sb_ + voff[0];                                   \
    vb1 = sb_ + voff[1];                                   \
  }
#define FL_RDK(D, KS, KG)                                                                      \
  asm volatile("ds_read_b128 %0, %1 offset:%2"                                                \
               : "=v"(D)                                                                      \
               : "v"(kb[(KS) & 3]), "i"(((KS) >> 2) * F_HALF + (KG) * 32 * 128)             \
               : "memory")
  // exp slice q4 of query group QG of SCE (rows 4 q4 .. +3) -> pb, l.  The
  // empty asm statements pin each slice between the MFMAs it is meant to
  // overlap (IR passes would otherwise sink it next to its first use).
#define FL_EXP(SCE, QG, Q4)                                                                         \
  {                                                                                                \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                                \
      SCE[QG][4 * (Q4) + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(SCE[QG][4 * (Q4) + i], sl2, nm[QG])); \
      asm volatile("" : "+v"(SCE[QG][4 * (Q4) + i]));                                               \
    }                                                                                              \
    if ((Q4) & 1) {                                                                                \
      const int b_ = 8 * ((Q4) >> 1);                                                              \
      const u32x4 pk_ = {pack_bf16(SCE[QG][b_], SCE[QG][b_ + 1]), pack_bf16(SCE[QG][b_ + 2], SCE[QG][b_ + 3]), \
                         pack_bf16(SCE[QG][b_ + 4], SCE[QG][b_ + 5]), pack_bf16(SCE[QG][b_ + 6], SCE[QG][b_ + 7])}; \
      pb[QG][(Q4) >> 1] = pk_;                                                                     \
      asm volatile("" : "+v"(pb[QG][(Q4) >> 1]));                                                  \
      _Pragma("unroll") for (int i = 0; i < 8; ++i) l_run[QG] += SCE[QG][b_ + i];                    \
      asm volatile("" : "+v"(l_run[QG]));                                                          \
    }                                                                                              \
  }
  // S^T of one 32-key group (half KG of the stage in kb/rb) into SC; with
  // DOEXP, the exp of SCE rides along (8 slices over the first 8 K steps)
#define FL_S(SC, KG, SCE, DOEXP, DMAT, DMAST)                                                       \
  {                                                                                                \
    u32x4 ka[FD];                                                                                  \
    _Pragma("unroll") for (int d = 0; d < FD; ++d) FL_RDK(ka[d], d, KG);                          \
    _Pragma("unroll") for (int ks = 0; ks < 12; ++ks) {                                            \
      const int c = ks % FD;                                                                       \
      const int later = (11 - ks) < (FD - 1) ? (11 - ks) : (FD - 1);                              \
      if (later == 3) asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(ka[c])::"memory");               \
      else if (later == 2) asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(ka[c])::"memory");          \
      else if (later == 1) asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(ka[c])::"memory");          \
      else asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ka[c])::"memory");                          \
      _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) {                                       \
        if (ks == 0)                                                                               \
          asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0"                          \
                       : "=&v"(SC[qg])                                                             \
                       : "v"(ka[c]), "a"(qf[qg][ks]));                                             \
        else                                                                                       \
          asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"                                    \
                       : "+v"(SC[qg])                                                              \
                       : "v"(ka[c]), "a"(qf[qg][ks]));                                             \
      }                                                                                            \
      if (ks + FD < 12) FL_RDK(ka[c], ks + FD, KG);                                               \
      if ((DMAT) >= 0 && ks < F_DMA) flash_dma_piece(p, h, (DMAT) * F_KT, DMAST, wave, fl, ks);     \
      __builtin_amdgcn_sched_barrier(0);                                                           \
      if ((DOEXP) && ks < 4 * F_NQG) FL_EXP(SCE, ks >> 2, ks & 3);                                 \
      __builtin_amdgcn_sched_barrier(0);                                                           \
    }                                                                                              \
    /* MFMA results are read by VALU code the compiler schedules: cover the */                     \
    /* write-to-read wait states of the asm MFMAs above */                                         \
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");                                   \
    _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) asm volatile("" : "+v"(SC[qg]));            \
  }
  // mask (keys of group GI past the lane's query) and max slice I of SCN
#define FL_MAXS(SCN, I, GI, MASKED)                                                                \
  {                                                                                                \
    const int qg_ = (I) >> 2, r0_ = 4 * ((I) & 3);                                                 \
    if (MASKED) {                                                                                  \
      const int lim_ = lim0[qg_] - 32 * (GI);                                                      \
      _Pragma("unroll") for (int i = 0; i < 4; ++i) if (8 * ((r0_ + i) >> 2) + ((r0_ + i) & 3) > lim_) \
          SCN[qg_][r0_ + i] = -INFINITY;                                                           \
    }                                                                                              \
    mx[qg_] = __builtin_fmaxf(__builtin_fmaxf(mx[qg_], SCN[qg_][r0_]), SCN[qg_][r0_ + 1]);        \
    mx[qg_] = __builtin_fmaxf(__builtin_fmaxf(mx[qg_], SCN[qg_][r0_ + 2]), SCN[qg_][r0_ + 3]);    \
    asm volatile("" : "+v"(mx[qg_]));                                                              \
  }
#define FL_TR(D, BASE, OFS)                                                                          \
  asm volatile(                                                                                     \
      "ds_read_b64_tr_b16 %0, %4 offset:%5\n\tds_read_b64_tr_b16 %1, %4 offset:%6\n\t"              \
      "ds_read_b64_tr_b16 %2, %4 offset:%7\n\tds_read_b64_tr_b16 %3, %4 offset:%8"                  \
      : "=&v"(D[0]), "=&v"(D[1]), "=&v"(D[2]), "=&v"(D[3])                                          \
      : "v"(BASE), "i"(OFS), "i"(OFS + 1024), "i"(OFS + 2048), "i"(OFS + 3072)                      \
      : "memory")
#define FL_WAIT(N, D) \
  asm volatile("s_waitcnt lgkmcnt(" #N ")" : "+v"(D[0]), "+v"(D[1]), "+v"(D[2]), "+v"(D[3])::"memory")
  // PV of one 16-key step kk of 32-column block VT, then max slice 2 VT + kk of SCN
#define FL_PVSTEP(VT, D, KK, SCN, GI, DOMAX, MASKED)                                                  \
  {                                                                                                  \
    const bf16x8 a_ = as_bf16x8(u32x4{D[2 * (KK)].x, D[2 * (KK)].y, D[2 * (KK) + 1].x, D[2 * (KK) + 1].y}); \
    _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) o[VT][qg] = mfma32(a_, as_bf16x8(pb[qg][KK]), o[VT][qg]); \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    if ((DOMAX) && 2 * (VT) + (KK) < 4 * F_NQG) FL_MAXS(SCN, 2 * (VT) + (KK), GI, MASKED);          \
    __builtin_amdgcn_sched_barrier(0);                                                               \
  }
  // O^T += V^T P^T for the group in half KG of the stage in vb0/vb1 (three
  // column blocks of transpose reads in flight); with DOMAX the mask/max of
  // SCN (group GI) rides along
#define FL_PV(KG, SCN, GI, DOMAX, MASKED)                                                             \
  {                                                                                                  \
    if (DOMAX) _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) mx[qg] = -INFINITY;              \
    u32x2 tv[3][4];                                                                                  \
    FL_TR(tv[0], vb0, (KG) * 4096);                                                                  \
    FL_TR(tv[1], vb1, (KG) * 4096);                                                                  \
    FL_TR(tv[2], vb0, (KG) * 4096 + F_HALF);                                                         \
    FL_WAIT(8, tv[0]);                                                                               \
    FL_PVSTEP(0, tv[0], 0, SCN, GI, DOMAX, MASKED);                                                  \
    FL_PVSTEP(0, tv[0], 1, SCN, GI, DOMAX, MASKED);                                                  \
    FL_TR(tv[0], vb1, (KG) * 4096 + F_HALF);                                                         \
    FL_WAIT(8, tv[1]);                                                                               \
    FL_PVSTEP(1, tv[1], 0, SCN, GI, DOMAX, MASKED);                                                  \
    FL_PVSTEP(1, tv[1], 1, SCN, GI, DOMAX, MASKED);                                                  \
    FL_WAIT(4, tv[2]);                                                                               \
    FL_PVSTEP(2, tv[2], 0, SCN, GI, DOMAX, MASKED);                                                  \
    FL_PVSTEP(2, tv[2], 1, SCN, GI, DOMAX, MASKED);                                                  \
    FL_WAIT(0, tv[0]);                                                                               \
    FL_PVSTEP(3, tv[0], 0, SCN, GI, DOMAX, MASKED);                                                  \
    FL_PVSTEP(3, tv[0], 1, SCN, GI, DOMAX, MASKED);                                                  \
  }
  // running max after the group's scores are maximised; O and l rescale when it moves
#define FL_MAXFIN()                                                                                 \
  {                                                                                                \
    bool grow_[F_NQG], any_ = false;                                                               \
    float mn_[F_NQG];                                                                              \
    _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) {                                         \
      const auto sw_ = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx[qg]), __float_as_uint(mx[qg]), false, false); \
      mn_[qg] = __builtin_fmaxf(__uint_as_float(sw_[0]), __uint_as_float(sw_[1])) * sl2;           \
      grow_[qg] = mn_[qg] > m_run[qg] + 8.f;                                                       \
      any_ = any_ || grow_[qg];                                                                    \
    }                                                                                              \
    if (__builtin_amdgcn_ballot_w64(any_)) {                                                       \
      _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) {                                       \
        const float alpha_ = grow_[qg] ? __builtin_amdgcn_exp2f(m_run[qg] - mn_[qg]) : 1.f;        \
        m_run[qg] = grow_[qg] ? mn_[qg] : m_run[qg];                                               \
        l_run[qg] *= alpha_;                                                                       \
        _Pragma("unroll") for (int vt = 0; vt < 4; ++vt) o[vt][qg] *= alpha_;                     \
      }                                                                                            \
    }                                                                                              \
    _Pragma("unroll") for (int qg = 0; qg < F_NQG; ++qg) nm[qg] = -m_run[qg];                      \
  }

  // prologue: tile 0 landed; S_0 and its max
  if (ntiles > 1) wait_vmcnt<F_DMA>();
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  FL_KBASE(0);
  FL_S(scA, 0, scB, 0, -1, fsm);
#pragma unroll
  for (int qg = 0; qg < F_NQG; ++qg) mx[qg] = -INFINITY;
  {
    const bool diag = 31 > pos0 + s_wave;
#pragma unroll
    for (int i = 0; i < 4 * F_NQG; ++i) FL_MAXS(scA, i, 0, diag);
  }
  FL_MAXFIN();

  int stg = 0;  // stage of tile j
  for (int j = 0; j < ntiles; ++j) {
    const int g = 2 * j;
    // ---- group g (even): S_{g+1} (same tile, half 1) || exp of scA; PV_g || max of scB.
    // Wave priority by phase: score steps 2, PV steps 1, the rest (max update,
    // waits, barrier) 0, so the two waves of a SIMD drift apart and one fills
    // the other's gaps (flash 882 -> 865 us at S = 4096 with the score steps
    // raised, a further 1.3 % with the PV steps between; a fixed priority per
    // wave gained nothing, the prologue's score step raised lost 1.5 %)
    __builtin_amdgcn_s_setprio(2);
    FL_S(scB, 1, scA, 1, -1, fsm);
    __builtin_amdgcn_s_setprio(0);
    FL_VBASE(stg);
    {
      const bool diag = 32 * (g + 1) + 31 > pos0 + s_wave;
      __builtin_amdgcn_s_setprio(1);
      FL_PV(0, scB, g + 1, 1, diag);
      __builtin_amdgcn_s_setprio(0);
    }
    FL_MAXFIN();
    // ---- group g+1 (odd): S_{g+2} (tile j+1, half 0) || exp of scB; PV_{g+1} || max of scA.
    // After the last tile S_{g+2} re-reads the current stage and is discarded.
    const bool more = j + 1 < ntiles;
    int stn = stg;
    int dmat = -1;  // tile whose copies go out one per score step below (wholly inside the keys in use)
    if (more) {
      // tile j+1 landed in every wave; tile j-1's stage is free for tile j+2
      wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      stn = stg == F_NST - 1 ? 0 : stg + 1;
      if (j + 2 < ntiles) {
        if ((j + 3) * F_KT <= Tlim) dmat = j + 2;
        else flash_dma(p, h, (j + 2) * F_KT, Tlim, fsm + (stn == F_NST - 1 ? 0 : stn + 1) * F_STAGE, wave, lane, fl);
      }
    }
    FL_KBASE(stn);
    __builtin_amdgcn_s_setprio(2);
    FL_S(scA, 0, scB, 1, dmat, fsm + (stn == F_NST - 1 ? 0 : stn + 1) * F_STAGE);
    __builtin_amdgcn_s_setprio(0);
    {
      const bool diag = 32 * (g + 2) + 31 > pos0 + s_wave;
      __builtin_amdgcn_s_setprio(1);
      FL_PV(1, scA, g + 2, 1, diag);
      __builtin_amdgcn_s_setprio(0);
    }
    if (more) FL_MAXFIN();
    stg = stn;
  }
#undef FL_KBASE
#undef FL_VBASE
#undef FL_RDK
#undef FL_EXP
#undef FL_S
#undef FL_MAXS
#undef FL_TR
#undef FL_WAIT
#undef FL_PVSTEP
#undef FL_PV
#undef FL_MAXFIN
  wait_vmcnt<0>();

  // normalise and store: lane holds query 32 qg + j32, values 32 vt + 8 (r/4) + 4 hh + r%4
#pragma unroll
  for (int qg = 0; qg < F_NQG; ++qg) {
    float l = l_run[qg];
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
      l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const int s = s_wave + 32 * qg + j32;
    if (!wave_active || s >= p.S) continue;
    const float inv = 1.f / l;
    uint16_t *dst = p.out + (size_t)(p.b * p.S + s) * (P_H * P_V) + h * P_V + 4 * hh;
#pragma unroll
    for (int vt = 0; vt < 4; ++vt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x16 &v = o[vt][qg];
        *reinterpret_cast<u32x2 *>(dst + 32 * vt + 8 * q4) =
            u32x2{pack_bf16(v[4 * q4] * inv, v[4 * q4 + 1] * inv), pack_bf16(v[4 * q4 + 2] * inv, v[4 * q4 + 3] * inv)};
      }
  }
}

// ---------------------------------------------------------------- orchestration

// p.part (lin_bytes) holds the K-part sums of the skinny plan or the split
// GEMM's partial sums (PrefillLayout::lin)
static int run_linear(const GemvParams &p, int mode, hipStream_t st, size_t lin_bytes) {
  if (p.M <= 64) return launch_gemv(p, mode, plan_linear(p.M, p.N, p.K), st);
  return launch_gemm(p, mode, st, p.part, lin_bytes);
}

struct PrefillLayout {
  size_t xn, qa, qan, q, kvn, kpe, kvb, attn, lin, lin_bytes, total;
  int Tmax;
};

static PrefillLayout prefill_layout(const amla_mla_args &a) {
  PrefillLayout L = {};
  const size_t M = (size_t)a.batch * a.seq_len;
  const int HD = a.qk_nope + a.qk_rope;
  L.Tmax = std::min(mla_context_bound(a), a.max_seq);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes, 256); return o; };
  L.xn = take(M * a.hidden * 2);
  L.qa = take(M * a.q_lora * 2);
  L.qan = take(M * a.q_lora * 2);
  L.q = take(M * a.heads * HD * 2);
  L.kvn = take((size_t)L.Tmax * a.kv_lora * 2);
  L.kpe = take((size_t)L.Tmax * a.qk_rope * 2);
  L.kvb = take((size_t)L.Tmax * a.heads * (a.qk_nope + a.v_dim) * 2);
  L.attn = take(M * a.heads * a.v_dim * 2);
  // K-part sums of the skinny linears (M <= 64), or the K-split partial sums
  // of the large-M GEMMs
  size_t lin = 0;
  const int HDv = a.qk_nope + a.v_dim;
  auto need = [&](int m, int n, int k) {
    lin = std::max(lin, m <= 64 ? plan_linear(m, n, k).part_bytes : gemm_ws_bytes(m, n, k));
  };
  need((int)M, a.q_lora + a.kv_lora + a.qk_rope, a.hidden);
  need((int)M, a.heads * HD, a.q_lora);
  need(L.Tmax, a.heads * HDv, a.kv_lora);
  need((int)M, a.hidden, a.heads * a.v_dim);
  L.lin = take(lin);
  L.lin_bytes = lin;
  L.total = off;
  return L;
}

// rope of the cached rope-key rows [0, T) of one sequence with table rows [0, T)
__global__ __launch_bounds__(256) void kpe_rope_kernel(const uint16_t *__restrict__ kpe, const float *__restrict__ tab,
                                                       int T, uint16_t *__restrict__ out) {
  const int e = blockIdx.x * 256 + threadIdx.x;  // one pair
  if (e >= T * (P_ROPE / 2)) return;
  const int t = e / (P_ROPE / 2), i = e % (P_ROPE / 2);
  const uint32_t x = reinterpret_cast<const uint32_t *>(kpe)[e];
  const float a = lo_bf(x), b = hi_bf(x);
  const float c = tab[((size_t)t * (P_ROPE / 2) + i) * 2], s = tab[((size_t)t * (P_ROPE / 2) + i) * 2 + 1];
  reinterpret_cast<uint32_t *>(out)[e] =
      pack_bf16(__fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s)), __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c)));
}

int prefill_impl(const amla_mla_args *a, hipStream_t st);

}  // namespace amla

namespace amla {

int prefill_impl(const amla_mla_args *a, hipStream_t st) {
  int rc = check_mla_common(a, "mla_prefill");
  if (rc) return rc;
  const PrefillLayout L = prefill_layout(*a);
  if (a->workspace_bytes < L.total)
    return fail(AMLA_EWORKSPACE, "mla_prefill: workspace %zu bytes < %zu needed", a->workspace_bytes, L.total);
  char *ws = reinterpret_cast<char *>(a->workspace);
  const int B = a->batch, S = a->seq_len, M = B * S;
  const int HD = a->qk_nope + a->qk_rope;

  const uint16_t *x = reinterpret_cast<const uint16_t *>(a->hidden_states);
  if (a->input_gamma) {
    uint16_t *xn = reinterpret_cast<uint16_t *>(ws + L.xn);
    if ((rc = launch_rms_norm(x, M, a->hidden, a->hidden, reinterpret_cast<const uint16_t *>(a->input_gamma),
                              a->eps, xn, a->hidden, st)))
      return rc;
    x = xn;
  }
  uint16_t *qa = reinterpret_cast<uint16_t *>(ws + L.qa);
  uint16_t *qan = reinterpret_cast<uint16_t *>(ws + L.qan);
  uint16_t *q = reinterpret_cast<uint16_t *>(ws + L.q);
  uint16_t *kvn = reinterpret_cast<uint16_t *>(ws + L.kvn);
  uint16_t *kpe = reinterpret_cast<uint16_t *>(ws + L.kpe);
  uint16_t *kvb = reinterpret_cast<uint16_t *>(ws + L.kvb);
  uint16_t *attn = reinterpret_cast<uint16_t *>(a->attn_out ? a->attn_out : ws + L.attn);

  GemvParams pa = {};
  pa.part = reinterpret_cast<float *>(ws + L.lin);
  pa.x = x; pa.M = M; pa.ldx = a->hidden;
  pa.w0 = reinterpret_cast<const uint8_t *>(a->w_q_a); pa.s0 = a->s_q_a;
  pa.w1 = reinterpret_cast<const uint8_t *>(a->w_kv_a); pa.s1 = a->s_kv_a;
  pa.N = a->q_lora + a->kv_lora + a->qk_rope; pa.K = a->hidden; pa.n_split = a->q_lora;
  pa.y = qa; pa.ldy = a->q_lora;
  pa.ckv = reinterpret_cast<uint16_t *>(a->ckv_cache);
  pa.kpe = reinterpret_cast<uint16_t *>(a->kpe_cache);
  pa.ckv_bstride = (int64_t)a->max_seq * a->kv_lora; pa.kpe_bstride = (int64_t)a->max_seq * a->qk_rope;
  pa.kv_lora = a->kv_lora; pa.rope = a->qk_rope; pa.pos = a->positions; pa.seq_len = S; pa.max_rows = a->max_seq;
  if ((rc = run_linear(pa, GEMV_QKVA, st, L.lin_bytes))) return rc;

  if ((rc = launch_rms_norm(qa, M, a->q_lora, a->q_lora, reinterpret_cast<const uint16_t *>(a->gamma_q), a->eps,
                            qan, a->q_lora, st)))
    return rc;

  GemvParams pb = {};
  pb.part = reinterpret_cast<float *>(ws + L.lin);
  pb.x = qan; pb.M = M; pb.ldx = a->q_lora;
  pb.w0 = reinterpret_cast<const uint8_t *>(a->w_q_b); pb.s0 = a->s_q_b;
  pb.N = a->heads * HD; pb.K = a->q_lora; pb.n_split = pb.N;
  pb.y = q; pb.ldy = pb.N;
  pb.pos = a->positions; pb.seq_len = S; pb.rope = a->qk_rope; pb.rope_table = a->rope_table;
  pb.rope_rows = a->rope_rows;
  pb.head_dim = HD; pb.nope = a->qk_nope;
  if ((rc = run_linear(pb, GEMV_QROPE, st, L.lin_bytes))) return rc;

  const int T = L.Tmax;
  FlashParams fp = {};
  fp.q = q; fp.kvb = kvb; fp.kpe = kpe; fp.out = attn; fp.pos = a->positions; fp.S = S; fp.tmax = T;
  fp.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  for (int b = 0; b < B; ++b) {
    const uint16_t *ckv_b = reinterpret_cast<const uint16_t *>(a->ckv_cache) + (size_t)b * a->max_seq * a->kv_lora;
    const uint16_t *kpe_b = reinterpret_cast<const uint16_t *>(a->kpe_cache) + (size_t)b * a->max_seq * a->qk_rope;
    // kv_a_layernorm of every cached row, then kv_b (inference/ops.py:148-151)
    if ((rc = launch_rms_norm(ckv_b, T, a->kv_lora, a->kv_lora, reinterpret_cast<const uint16_t *>(a->gamma_kv),
                              a->eps, kvn, a->kv_lora, st)))
      return rc;
    kpe_rope_kernel<<<dim3((T * (P_ROPE / 2) + 255) / 256), 256, 0, st>>>(kpe_b, a->rope_table, T, kpe);
    if ((rc = check_launch("kpe rope"))) return rc;
    GemvParams pk = {};
    pk.part = reinterpret_cast<float *>(ws + L.lin);
    pk.x = kvn; pk.M = T; pk.ldx = a->kv_lora;
    pk.w0 = reinterpret_cast<const uint8_t *>(a->w_kv_b); pk.s0 = a->s_kv_b;
    pk.N = a->heads * (a->qk_nope + a->v_dim); pk.K = a->kv_lora; pk.n_split = pk.N;
    pk.y = kvb; pk.ldy = pk.N; pk.seq_len = 1;
    if ((rc = run_linear(pk, GEMV_PLAIN, st, L.lin_bytes))) return rc;
    fp.b = b;
    static bool flash_attr = false;  // dynamic LDS above 64 KB
    if (!flash_attr) {
      (void)hipFuncSetAttribute((const void *)flash_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, F_LDS);
      flash_attr = true;
    }
    fp.nqb = (S + F_QB - 1) / F_QB;
    flash_kernel<<<dim3(P_H * fp.nqb), F_NW * 64, F_LDS, st>>>(fp);
    if ((rc = check_launch("flash attention"))) return rc;
  }

  GemvParams po = {};
  po.part = reinterpret_cast<float *>(ws + L.lin);
  po.x = attn; po.M = M; po.ldx = a->heads * a->v_dim;
  po.w0 = reinterpret_cast<const uint8_t *>(a->w_o); po.s0 = a->s_o;
  po.N = a->hidden; po.K = a->heads * a->v_dim; po.n_split = po.N;
  po.y = reinterpret_cast<uint16_t *>(a->out); po.ldy = a->hidden;
  po.res = reinterpret_cast<const uint16_t *>(a->residual); po.ldr = a->hidden; po.seq_len = 1;
  return run_linear(po, a->residual ? GEMV_RESID : GEMV_PLAIN, st, L.lin_bytes);
}

}  // namespace amla

extern "C" {

size_t amla_mla_prefill_workspace_bytes(const amla_mla_args *a) {
  if (!a || a->batch <= 0 || a->seq_len <= 0) return 0;
  return amla::prefill_layout(*a).total;
}

int amla_mla_prefill(const amla_mla_args *a, void *stream) {
  return amla::prefill_impl(a, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
