// Absorbed-MLA decode for gfx950: amla_mla_decode replaces mla_attention for
// S == 1 (inference/ops.py:100-183).
//
// The reference decompresses every cached latent row through kv_b on every
// step (ops.py:144-151).  Here the kv_b halves are absorbed instead:
//   W_UK[h] = kv_b rows h*256 .. +127, W_UV[h] = rows h*256+128 .. +255,
//   qt[h]   = gamma_kv * (W_UK[h]^T q_nope[h])                     (absorb_kernel)
//   s[h,t]  = sigma * ( r_t (qt[h] . c_t) + q_pe[h] . rope(t, kpe_t) )
//   O[h]    = sum_t softmax(s[h])_t r_t c_t                         (attn_kernel)
//   out[h]  = W_UV[h] (gamma_kv * O[h])                             (combine_uv_kernel)
// with c_t the raw cached latent row, r_t = rsqrt(mean(c_t^2) + eps) its
// RMSNorm factor (the cache holds pre-norm rows, ops.py:137-148) and rope(t, .)
// the rotation of the raw cached rope key (ops.py:158-159), both applied on the
// fly, once per row instead of once per row and head.
//
// Launch sequence per layer:
//   [rms_norm(hidden, input_gamma)]          optional (layer mode)
//   gemv  QKVA : q_a and kv_a from hidden; kv_a goes straight into the caches
//   rms_norm   : q_a with q_a_layernorm
//   gemv  QROPE: q = q_a W_qb^T; RoPE on the q_pe rows at pos[b]
//   absorb     : qt = gamma_kv * W_UK^T q_nope  -> qbuf (B, H, 576) with q_pe
//   attn       : split over context, online softmax, fp32 partial (m, l, O)
//   combine_uv : merge splits, gamma_kv, W_UV -> (B, H*128) bf16
//   gemv  PLAIN/RESID : wo
#include <math.h>

#include "amla_common.h"
#include "amla_internal.h"

namespace amla {

constexpr int LORA = 512;   // kv_lora_rank
constexpr int ROPE = 64;    // qk_rope_head_dim
constexpr int QKD = LORA + ROPE;
constexpr int HEADS = 128;
constexpr int NOPE = 128;
constexpr int VD = 128;
constexpr int TT = 32;               // cache rows per tile
constexpr int KT_STRIDE = QKD + 8;   // bf16 elements per t-major LDS row (16 B pad)
constexpr int CT_STRIDE = TT + 4;    // bf16 elements per latent-major LDS row (8 B pad)

// ---------------------------------------------------------------- absorb

// One workgroup per (head, group of 8 sequences).  Thread (dg, cc) sums over
// 32 rows d of W_UK[h] for 8 latent columns c; four row groups reduce in LDS.
__global__ __launch_bounds__(256) void absorb_kernel(const uint16_t *__restrict__ q,  // (B, H, 192)
                                                     const uint8_t *__restrict__ wkvb,
                                                     const float *__restrict__ skvb,
                                                     const uint16_t *__restrict__ gamma,
                                                     int B, uint16_t *__restrict__ qbuf) {
  constexpr int BB = 8;
  const int h = blockIdx.x;
  const int b0 = blockIdx.y * BB;
  const int nb = min(BB, B - b0);
  const int tid = threadIdx.x;
  const int cc = tid & 63, dg = tid >> 6;
  __shared__ float qn[BB][NOPE];
  __shared__ f32x4 red[4][BB][64][2];
  for (int e = tid; e < BB * NOPE; e += 256) {
    const int bb = e / NOPE, d = e % NOPE;
    qn[bb][d] = bb < nb ? bf2f(q[((size_t)(b0 + bb) * HEADS + h) * (NOPE + ROPE) + d]) : 0.f;
  }
  __syncthreads();
  const uint8_t *wp = wkvb + ((size_t)h * (NOPE + VD) + dg * 32) * LORA + cc * 8;
  f32x4 acc[BB][2];
#pragma unroll
  for (int bb = 0; bb < BB; ++bb) acc[bb][0] = acc[bb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int d = 0; d < 32; ++d) {
    const u32x2 raw = ldg8(wp + (size_t)d * LORA);
    const f32x2 w01 = fp8x2_to_f32<false>(raw.x), w23 = fp8x2_to_f32<true>(raw.x);
    const f32x2 w45 = fp8x2_to_f32<false>(raw.y), w67 = fp8x2_to_f32<true>(raw.y);
    const f32x4 wa = {w01.x, w01.y, w23.x, w23.y}, wb = {w45.x, w45.y, w67.x, w67.y};
#pragma unroll
    for (int bb = 0; bb < BB; ++bb) {
      const float qv = qn[bb][dg * 32 + d];
      acc[bb][0] += qv * wa;
      acc[bb][1] += qv * wb;
    }
  }
#pragma unroll
  for (int bb = 0; bb < BB; ++bb) {
    red[dg][bb][cc][0] = acc[bb][0];
    red[dg][bb][cc][1] = acc[bb][1];
  }
  __syncthreads();
  // 256 threads finish 8 sequences x 64 column groups x 2 halves
  for (int e = tid; e < BB * 64 * 2; e += 256) {
    const int bb = e / 128, c64 = (e / 2) % 64, half = e & 1;
    if (bb >= nb) continue;
    const f32x4 v = red[0][bb][c64][half] + red[1][bb][c64][half] + red[2][bb][c64][half] +
                    red[3][bb][c64][half];
    const float sc = skvb[(size_t)(2 * h) * (LORA / 128) + (c64 * 8) / 128];
    const int c = c64 * 8 + half * 4;
    const u32x2 g = *reinterpret_cast<const u32x2 *>(gamma + c);
    u32x2 o = {pack_bf16(v.x * sc * lo_bf(g.x), v.y * sc * hi_bf(g.x)),
               pack_bf16(v.z * sc * lo_bf(g.y), v.w * sc * hi_bf(g.y))};
    *reinterpret_cast<u32x2 *>(qbuf + ((size_t)(b0 + bb) * HEADS + h) * QKD + c) = o;
  }
  // rope half of the query: copied next to the absorbed latent query
  for (int e = tid; e < nb * (ROPE / 2); e += 256) {
    const int bb = e / (ROPE / 2), j = (e % (ROPE / 2)) * 2;
    const uint32_t v =
        *reinterpret_cast<const uint32_t *>(q + ((size_t)(b0 + bb) * HEADS + h) * (NOPE + ROPE) + NOPE + j);
    *reinterpret_cast<uint32_t *>(qbuf + ((size_t)(b0 + bb) * HEADS + h) * QKD + LORA + j) = v;
  }
}

// ---------------------------------------------------------------- attention

struct AttnParams {
  const uint16_t *qbuf;  // (B, H, 576) bf16: absorbed latent query | rotated rope query
  const uint16_t *ckv;   // cache (B_alloc, max_seq, 512)
  const uint16_t *kpe;   // cache (B_alloc, max_seq, 64)
  int64_t ckv_bstride, kpe_bstride;  // elements per sequence
  const float *rope_table;           // (rows, 32, 2)
  const int32_t *pos;                // decode position per sequence; context T = pos + 1
  int splits, tiles_per_split;
  float scale_log2;  // softmax scale * log2(e)
  float eps;
  float *part_o;   // (B, splits, H, 512) unnormalised sum_t p r_t c_t
  float *part_ml;  // (B, splits, H, 2) running max (log2 units) and sum of p
};

struct TileRegs {
  u32x4 c[4][2];  // 4 rows x 16 latent values
  u32x4 k;        // 8 rope values of one row
  f32x4 cs[2];    // 4 (cos, sin) pairs
};

// Thread roles in the loader: rows 4*rg .. 4*rg+3, latent columns 16*cg .. +15;
// rope key row tid/8, pairs 4*(tid%8) .. +3.
AMLA_DEV void load_tile(const AttnParams &p, int b, int t0, int T, TileRegs &R) {
  const int tid = threadIdx.x;
  const int rg = tid >> 5, cg = tid & 31;
  const uint16_t *cbase = p.ckv + (size_t)b * p.ckv_bstride;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + rg * 4 + r;
    if (t < T) {
      const uint16_t *src = cbase + (size_t)t * LORA + cg * 16;
      R.c[r][0] = ldg16_nt(src);
      R.c[r][1] = ldg16_nt(src + 8);
    } else {
      R.c[r][0] = R.c[r][1] = u32x4{0, 0, 0, 0};
    }
  }
  const int kt = t0 + (tid >> 3);
  const int kq = tid & 7;
  if (kt < T) {
    R.k = ldg16_nt(p.kpe + (size_t)b * p.kpe_bstride + (size_t)kt * ROPE + kq * 8);
    const f32x4 *tab = reinterpret_cast<const f32x4 *>(p.rope_table + ((size_t)kt * (ROPE / 2) + kq * 4) * 2);
    R.cs[0] = tab[0];
    R.cs[1] = tab[1];
  } else {
    R.k = u32x4{0, 0, 0, 0};
    R.cs[0] = R.cs[1] = f32x4{1.f, 0.f, 1.f, 0.f};
  }
}

AMLA_DEV uint32_t rot_pair(uint32_t x, float c, float s) {
  const float a = lo_bf(x), b = hi_bf(x);
  return pack_bf16(__fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s)), __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c)));
}

AMLA_DEV void store_tile(const AttnParams &p, const TileRegs &R, uint16_t *kt, uint16_t *ct, float *rs) {
  const int tid = threadIdx.x;
  const int rg = tid >> 5, cg = tid & 31;
  // t-major copy and per-row sum of squares
  float ss[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = rg * 4 + r;
    u32x4 *dst = reinterpret_cast<u32x4 *>(kt + t * KT_STRIDE + cg * 16);
    dst[0] = R.c[r][0];
    dst[1] = R.c[r][1];
    float a = 0.f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float x0 = lo_bf(R.c[r][h][q]), x1 = hi_bf(R.c[r][h][q]);
        a += x0 * x0 + x1 * x1;
      }
    ss[r] = a;
  }
  // reduce over the 32 column groups of the same rows (lanes 0-31 / 32-63)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) ss[r] += __shfl_xor(ss[r], o, 64);
  }
  if (cg == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) rs[rg * 4 + r] = rsqrtf(ss[r] * (1.f / LORA) + p.eps);
  }
  // latent-major (transposed) copy: column c holds rows 4rg .. 4rg+3
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t d0 = R.c[0][h][q], d1 = R.c[1][h][q], d2 = R.c[2][h][q], d3 = R.c[3][h][q];
      const int c = cg * 16 + h * 8 + q * 2;
      u32x2 even = {__builtin_amdgcn_perm(d1, d0, 0x05040100u), __builtin_amdgcn_perm(d3, d2, 0x05040100u)};
      u32x2 odd = {__builtin_amdgcn_perm(d1, d0, 0x07060302u), __builtin_amdgcn_perm(d3, d2, 0x07060302u)};
      *reinterpret_cast<u32x2 *>(ct + c * CT_STRIDE + rg * 4) = even;
      *reinterpret_cast<u32x2 *>(ct + (c + 1) * CT_STRIDE + rg * 4) = odd;
    }
  // rotated rope key (fp32 rotation rounded to bf16, as inference/ops.py:97)
  const int krow = tid >> 3, kq = tid & 7;
  u32x4 kr;
  kr.x = rot_pair(R.k.x, R.cs[0].x, R.cs[0].y);
  kr.y = rot_pair(R.k.y, R.cs[0].z, R.cs[0].w);
  kr.z = rot_pair(R.k.z, R.cs[1].x, R.cs[1].y);
  kr.w = rot_pair(R.k.w, R.cs[1].z, R.cs[1].w);
  *reinterpret_cast<u32x4 *>(kt + krow * KT_STRIDE + LORA + kq * 8) = kr;
}

// Grid (splits, B), 256 threads.  Wave w owns heads 32w .. 32w+31 for the
// whole tile: S^T = K_tile (32 x 576) . Q^T (576 x 32 heads) with the rows of
// the tile as the MFMA M dimension, so each lane ends with 8 scores of one
// head; those are exactly the B operand of O^T += C^T (512 x 32) . P^T, so the
// probabilities never leave registers.  O^T (512 x 32 heads, fp32) lives in
// 256 accumulator registers per lane.
__global__ __launch_bounds__(256, 1) void attn_kernel(AttnParams p) {
  const int split = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int T = p.pos[b] + 1;
  const int ntiles = (T + TT - 1) / TT;
  const int tb = split * p.tiles_per_split;
  const int te = min(tb + p.tiles_per_split, ntiles);

  extern __shared__ __align__(16) uint8_t smem[];
  // [kt 0 | kt 1 | ct 0 | ct 1 | rs 0 | rs 1]
  uint16_t *const kt_base = reinterpret_cast<uint16_t *>(smem);
  uint16_t *const ct_base = kt_base + 2 * TT * KT_STRIDE;
  float *const rs_base = reinterpret_cast<float *>(ct_base + 2 * LORA * CT_STRIDE);

  const int head0 = wave * 32;
  // query fragments (B operand): lane holds Q[head][ks*32 + 8*lg .. +7]
  bf16x8 qf[2][QKD / 32];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const uint16_t *qr = p.qbuf + ((size_t)b * HEADS + head0 + nt * 16 + li) * QKD + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < QKD / 32; ++ks) qf[nt][ks] = as_bf16x8(ldg16(qr + ks * 32));
  }

  f32x4 o[LORA / 16][2];
#pragma unroll
  for (int mt = 0; mt < LORA / 16; ++mt) o[mt][0] = o[mt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  if (tb < te) {
    TileRegs R;
    load_tile(p, b, tb * TT, T, R);
    store_tile(p, R, kt_base, ct_base, rs_base);
    __syncthreads();
    for (int tile = tb; tile < te; ++tile) {
      const int buf = (tile - tb) & 1;
      const bool more = tile + 1 < te;
      const uint16_t *K = kt_base + buf * (TT * KT_STRIDE);
      const uint16_t *C = ct_base + buf * (LORA * CT_STRIDE);
      const float *RS = rs_base + buf * TT;

      // ---- scores: S^T (t x head)
      f32x4 sl[2][2], sp[2][2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) sl[mt][nt] = sp[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < QKD / 32; ++ks) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const bf16x8 a = as_bf16x8(
              *reinterpret_cast<const u32x4 *>(K + (mt * 16 + li) * KT_STRIDE + ks * 32 + 8 * lg));
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            if (ks < LORA / 32) sl[mt][nt] = mfma16(a, qf[nt][ks], sl[mt][nt]);
            else sp[mt][nt] = mfma16(a, qf[nt][ks], sp[mt][nt]);
          }
        }
      }
      // next tile's rows are fetched while softmax and P.V run
      if (more) load_tile(p, b, (tile + 1) * TT, T, R);
      // ---- online softmax per head (column); lane holds t = mt*16 + 4*lg + r
      const int tbase = tile * TT;
      bf16x8 pf[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        float sv[8];
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int tl = mt * 16 + 4 * lg + r;
            float v = p.scale_log2 * (RS[tl] * sl[mt][nt][r] + sp[mt][nt][r]);
            v = (tbase + tl < T) ? v : -INFINITY;
            sv[mt * 4 + r] = v;
            mx = fmaxf(mx, v);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[nt], mx);
        const float alpha = (m_run[nt] == -INFINITY) ? 0.f : exp2f(m_run[nt] - m_new);
        float lsum = 0.f;
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = (sv[e] == -INFINITY) ? 0.f : exp2f(sv[e] - m_new);
          lsum += pe;
          const int tl = (e >> 2) * 16 + 4 * lg + (e & 3);
          pv[e] = pe * RS[tl];
        }
        l_run[nt] = l_run[nt] * alpha + lsum;
        m_run[nt] = m_new;
        if (__any(alpha != 1.f)) {
#pragma unroll
          for (int mt = 0; mt < LORA / 16; ++mt) o[mt][nt] *= alpha;
        }
        u32x4 pk = {pack_bf16(pv[0], pv[1]), pack_bf16(pv[2], pv[3]), pack_bf16(pv[4], pv[5]),
                    pack_bf16(pv[6], pv[7])};
        pf[nt] = as_bf16x8(pk);
      }
      // ---- O^T (latent x head) += C^T (latent x t) . P^T (t x head)
#pragma unroll
      for (int mt = 0; mt < LORA / 16; ++mt) {
        const uint16_t *cr = C + (mt * 16 + li) * CT_STRIDE + 4 * lg;
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(cr);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(cr + 16);
        const bf16x8 a = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
        o[mt][0] = mfma16(a, pf[0], o[mt][0]);
        o[mt][1] = mfma16(a, pf[1], o[mt][1]);
      }
      if (more)
        store_tile(p, R, kt_base + (buf ^ 1) * (TT * KT_STRIDE), ct_base + (buf ^ 1) * (LORA * CT_STRIDE),
                   rs_base + (buf ^ 1) * TT);
      __syncthreads();
    }
  }

  // ---- partial results of this split
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float l = l_run[nt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int head = head0 + nt * 16 + li;
    const size_t row = ((size_t)b * p.splits + split) * HEADS + head;
    if (lg == 0) {
      p.part_ml[row * 2] = m_run[nt];
      p.part_ml[row * 2 + 1] = l;
    }
    float *dst = p.part_o + row * LORA + 4 * lg;
#pragma unroll
    for (int mt = 0; mt < LORA / 16; ++mt) *reinterpret_cast<f32x4 *>(dst + mt * 16) = o[mt][nt];
  }
}

constexpr size_t ATTN_LDS = (size_t)2 * TT * KT_STRIDE * 2 + (size_t)2 * LORA * CT_STRIDE * 2 + 2 * TT * 4;

// ---------------------------------------------------------------- combine + W_UV

// Grid (H, B): blockIdx.x = head so consecutive workgroups of one head (same
// XCD, shared L2) reuse its W_UV rows across the batch.
__global__ __launch_bounds__(256) void combine_uv_kernel(const float *__restrict__ part_o,
                                                         const float *__restrict__ part_ml, int splits,
                                                         const uint8_t *__restrict__ wkvb,
                                                         const float *__restrict__ skvb,
                                                         const uint16_t *__restrict__ gamma,
                                                         uint16_t *__restrict__ attn) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float wsp[256];
  __shared__ float lat[LORA];
  __shared__ float red[4];
  const size_t base = (size_t)b * splits * HEADS + h;  // row of split 0
  float m = -INFINITY;
  for (int s = tid; s < splits; s += 256) m = fmaxf(m, part_ml[(base + (size_t)s * HEADS) * 2]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float lsum = 0.f;
  for (int s = tid; s < splits; s += 256) {
    const float ms = part_ml[(base + (size_t)s * HEADS) * 2];
    const float w = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
    wsp[s] = w;
    lsum += w * part_ml[(base + (size_t)s * HEADS) * 2 + 1];
  }
  lsum = wave_sum(lsum);
  if (lane == 0) red[wave] = lsum;
  __syncthreads();
  const float inv_l = 1.f / (red[0] + red[1] + red[2] + red[3]);
  for (int c = tid; c < LORA; c += 256) {
    float a = 0.f;
    for (int s = 0; s < splits; ++s) a += wsp[s] * part_o[(base + (size_t)s * HEADS) * LORA + c];
    lat[c] = a * inv_l * bf2f(gamma[c]);
  }
  __syncthreads();
  // out[v] = sum_c W_UV[h][v][c] * scale * lat[c]; wave handles 32 rows, lane 8 columns
  float lv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) lv[j] = lat[lane * 8 + j];
  const float sc = skvb[(size_t)(2 * h + 1) * (LORA / 128) + (lane * 8) / 128];
  const uint8_t *wrow = wkvb + ((size_t)h * (NOPE + VD) + NOPE) * LORA + lane * 8;
  for (int v = wave * 32; v < wave * 32 + 32; ++v) {
    const u32x2 raw = ldg8(wrow + (size_t)v * LORA);
    const f32x2 w01 = fp8x2_to_f32<false>(raw.x), w23 = fp8x2_to_f32<true>(raw.x);
    const f32x2 w45 = fp8x2_to_f32<false>(raw.y), w67 = fp8x2_to_f32<true>(raw.y);
    float a = w01.x * lv[0] + w01.y * lv[1] + w23.x * lv[2] + w23.y * lv[3] + w45.x * lv[4] +
              w45.y * lv[5] + w67.x * lv[6] + w67.y * lv[7];
    a = wave_sum(a * sc);
    if (lane == 0) attn[(size_t)b * HEADS * VD + h * VD + v] = f2bf(a);
  }
}

// ---------------------------------------------------------------- orchestration

struct DecodeLayout {
  size_t counters, partials, xn, qa, qan, q, qbuf, part_ml, part_o, attn, total;
  GemvPlan pa, pb, po;
  int splits, tiles_per_split;
};

static DecodeLayout decode_layout(const amla_mla_args &a) {
  DecodeLayout L = {};
  const int B = a.batch;
  const int HD = a.qk_nope + a.qk_rope;
  L.pa = plan_gemv(B, a.q_lora + a.kv_lora + a.qk_rope, a.hidden);
  L.pb = plan_gemv(B, a.heads * HD, a.q_lora);
  L.po = plan_gemv(B, a.hidden, a.heads * a.v_dim);
  const int maxT = a.max_context > 0 ? a.max_context : a.max_seq;
  const int ntiles = (maxT + TT - 1) / TT;
  int splits = (256 + B - 1) / B;
  splits = std::max(1, std::min(splits, (ntiles + 1) / 2));
  L.tiles_per_split = (ntiles + splits - 1) / splits;
  L.splits = (ntiles + L.tiles_per_split - 1) / L.tiles_per_split;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes, 256); return o; };
  L.counters = take(COUNTER_BYTES);
  L.partials = take(std::max({L.pa.partial_bytes, L.pb.partial_bytes, L.po.partial_bytes, (size_t)256}));
  L.xn = take((size_t)B * a.hidden * 2);
  L.qa = take((size_t)B * a.q_lora * 2);
  L.qan = take((size_t)B * a.q_lora * 2);
  L.q = take((size_t)B * a.heads * HD * 2);
  L.qbuf = take((size_t)B * a.heads * QKD * 2);
  L.part_ml = take((size_t)B * L.splits * a.heads * 2 * 4);
  L.part_o = take((size_t)B * L.splits * a.heads * LORA * 4);
  L.attn = take((size_t)B * a.heads * a.v_dim * 2);
  L.total = off;
  return L;
}

static int check_common(const amla_mla_args *a, const char *who) {
  if (!a) return fail(AMLA_EINVAL, "%s: null args", who);
  if (a->heads != HEADS || a->kv_lora != LORA || a->qk_rope != ROPE || a->qk_nope != NOPE || a->v_dim != VD)
    return fail(AMLA_EUNSUPPORTED,
                "%s: kernels are built for heads=128 kv_lora=512 rope=64 nope=128 v=128 (got %d/%d/%d/%d/%d)",
                who, a->heads, a->kv_lora, a->qk_rope, a->qk_nope, a->v_dim);
  if (a->hidden <= 0 || a->hidden % 128 || a->q_lora <= 0 || a->q_lora % 128)
    return fail(AMLA_EUNSUPPORTED, "%s: hidden and q_lora must be positive multiples of 128", who);
  if (a->batch <= 0 || a->seq_len <= 0) return fail(AMLA_EINVAL, "%s: batch and seq_len must be >= 1", who);
  if (a->max_seq <= 0 || a->rope_rows <= 0) return fail(AMLA_EINVAL, "%s: max_seq / rope_rows must be >= 1", who);
  const void *ptrs[] = {a->positions, a->hidden_states, a->out, a->w_q_a, a->s_q_a, a->w_q_b, a->s_q_b,
                        a->w_kv_a, a->s_kv_a, a->w_kv_b, a->s_kv_b, a->w_o, a->s_o, a->gamma_q,
                        a->gamma_kv, a->ckv_cache, a->kpe_cache, a->rope_table, a->workspace};
  for (const void *q : ptrs)
    if (!q) return fail(AMLA_EINVAL, "%s: a required pointer is null", who);
  if (!aligned16(a->hidden_states) || !aligned16(a->ckv_cache) || !aligned16(a->kpe_cache) ||
      !aligned16(a->rope_table) || !aligned16(a->out) || !aligned16(a->workspace))
    return fail(AMLA_EINVAL, "%s: activations, caches, rope table and workspace must be 16-byte aligned", who);
  return AMLA_OK;
}

// Optional stage events (bench instrumentation): ev[i] is recorded before
// stage i and ev[NSTAGE] after the last one.
constexpr int NSTAGE = 7;  // qkva, q_a norm, q_b, absorb, attention, combine, o_proj

static inline void mark(hipEvent_t const *ev, int i, hipStream_t st) {
  if (ev) (void)hipEventRecord(ev[i], st);
}

static int decode_impl(const amla_mla_args *a, hipStream_t st, hipEvent_t const *ev = nullptr) {
  int rc = check_common(a, "mla_decode");
  if (rc) return rc;
  if (a->seq_len != 1) return fail(AMLA_EINVAL, "mla_decode: seq_len must be 1 (use mla_prefill)");
  if (a->batch > 64) return fail(AMLA_EUNSUPPORTED, "mla_decode: batch > 64 not supported");
  const DecodeLayout L = decode_layout(*a);
  if (a->workspace_bytes < L.total)
    return fail(AMLA_EWORKSPACE, "mla_decode: workspace %zu bytes < %zu needed", a->workspace_bytes, L.total);
  char *ws = reinterpret_cast<char *>(a->workspace);
  float *partials = reinterpret_cast<float *>(ws + L.partials);
  const int B = a->batch;
  const int HD = a->qk_nope + a->qk_rope;

  const uint16_t *x = reinterpret_cast<const uint16_t *>(a->hidden_states);
  if (a->input_gamma) {
    uint16_t *xn = reinterpret_cast<uint16_t *>(ws + L.xn);
    rc = launch_rms_norm(x, B, a->hidden, a->hidden, reinterpret_cast<const uint16_t *>(a->input_gamma),
                         a->eps, xn, a->hidden, st);
    if (rc) return rc;
    x = xn;
  }
  uint16_t *qa = reinterpret_cast<uint16_t *>(ws + L.qa);
  uint16_t *qan = reinterpret_cast<uint16_t *>(ws + L.qan);
  uint16_t *q = reinterpret_cast<uint16_t *>(ws + L.q);
  uint16_t *qbuf = reinterpret_cast<uint16_t *>(ws + L.qbuf);

  // 1. q_a | kv_a  (kv_a written raw into the caches, inference/ops.py:136-141)
  mark(ev, 0, st);
  GemvParams pa = {};
  pa.x = x; pa.M = B; pa.ldx = a->hidden;
  pa.w0 = reinterpret_cast<const uint8_t *>(a->w_q_a); pa.s0 = a->s_q_a;
  pa.w1 = reinterpret_cast<const uint8_t *>(a->w_kv_a); pa.s1 = a->s_kv_a;
  pa.N = a->q_lora + LORA + ROPE; pa.K = a->hidden; pa.n_split = a->q_lora;
  pa.y = qa; pa.ldy = a->q_lora;
  pa.ckv = reinterpret_cast<uint16_t *>(a->ckv_cache);
  pa.kpe = reinterpret_cast<uint16_t *>(a->kpe_cache);
  pa.ckv_bstride = (int64_t)a->max_seq * LORA; pa.kpe_bstride = (int64_t)a->max_seq * ROPE;
  pa.kv_lora = LORA; pa.rope = ROPE; pa.pos = a->positions; pa.seq_len = 1;
  pa.ws = partials; pa.counters = counter_slot(ws, 1);
  if ((rc = launch_gemv(pa, GEMV_QKVA, L.pa, st))) return rc;

  // 2. q_a_layernorm (inference/ops.py:130)
  mark(ev, 1, st);
  if ((rc = launch_rms_norm(qa, B, a->q_lora, a->q_lora, reinterpret_cast<const uint16_t *>(a->gamma_q), a->eps,
                            qan, a->q_lora, st)))
    return rc;

  // 3. q = q_a W_qb^T, RoPE on q_pe at pos[b] (inference/ops.py:131-133, :156)
  mark(ev, 2, st);
  GemvParams pb = {};
  pb.x = qan; pb.M = B; pb.ldx = a->q_lora;
  pb.w0 = reinterpret_cast<const uint8_t *>(a->w_q_b); pb.s0 = a->s_q_b;
  pb.N = a->heads * HD; pb.K = a->q_lora; pb.n_split = pb.N;
  pb.y = q; pb.ldy = pb.N;
  pb.pos = a->positions; pb.seq_len = 1; pb.rope = ROPE; pb.rope_table = a->rope_table;
  pb.head_dim = HD; pb.nope = a->qk_nope;
  pb.ws = partials; pb.counters = counter_slot(ws, 2);
  if ((rc = launch_gemv(pb, GEMV_QROPE, L.pb, st))) return rc;

  // 4. absorb W_UK into the query
  mark(ev, 3, st);
  absorb_kernel<<<dim3(HEADS, (B + 7) / 8), 256, 0, st>>>(
      q, reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b, reinterpret_cast<const uint16_t *>(a->gamma_kv),
      B, qbuf);
  if ((rc = check_launch("mla absorb"))) return rc;

  // 5. attention over the latent cache, split over context
  mark(ev, 4, st);
  AttnParams ap = {};
  ap.qbuf = qbuf;
  ap.ckv = reinterpret_cast<const uint16_t *>(a->ckv_cache);
  ap.kpe = reinterpret_cast<const uint16_t *>(a->kpe_cache);
  ap.ckv_bstride = (int64_t)a->max_seq * LORA; ap.kpe_bstride = (int64_t)a->max_seq * ROPE;
  ap.rope_table = a->rope_table; ap.pos = a->positions;
  ap.splits = L.splits; ap.tiles_per_split = L.tiles_per_split;
  ap.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  ap.eps = a->eps;
  ap.part_o = reinterpret_cast<float *>(ws + L.part_o);
  ap.part_ml = reinterpret_cast<float *>(ws + L.part_ml);
  attn_kernel<<<dim3(L.splits, B), 256, ATTN_LDS, st>>>(ap);
  if ((rc = check_launch("mla attention"))) return rc;

  // 6. merge splits, W_UV
  mark(ev, 5, st);
  uint16_t *attn = reinterpret_cast<uint16_t *>(ws + L.attn);
  combine_uv_kernel<<<dim3(HEADS, B), 256, 0, st>>>(ap.part_o, ap.part_ml, L.splits,
                                                     reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b,
                                                     reinterpret_cast<const uint16_t *>(a->gamma_kv), attn);
  if ((rc = check_launch("mla combine"))) return rc;

  // 7. o_proj (+ residual in layer mode)
  mark(ev, 6, st);
  GemvParams po = {};
  po.x = attn; po.M = B; po.ldx = a->heads * a->v_dim;
  po.w0 = reinterpret_cast<const uint8_t *>(a->w_o); po.s0 = a->s_o;
  po.N = a->hidden; po.K = a->heads * a->v_dim; po.n_split = po.N;
  po.y = reinterpret_cast<uint16_t *>(a->out); po.ldy = a->hidden;
  po.res = reinterpret_cast<const uint16_t *>(a->residual); po.ldr = a->hidden;
  po.seq_len = 1;
  po.ws = partials; po.counters = counter_slot(ws, 3);
  rc = launch_gemv(po, a->residual ? GEMV_RESID : GEMV_PLAIN, L.po, st);
  mark(ev, NSTAGE, st);
  return rc;
}

static bool g_attr_set = false;

}  // namespace amla

using namespace amla;

extern "C" {

size_t amla_mla_decode_workspace_bytes(const amla_mla_args *a) {
  if (!a || a->batch <= 0) return 0;
  return decode_layout(*a).total;
}

int amla_mla_decode(const amla_mla_args *a, void *stream) {
  if (!g_attr_set) {
    // Opt in to more than 64 KB of dynamic LDS (gfx950 has 160 KB per CU).
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)ATTN_LDS);
    (void)hipGetLastError();
    g_attr_set = true;
  }
  return decode_impl(a, reinterpret_cast<hipStream_t>(stream));
}

int amla_mla_decode_profiled(const amla_mla_args *a, void *stream, void *const *events) {
  if (!events) return fail(AMLA_EINVAL, "mla_decode_profiled: null events");
  for (int i = 0; i <= NSTAGE; ++i)
    if (!events[i]) return fail(AMLA_EINVAL, "mla_decode_profiled: null event %d", i);
  if (!g_attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)ATTN_LDS);
    (void)hipGetLastError();
    g_attr_set = true;
  }
  return decode_impl(a, reinterpret_cast<hipStream_t>(stream), reinterpret_cast<hipEvent_t const *>(events));
}

}  // extern "C"
