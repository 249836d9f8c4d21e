// MLA prefill for gfx950: amla_mla_prefill replaces mla_attention for S >= 1
// tokens per sequence with a causal mask (inference/ops.py:100-183, :172-177),
// and the large-M block-FP8 GEMM that amla_fp8_linear uses for M > 64.
//
// Prefill keeps the reference's non-absorbed formulation (absorption would
// cost more FLOPs at S = T): kv_b decompresses the RMS-normed latent rows once
// per call (one GEMM), and causal flash attention runs per head with
// d_qk = 128 + 64 (the rope key shared by all heads) and d_v = 128.
//
// GEMM (K3): C[m, n] = sum_k X[m, k] W[n, k] scale_inv[n/128, k/128].
//   Workgroup tile 128 (weight rows n) x 128 (activation rows m), K step 64,
//   double-buffered in LDS; fp8 weights are converted exactly to bf16 when
//   staged.  The weight tile spans one 128-row scale block, so the scale of a
//   128-wide K block is one scalar per workgroup: MFMAs accumulate the block
//   into a fresh fp32 tile which is then added to the result times that scale.
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
      const int64_t row = prow_position(p, m);
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

constexpr int G_BN = 128, G_BM = 128, G_BK = 64;
constexpr int G_LD = G_BK + 8;  // bf16 per LDS row (16 B pad)

template <int MODE>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemvParams p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;
  const int nb = blockIdx.x;  // 128-row weight block == scale row block
  const int m0 = blockIdx.y * G_BM;
  const int KB = p.K >> 7;

  __shared__ __align__(16) uint16_t Ws[2][G_BN * G_LD];
  __shared__ __align__(16) uint16_t Xs[2][G_BM * G_LD];

  const int n0 = nb * G_BN;
  const bool seg1 = (MODE == GEMV_QKVA) && n0 >= p.n_split;
  const uint8_t *W = seg1 ? p.w1 : p.w0;
  const float *S = seg1 ? p.s1 : p.s0;
  const int nl0 = seg1 ? n0 - p.n_split : n0;
  const int nrows = (seg1 ? p.N - p.n_split : p.n_split) - nl0;  // valid rows of this segment from nl0
  const float *srow = S + (size_t)(nl0 >> 7) * KB;

  // loader roles: weight row tid/2 (32 bytes at (tid&1)*32), x row tid/2 (32 elements)
  const int lr = tid >> 1, lh = tid & 1;
  const bool wvalid = lr < nrows;
  const uint8_t *wsrc = W + (size_t)(wvalid ? nl0 + lr : 0) * p.K + lh * 32;
  const bool xvalid = m0 + lr < p.M;
  const uint16_t *xsrc = p.x + (size_t)(xvalid ? m0 + lr : 0) * p.ldx + lh * 32;

  u32x4 wreg[2], xreg[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) wreg[j] = wvalid ? ldg16(wsrc + k0 + j * 16) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) xreg[j] = xvalid ? ldg16(xsrc + k0 + j * 8) : u32x4{0, 0, 0, 0};
  };
  auto sstore = [&](int buf) {
    uint16_t *wd = &Ws[buf][lr * G_LD + lh * 32];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      bf16x8 lo, hi;
      fp8x16_to_bf16x16(wreg[j], lo, hi);
      *reinterpret_cast<bf16x8 *>(wd + j * 16) = lo;
      *reinterpret_cast<bf16x8 *>(wd + j * 16 + 8) = hi;
    }
    uint16_t *xd = &Xs[buf][lr * G_LD + lh * 32];
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4 *>(xd + j * 8) = xreg[j];
  };

  f32x4 acc[4][4], blk[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = blk[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int iters = p.K / G_BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int it = 0; it < iters; ++it) {
    const int buf = it & 1;
    if (it + 1 < iters) gload((it + 1) * G_BK);
    const uint16_t *wb = Ws[buf];
    const uint16_t *xb = Xs[buf];
#pragma unroll
    for (int ks = 0; ks < G_BK / 32; ++ks) {
      bf16x8 a[4], bm[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const bf16x8 *>(wb + (wn * 64 + i * 16 + li) * G_LD + ks * 32 + 8 * lg);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bm[j] = *reinterpret_cast<const bf16x8 *>(xb + (wm * 64 + j * 16 + li) * G_LD + ks * 32 + 8 * lg);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) blk[i][j] = mfma16(a[i], bm[j], blk[i][j]);
    }
    if (it & 1) {  // end of a 128-wide K block: apply its scale
      const float sk = srow[it >> 1];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] += sk * blk[i][j];
          blk[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    if (it + 1 < iters) sstore(buf ^ 1);
    __syncthreads();
  }
  // C layout: lane holds m = mt*16 + li, n = nt*16 + 4*lg .. +3
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = n0 + wn * 64 + i * 16 + 4 * lg;
    if (n >= p.N) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + wm * 64 + j * 16 + li;
      if (m < p.M) pstore4<MODE>(p, m, n, acc[i][j]);
    }
  }
}

size_t gemm_ws_bytes(int, int, int) { return 0; }

int launch_gemm(const GemvParams &p, int mode, hipStream_t st) {
  if (p.K % 128 || p.N % 16) return fail(AMLA_EUNSUPPORTED, "fp8 GEMM needs K %% 128 == 0 and N %% 16 == 0");
  if (mode == GEMV_QKVA ? (p.n_split % 128) : 0)
    return fail(AMLA_EUNSUPPORTED, "fp8 GEMM: q_lora must be a multiple of 128");
  dim3 grid((p.N + G_BN - 1) / G_BN, (p.M + G_BM - 1) / G_BM);
  switch (mode) {
    case GEMV_PLAIN: gemm_kernel<GEMV_PLAIN><<<grid, 256, 0, st>>>(p); break;
    case GEMV_RESID: gemm_kernel<GEMV_RESID><<<grid, 256, 0, st>>>(p); break;
    case GEMV_QKVA: gemm_kernel<GEMV_QKVA><<<grid, 256, 0, st>>>(p); break;
    default: gemm_kernel<GEMV_QROPE><<<grid, 256, 0, st>>>(p); break;
  }
  return check_launch("fp8 GEMM");
}

// ---------------------------------------------------------------- K10 causal flash attention

constexpr int P_NOPE = 128, P_ROPE = 64, P_QK = 192, P_V = 128, P_H = 128;
constexpr int P_KT = 32;                // keys per tile
constexpr int P_KLD = P_QK + 8;         // t-major key row (bf16)
constexpr int P_VLD = P_KT + 4;         // v-major value row (bf16)
constexpr int P_QW = 64;                // queries per wave
constexpr int P_QB = 4 * P_QW;          // queries per workgroup

struct FlashParams {
  const uint16_t *q;      // (rows, H, 192): row = b*S + s, q_pe already rotated
  const uint16_t *kvb;    // (Tmax, H*256): k_nope | v per head
  const uint16_t *kpe;    // (Tmax, 64) rotated rope keys
  uint16_t *out;          // (rows, H*128)
  const int32_t *pos;
  int b, S;
  float scale_log2;
};

struct FlashRegs {
  u32x4 kn[2];  // key row tid/8: nope elements (tid%8)*16 .. +15
  u32x4 kr;     // key row tid/8: rope elements (tid%8)*8 .. +7
  u32x2 v[4];   // keys 4*(tid/32) .. +3, v columns 4*(tid%32) .. +3
};

AMLA_DEV void flash_load(const FlashParams &p, int h, int t0, int Tlim, FlashRegs &R) {
  const int tid = threadIdx.x;
  const int kr = tid >> 3, kc = tid & 7;
  const int t = t0 + kr;
  if (t < Tlim) {
    const uint16_t *src = p.kvb + (size_t)t * (P_H * 256) + h * 256 + kc * 16;
    R.kn[0] = ldg16(src);
    R.kn[1] = ldg16(src + 8);
    R.kr = ldg16(p.kpe + (size_t)t * P_ROPE + kc * 8);
  } else {
    R.kn[0] = R.kn[1] = R.kr = u32x4{0, 0, 0, 0};
  }
  const int vr = tid >> 5, vc = tid & 31;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tv = t0 + vr * 4 + j;
    R.v[j] = tv < Tlim ? ldg8(p.kvb + (size_t)tv * (P_H * 256) + h * 256 + P_NOPE + vc * 4) : u32x2{0, 0};
  }
}

AMLA_DEV void flash_store(const FlashRegs &R, uint16_t *Ks, uint16_t *Vs) {
  const int tid = threadIdx.x;
  const int kr = tid >> 3, kc = tid & 7;
  *reinterpret_cast<u32x4 *>(Ks + kr * P_KLD + kc * 16) = R.kn[0];
  *reinterpret_cast<u32x4 *>(Ks + kr * P_KLD + kc * 16 + 8) = R.kn[1];
  *reinterpret_cast<u32x4 *>(Ks + kr * P_KLD + P_NOPE + kc * 8) = R.kr;
  const int vr = tid >> 5, vc = tid & 31;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t d0 = R.v[0][q], d1 = R.v[1][q], d2 = R.v[2][q], d3 = R.v[3][q];
    const int c = vc * 4 + q * 2;
    u32x2 even = {__builtin_amdgcn_perm(d1, d0, 0x05040100u), __builtin_amdgcn_perm(d3, d2, 0x05040100u)};
    u32x2 odd = {__builtin_amdgcn_perm(d1, d0, 0x07060302u), __builtin_amdgcn_perm(d3, d2, 0x07060302u)};
    *reinterpret_cast<u32x2 *>(Vs + c * P_VLD + vr * 4) = even;
    *reinterpret_cast<u32x2 *>(Vs + (c + 1) * P_VLD + vr * 4) = odd;
  }
}

// Grid (H, query blocks).  Wave w handles queries qb*256 + 64w .. +63 of one
// head: S^T = K (keys x 192) . Q^T with keys as the MFMA M dimension, so each
// lane holds 8 scores of one query, which are the B operand of
// O^T (128 x queries) += V^T (128 x keys) . P^T.
__global__ __launch_bounds__(256, 1) void flash_kernel(FlashParams p) {
  const int h = blockIdx.x;
  const int qblk = gridDim.y - 1 - blockIdx.y;  // heaviest causal blocks first
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int pos0 = p.pos[p.b];
  const int s_begin = qblk * P_QB;
  const int s_wave = s_begin + wave * P_QW;
  const int s_last_blk = min(s_begin + P_QB, p.S) - 1;
  const int Tlim = pos0 + s_last_blk + 1;   // keys needed by this block
  const int ntiles = (Tlim + P_KT - 1) / P_KT;

  __shared__ __align__(16) uint16_t Ks[2][P_KT * P_KLD];
  __shared__ __align__(16) uint16_t Vs[2][P_V * P_VLD];

  bf16x8 qf[4][P_QK / 32];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int s = min(s_wave + nt * 16 + li, p.S - 1);
    const uint16_t *qr = p.q + ((size_t)(p.b * p.S + s) * P_H + h) * P_QK + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < P_QK / 32; ++ks) qf[nt][ks] = as_bf16x8(ldg16(qr + ks * 32));
  }
  f32x4 o[P_V / 16][4];
#pragma unroll
  for (int vt = 0; vt < P_V / 16; ++vt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) o[vt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[4], l_run[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) { m_run[nt] = -INFINITY; l_run[nt] = 0.f; }

  FlashRegs R;
  flash_load(p, h, 0, Tlim, R);
  flash_store(R, Ks[0], Vs[0]);
  __syncthreads();
  const int wave_last_pos = pos0 + min(s_wave + P_QW, p.S) - 1;
  for (int tile = 0; tile < ntiles; ++tile) {
    const int buf = tile & 1;
    const bool more = tile + 1 < ntiles;
    if (more) flash_load(p, h, (tile + 1) * P_KT, Tlim, R);
    const int t0 = tile * P_KT;
    if (t0 <= wave_last_pos && s_wave < p.S) {
      const uint16_t *K = Ks[buf];
      const uint16_t *V = Vs[buf];
      f32x4 sc[2][4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) sc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < P_QK / 32; ++ks) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const bf16x8 a = *reinterpret_cast<const bf16x8 *>(K + (mt * 16 + li) * P_KLD + ks * 32 + 8 * lg);
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) sc[mt][nt] = mfma16(a, qf[nt][ks], sc[mt][nt]);
        }
      }
      bf16x8 pf[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int qpos = pos0 + s_wave + nt * 16 + li;
        float sv[8];
        float mx = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = t0 + mt * 16 + 4 * lg + r;
            const float v = (t <= qpos) ? sc[mt][nt][r] * p.scale_log2 : -INFINITY;
            sv[mt * 4 + r] = v;
            mx = fmaxf(mx, v);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[nt], mx);
        const float alpha = (m_run[nt] == -INFINITY) ? 0.f : exp2f(m_run[nt] - m_new);
        float pv[8], lsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = (sv[e] == -INFINITY) ? 0.f : exp2f(sv[e] - m_new);
          lsum += pv[e];
        }
        l_run[nt] = l_run[nt] * alpha + lsum;
        m_run[nt] = m_new;
        if (__any(alpha != 1.f)) {
#pragma unroll
          for (int vt = 0; vt < P_V / 16; ++vt) o[vt][nt] *= alpha;
        }
        u32x4 pk = {pack_bf16(pv[0], pv[1]), pack_bf16(pv[2], pv[3]), pack_bf16(pv[4], pv[5]),
                    pack_bf16(pv[6], pv[7])};
        pf[nt] = as_bf16x8(pk);
      }
#pragma unroll
      for (int vt = 0; vt < P_V / 16; ++vt) {
        const uint16_t *vr = V + (vt * 16 + li) * P_VLD + 4 * lg;
        const u32x2 lo = *reinterpret_cast<const u32x2 *>(vr);
        const u32x2 hi = *reinterpret_cast<const u32x2 *>(vr + 16);
        const bf16x8 a = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) o[vt][nt] = mfma16(a, pf[nt], o[vt][nt]);
      }
    }
    if (more) flash_store(R, Ks[buf ^ 1], Vs[buf ^ 1]);
    __syncthreads();
  }
  // normalise and store: lane holds query col nt*16+li, v rows vt*16 + 4*lg .. +3
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    float l = l_run[nt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int s = s_wave + nt * 16 + li;
    if (s >= p.S) continue;
    const float inv = 1.f / l;
    uint16_t *dst = p.out + (size_t)(p.b * p.S + s) * (P_H * P_V) + h * P_V + 4 * lg;
#pragma unroll
    for (int vt = 0; vt < P_V / 16; ++vt) {
      const f32x4 v = o[vt][nt] * inv;
      *reinterpret_cast<u32x2 *>(dst + vt * 16) = u32x2{pack_bf16(v.x, v.y), pack_bf16(v.z, v.w)};
    }
  }
}

// ---------------------------------------------------------------- orchestration

// p.part must hold the K-part sums of the skinny plan (PrefillLayout::lin)
static int run_linear(const GemvParams &p, int mode, hipStream_t st) {
  if (p.M <= 64) return launch_gemv(p, mode, plan_gemv(p.M, p.N, p.K), st);
  return launch_gemm(p, mode, st);
}

struct PrefillLayout {
  size_t xn, qa, qan, q, kvn, kpe, kvb, attn, lin, total;
  int Tmax;
};

static PrefillLayout prefill_layout(const amla_mla_args &a) {
  PrefillLayout L = {};
  const size_t M = (size_t)a.batch * a.seq_len;
  const int HD = a.qk_nope + a.qk_rope;
  L.Tmax = a.max_context > 0 ? std::min(a.max_context, a.max_seq) : a.max_seq;
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
  // K-part sums of the skinny linears (M <= 64)
  size_t lin = 0;
  const int HDv = a.qk_nope + a.v_dim;
  auto need = [&](int m, int n, int k) {
    if (m <= 64) lin = std::max(lin, plan_gemv(m, n, k).part_bytes);
  };
  need((int)M, a.q_lora + a.kv_lora + a.qk_rope, a.hidden);
  need((int)M, a.heads * HD, a.q_lora);
  need(L.Tmax, a.heads * HDv, a.kv_lora);
  need((int)M, a.hidden, a.heads * a.v_dim);
  L.lin = take(lin);
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
  if (!a) return fail(AMLA_EINVAL, "mla_prefill: null args");
  if (a->heads != P_H || a->kv_lora != 512 || a->qk_rope != P_ROPE || a->qk_nope != P_NOPE || a->v_dim != P_V)
    return fail(AMLA_EUNSUPPORTED, "mla_prefill: kernels are built for R1 head dimensions");
  if (a->batch <= 0 || a->seq_len <= 0) return fail(AMLA_EINVAL, "mla_prefill: batch and seq_len must be >= 1");
  if (a->hidden <= 0 || a->hidden % 128 || a->q_lora <= 0 || a->q_lora % 128)
    return fail(AMLA_EUNSUPPORTED, "mla_prefill: hidden and q_lora must be positive multiples of 128");
  const void *ptrs[] = {a->positions, a->hidden_states, a->out, a->w_q_a, a->s_q_a, a->w_q_b, a->s_q_b,
                        a->w_kv_a, a->s_kv_a, a->w_kv_b, a->s_kv_b, a->w_o, a->s_o, a->gamma_q,
                        a->gamma_kv, a->ckv_cache, a->kpe_cache, a->rope_table, a->workspace};
  for (const void *q : ptrs)
    if (!q) return fail(AMLA_EINVAL, "mla_prefill: a required pointer is null");
  const PrefillLayout L = prefill_layout(*a);
  if (a->max_context < a->seq_len)
    return fail(AMLA_EINVAL, "mla_prefill: max_context (%d) must be >= seq_len (%d)", a->max_context, a->seq_len);
  if (a->workspace_bytes < L.total)
    return fail(AMLA_EWORKSPACE, "mla_prefill: workspace %zu bytes < %zu needed", a->workspace_bytes, L.total);
  char *ws = reinterpret_cast<char *>(a->workspace);
  const int B = a->batch, S = a->seq_len, M = B * S;
  const int HD = a->qk_nope + a->qk_rope;
  int rc;

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
  uint16_t *attn = reinterpret_cast<uint16_t *>(ws + L.attn);

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
  pa.kv_lora = a->kv_lora; pa.rope = a->qk_rope; pa.pos = a->positions; pa.seq_len = S;
  if ((rc = run_linear(pa, GEMV_QKVA, st))) return rc;

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
  pb.head_dim = HD; pb.nope = a->qk_nope;
  if ((rc = run_linear(pb, GEMV_QROPE, st))) return rc;

  const int T = L.Tmax;
  FlashParams fp = {};
  fp.q = q; fp.kvb = kvb; fp.kpe = kpe; fp.out = attn; fp.pos = a->positions; fp.S = S;
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
    if ((rc = run_linear(pk, GEMV_PLAIN, st))) return rc;
    fp.b = b;
    flash_kernel<<<dim3(P_H, (S + P_QB - 1) / P_QB), 256, 0, st>>>(fp);
    if ((rc = check_launch("flash attention"))) return rc;
  }

  GemvParams po = {};
  po.part = reinterpret_cast<float *>(ws + L.lin);
  po.x = attn; po.M = M; po.ldx = a->heads * a->v_dim;
  po.w0 = reinterpret_cast<const uint8_t *>(a->w_o); po.s0 = a->s_o;
  po.N = a->hidden; po.K = a->heads * a->v_dim; po.n_split = po.N;
  po.y = reinterpret_cast<uint16_t *>(a->out); po.ldy = a->hidden;
  po.res = reinterpret_cast<const uint16_t *>(a->residual); po.ldr = a->hidden; po.seq_len = 1;
  return run_linear(po, a->residual ? GEMV_RESID : GEMV_PLAIN, st);
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
