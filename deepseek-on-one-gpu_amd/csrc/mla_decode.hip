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
//   rms_norm   : input RMSNorm of hidden (layer mode only, when it cannot be
//                folded into the next GEMV)
//   gemv  QKVA : q_a | kv_a in K parts (fp32 partial sums), or one streaming
//                pass for batch 1 that also writes the new cache row
//   finish     : sums the K parts, writes the new cache row (raw latent + raw
//                k_pe) and q_a_layernorm(q_a) (a row norm in place when the
//                GEMV needs no K parts, folded into q_b at batch 1)
//   gemv  QROPE: q = q_a_norm W_qb^T, RoPE on the q_pe rows at pos[b]
//   absorb     : qt = gamma_kv * W_UK^T q_nope -> qbuf (B, H, 576) with q_pe,
//                stored in attn_kernel's fragment order; one more workgroup
//                makes the split plan from the positions
//   attn       : split over context, fixed-reference softmax, bf16 partial O, (m, l)
//   combine_uv : merge splits, gamma_kv, W_UV -> (B, H*128) bf16
//   gemv  PLAIN/RESID : wo (+ residual), then its K-part finish
#include <limits.h>
#include <math.h>

#include <mutex>

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

// The absorbed query buffer holds, per sequence, the (H, 576) query matrix in
// the order attn_kernel's B fragments are loaded: for wave w (heads 32w ..
// 32w+31), head block nt (16 heads), K step ks (32 columns) and lane l, the
// 8 columns 32ks + 8(l/16) .. +7 of head 32w + 16nt + l%16 are 16 contiguous
// bytes, and one wave-wide 16-byte load reads 1 KB contiguously.
AMLA_DEV size_t qfrag_index(int b, int h, int c) {
  const int lane = (h & 15) + 16 * ((c & 31) >> 3);
  return ((((size_t)b * (HEADS / 16) + (h >> 4)) * (QKD / 32) + (c >> 5)) * 64 + lane) * 8 + (c & 7);
}

// ---------------------------------------------------------------- split plan

// Split plan of a decode batch, made on the device from the positions (no
// host synchronisation):
//   sequence b has N_b = ceil(T_b / TT) tiles (T_b = min(pos[b] + 1, tmax));
//   L is the smallest split length with sum_b ceil(N_b / L) <= units (reached
//   by L = max N_b at the latest, as batch <= units);
//   sequence b gets s_b = max(1, ceil(N_b / L)) splits in consecutive slots
//   first_b = s_0 + .. + s_{b-1}, and split j of b covers tiles
//   [j N_b / s_b, (j + 1) N_b / s_b), at most L of them.
// The launch takes as long as its longest split when every split has a CU, so
// a ragged batch is balanced by its total tokens, not by its longest sequence.
// A batch whose sequences all have the same tile count n has the plan in
// closed form (L = ceil(n / floor(units / B)), s_b = ceil(n / L), first_b =
// b s_b), which the attention and combine launches form themselves.  For any
// other batch one workgroup of the absorb launch writes the plan to a table
// that they read (int32): [0] L, [1] sum of s_b, [PLAN_HDR + 2b] first_b and
// [PLAN_HDR + 2b + 1] s_b (one 8-byte load), [PLAN_HDR + 2B + slot] the
// sequence of each slot (-1 past the plan).
constexpr int PLAN_HDR = 4;
inline size_t plan_ints(int B, int slots) { return PLAN_HDR + 2 * (size_t)B + slots; }

AMLA_DEV int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Smallest and largest tile count of the batch (B <= 64), wave-uniform: lane
// b loads sequence b's position (one vector load: a loop of scalar loads
// waited for each one in turn, a round trip per sequence), then a butterfly
// over the wave.  Every lane of the wave must call it.
AMLA_DEV int2 batch_tile_range(const int32_t *pos, int tmax, int B) {
  const int lane = threadIdx.x & 63;
  int lo = INT_MAX, hi = 0;
  if (lane < B) {
    const int T = min(pos[lane] + 1, tmax);
    lo = hi = T > 0 ? ceil_div(T, TT) : 0;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o, 64));
    hi = max(hi, __shfl_xor(hi, o, 64));
  }
  return int2{__builtin_amdgcn_readfirstlane(lo), __builtin_amdgcn_readfirstlane(hi)};
}

// Splits per sequence of a batch whose sequences all have n tiles.
AMLA_DEV int uniform_splits(int n, int units, int B) {
  return n > 0 ? ceil_div(n, ceil_div(n, units / B)) : 1;
}

// ceil(a / b) for 0 <= a < 2^22, b >= 1, with rb = 1 / b in fp32: the product
// is within 1 of a / b, so one correction step makes the quotient exact (an
// integer division is a long instruction sequence on the GPU).
AMLA_DEV int ceil_div_rcp(int a, int b, float rb) {
  int q = static_cast<int>(static_cast<float>(a) * rb);
  int r = a - q * b;
  if (r < 0) {
    --q;
    r += b;
  } else if (r >= b) {
    ++q;
    r -= b;
  }
  return q + (r > 0);
}

AMLA_DEV int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
AMLA_DEV int wave_max_int(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}

// The table of a batch with unequal tile counts, by one 256-thread workgroup
// (batch <= 64, the decode limit; lds holds 2 * B + 4 ints).  Wave 0 holds
// sequence b's tile count in lane b and finds L by bisection (the sum of
// ceil(N_b / L) does not grow with L, and L = max N_b fits), then s_b and
// first_b by a scan over its lanes; every thread then writes the sequence of
// its slots (a binary search over first_b).
AMLA_DEV void build_split_plan(const int32_t *__restrict__ pos, int tmax, int B, int units, int slots,
                               int32_t *__restrict__ plan, int *lds) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int *first = lds + B, *sh = lds + 2 * B;
  if (wave == 0) {
    int n = 0;
    if (lane < B) {
      const int T = min(pos[lane] + 1, tmax);
      n = T > 0 ? ceil_div(T, TT) : 0;
    }
    const int N = wave_sum_int(n), most = wave_max_int(n);
    int lo = max(1, ceil_div(N, units)), hi = max(lo, most);
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const float rm = 1.f / static_cast<float>(mid);
      const int f = wave_sum_int(lane < B ? ceil_div_rcp(n, mid, rm) : 0);
      if (f <= units) hi = mid;
      else lo = mid + 1;
    }
    const int L = lo;
    const int sb = lane < B ? max(1, ceil_div(n, L)) : 0;
    int incl = sb;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    if (lane < B) {
      first[lane] = incl - sb;
      plan[PLAN_HDR + 2 * lane] = incl - sb;
      plan[PLAN_HDR + 2 * lane + 1] = sb;
    }
    if (lane == B - 1) {
      plan[0] = L;
      plan[1] = incl;
      sh[0] = incl;
    }
  }
  __syncthreads();
  const int total = sh[0];
  // the sequence of each slot: the last b with first_b <= slot (first is
  // increasing, every s_b >= 1)
  for (int slot = tid; slot < slots; slot += 256) {
    int b = -1;
    if (slot < total) {
      int l = 0, r = B - 1;
      while (l < r) {
        const int mid = (l + r + 1) >> 1;
        if (first[mid] <= slot) l = mid;
        else r = mid - 1;
      }
      b = l;
    }
    plan[PLAN_HDR + 2 * B + slot] = b;
  }
}

// ---------------------------------------------------------------- absorb

// One workgroup (4 waves) per (head h, 128-column quarter q of the latent,
// group of 16 or 32 sequences): it stages the quarter W_UK[h][:, 128q .. +127]
// (16 KB, W_UK[h] = kv_b rows h*256 .. h*256+127, one 128-row scale block)
// and the group's q_nope rows in LDS; wave w computes latent columns
// 32w .. +31 of it by 16x16x32 MFMAs: A = q_nope (sequences x d; rows past
// the batch repeat real rows and are not stored), B = W_UK (d x latent
// column) by the 8-bit transpose read (lane L of a 16-lane group receives
// column L of the eight rows its group addresses), fp8 -> bf16 exactly;
// qt = gamma_kv * s_UK * sum, through LDS into 16-byte stores of the
// fragment-ordered query.  An extra workgroup (HEADS, 0, 0) writes the split
// plan table of a batch with unequal tile counts.
constexpr int AB_SEQ = 16;                // sequences per MFMA row tile (the MFMA's 16 rows)
constexpr int AB_WPITCH = 128 + 16;       // bytes per W_UK quarter row in LDS (fp8)
constexpr int AB_NPITCH = NOPE * 2 + 16;  // bytes per q_nope row (bf16)
constexpr int AB_OPITCH = 128 * 2 + 16;   // bytes per output row (bf16)

// RT row tiles of 16 sequences per workgroup (2 above 16 sequences: each
// W_UK fragment read feeds both, and the quarter is read once per 32)
template <int RT>
__global__ __launch_bounds__(256) void absorb_kernel(const uint16_t *__restrict__ q,  // (B, H, 192)
                                                     const uint8_t *__restrict__ wkvb,
                                                     const float *__restrict__ skvb,
                                                     const uint16_t *__restrict__ gamma, int B,
                                                     uint16_t *__restrict__ qbuf,
                                                     const int32_t *__restrict__ pos, int tmax, int units,
                                                     int slots, int32_t *__restrict__ plan) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef int v2i __attribute__((ext_vector_type(2)));
  constexpr int NS = RT * AB_SEQ;  // sequences of the workgroup
  __shared__ __align__(16) uint8_t wsm[NOPE * AB_WPITCH];
  __shared__ __align__(16) uint8_t nsm[NS * AB_NPITCH];
  __shared__ __align__(16) uint8_t osm[NS * AB_OPITCH];
  static_assert(sizeof(wsm) >= (2 * 64 + 8) * sizeof(int), "the plan's scratch (batch <= 64) fits wsm");
  const int h = blockIdx.x, quarter = blockIdx.y, b0 = blockIdx.z * NS;
  const int nb = min(NS, B - b0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  if (h == HEADS) {
    // the extra column of workgroups: (HEADS, 0, 0) writes the split plan of
    // a batch with unequal tile counts (alongside the absorb workgroups, not
    // before one of them), the others have no work
    if (quarter == 0 && blockIdx.z == 0) {
      const int2 r = batch_tile_range(pos, tmax, B);
      if (r.x != r.y) build_split_plan(pos, tmax, B, units, slots, plan, reinterpret_cast<int *>(wsm));
    }
    return;
  }
  // W_UK quarter: 128 rows x 128 bytes, four 16-byte pieces per thread
  // (non-temporal when this is the only group of sequences reading it);
  // q_nope rows, one 16-byte piece per thread (rows past the batch re-read
  // its last row)
  const uint8_t *wq = wkvb + (size_t)h * (NOPE + VD) * LORA + quarter * 128;
  u32x4 wv[4];
  if (gridDim.z == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 256 * i;
      wv[i] = ldg16_nt(wq + (size_t)(p >> 3) * LORA + (p & 7) * 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 256 * i;
      wv[i] = ldg16(wq + (size_t)(p >> 3) * LORA + (p & 7) * 16);
    }
  }
  u32x4 nv[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    nv[r] = ldg16(q + ((size_t)(b0 + min(16 * r + (tid >> 4), nb - 1)) * HEADS + h) * (NOPE + ROPE) + (tid & 15) * 8);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 256 * i;
    *reinterpret_cast<u32x4 *>(wsm + (p >> 3) * AB_WPITCH + (p & 7) * 16) = wv[i];
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) *reinterpret_cast<u32x4 *>(nsm + (16 * r + (tid >> 4)) * AB_NPITCH + (tid & 15) * 16) = nv[r];
  __syncthreads();

  bf16x8 a[RT][NOPE / 32];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int ks = 0; ks < NOPE / 32; ++ks)
      a[r][ks] = as_bf16x8(*reinterpret_cast<const u32x4 *>(nsm + (16 * r + li) * AB_NPITCH + (32 * ks + 8 * lg) * 2));
  const float sc = skvb[(size_t)(2 * h) * (LORA / 128) + quarter];
#pragma unroll
  for (int cbi = 0; cbi < 2; ++cbi) {
    const int cb = 2 * wave + cbi;
    f32x4 d4[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) d4[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NOPE / 32; ++ks) {
      const uint8_t *ap = wsm + (32 * ks + 8 * lg + (li >> 1)) * AB_WPITCH + 16 * cb + 8 * (li & 1);
      const v2i w2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i *)ap);
      const bf16x2_t c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w2.x, 1.f, false);
      const bf16x2_t c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w2.x, 1.f, true);
      const bf16x2_t c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w2.y, 1.f, false);
      const bf16x2_t c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w2.y, 1.f, true);
      const bf16x8 bw = {c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
#pragma unroll
      for (int r = 0; r < RT; ++r) d4[r] = mfma16(a[r][ks], bw, d4[r]);
    }
    // D: latent column 16 cb + li of the quarter, sequences b0 + 16 r + 4 lg .. +3
    const int c = 16 * cb + li;
    const float g = bf2f(gamma[quarter * 128 + c]);
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<uint16_t *>(osm + (16 * r + 4 * lg + e) * AB_OPITCH + c * 2) = f2bf(d4[r][e] * sc * g);
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int m = 16 * r + (tid >> 4), c8 = tid & 15;
    if (m < nb)
      *reinterpret_cast<u32x4 *>(qbuf + qfrag_index(b0 + m, h, quarter * 128 + c8 * 8)) =
          *reinterpret_cast<const u32x4 *>(osm + m * AB_OPITCH + c8 * 16);
  }
  // rope half of the query: copied next to the absorbed latent query
  if (quarter == 0) {
    for (int e = tid; e < nb * (ROPE / 2); e += 256) {
      const int m = e / (ROPE / 2), j = (e % (ROPE / 2)) * 2;
      const uint32_t v =
          *reinterpret_cast<const uint32_t *>(q + ((size_t)(b0 + m) * HEADS + h) * (NOPE + ROPE) + NOPE + j);
      *reinterpret_cast<uint32_t *>(qbuf + qfrag_index(b0 + m, h, LORA + j)) = v;
    }
  }
}

// ---------------------------------------------------------------- attention

template <bool V>
struct BoolC {
  static constexpr bool value = V;
};

struct AttnParams {
  const uint16_t *qbuf;  // B x (H, 576) bf16 in fragment order (qfrag_index): absorbed latent query | rotated rope query
  const uint16_t *ckv;   // cache (B_alloc, max_seq, 512)
  const uint16_t *kpe;   // cache (B_alloc, max_seq, 64)
  int64_t ckv_bstride, kpe_bstride;  // elements per sequence
  const float *rope_table;           // (rows, 32, 2)
  const int32_t *pos;                // decode position per sequence; context T = min(pos + 1, tmax)
  int tmax;                          // context bound (rows of cache and rope table that may be read)
  int units;         // splits shared out over the batch (the grid has units + batch workgroups)
  int batch;
  const int32_t *plan;  // split plan (build_split_plan)
  float scale_log2;  // softmax scale * log2(e)
  float eps;
  uint16_t *part_o;  // (units + B, H, 512) bf16 by split slot: sum_t p_t r_t c_t, p relative to the split's reference max
  float *part_ml;  // (units + B, H, 2) reference max (log2 units) and sum of p; sum < 0 marks a
                   // (split, head) whose scores overflowed the reference (recomputed by the combine)
};

// A sequence's splits in the plan: first slot, count, and its tile count.
struct SeqSplits {
  int first, count, ntiles;
};

AMLA_DEV int seq_tiles(const AttnParams &p, int b) {
  const int T = min(p.pos[b] + 1, p.tmax);
  return T > 0 ? (T + TT - 1) / TT : 0;
}

AMLA_DEV SeqSplits seq_splits(const AttnParams &p, int b) {
  const int2 r = batch_tile_range(p.pos, p.tmax, p.batch);
  if (r.x == r.y) {
    const int s = uniform_splits(r.x, p.units, p.batch);
    return SeqSplits{b * s, s, r.x};
  }
  const int2 fs = *reinterpret_cast<const int2 *>(p.plan + PLAN_HDR + 2 * b);
  return SeqSplits{fs.x, fs.y, seq_tiles(p, b)};
}

// tile range of split j of a sequence with nb tiles in s splits
AMLA_DEV int split_tile(int nb, int s, int j) { return (int)(((int64_t)j * nb) / s); }

// LDS: a ring of NST stages, each one tile of TT cache rows
//   K   [TT][KROW] bf16: raw latent row (DMA) | rotated rope key / r_t (written after DMA)
//   raw [TT][64]   bf16: raw rope keys (DMA)
//   rt  [TT]       fp32: r_t = rsqrt(mean(c_t^2) + eps) of each row
// plus two (cos, sin) table blocks (tiles of even / odd index), copied two
// tiles ahead like the rows, and the tile's probabilities P^T of all heads.
constexpr int NST = 3;
// 1184 B rows (592 bf16).  A 16-byte LDS read is served 16 consecutive lanes
// per pass, free of bank conflicts when their addresses differ in bits 4-7
// (measured on MI355X), so the score fragment reads (16 rows of one chunk per
// pass, stride 74 x 16 B) pair rows r and r + 8; an odd pitch (1168 B) removes
// that and measured the same, the second passes being hidden in this kernel
constexpr int KROW = QKD + 16;
constexpr int K_BYTES = TT * KROW * 2;
constexpr int RAW_BYTES = TT * ROPE * 2;
constexpr int RT_OFF = K_BYTES + RAW_BYTES;  // r_t of the tile's rows, fp32
constexpr int STAGE_BYTES = RT_OFF + TT * 4;
constexpr int TAB_OFF = NST * STAGE_BYTES;
constexpr int TAB_BYTES = TT * ROPE * 4;
constexpr int P_OFF = TAB_OFF + 2 * TAB_BYTES;
constexpr int PROW = TT * 2 + 16;  // bf16 probabilities of one head, 80 B rows (conflict-free 16 B reads)
constexpr int ATTN_LDS_BYTES = P_OFF + HEADS * PROW;
constexpr int OROW = LORA * 2 + 32;  // LDS row of one head's partial O at the end (bf16, padded)
static_assert(HEADS * OROW <= ATTN_LDS_BYTES, "partial O staging must fit the attention LDS");
constexpr int TILE_DMA = 11;  // copies per wave per tile: 8 latent rows, 1 block of rope keys, 2 table blocks
// p = 2^(s - m_ref): a split whose sum of p reaches 2^64 (a later score far
// above the first tile's maximum) is flagged and recomputed exactly
constexpr float REF_HEADROOM_SUM = 18446744073709551616.f;  // 2^64

// Wave w copies rows 8w .. 8w+7 of a tile straight into LDS (no VGPRs):
// every global_load_lds_dwordx4 writes 64 lanes x 16 B contiguously at its
// LDS base.  Row indices are wave-uniform (scalar bases, one lane offset).
// Rows past the context re-read row T-1 (in bounds; their scores are masked).
// The cache rows are copied non-temporal (aux 2: each is read once per step);
// the (cos, sin) rows, which every sequence of the batch reads, are not.
// Piece 0..7: latent row 8w + piece; 8: the 8 rows' raw rope keys; 9, 10: the
// (cos, sin) table rows of the 8 rows (2 x 1 KB), into the table block of the
// tile's parity.  The tile loop issues one piece per score step: a burst of
// LDS copies stalls the issuing wave for tens of cycles per copy.
AMLA_DEV void dma_piece(const AttnParams &p, int b, int tile, int parity, int T, uint8_t *smem, uint8_t *stage,
                        int wave, int lane, uint32_t lane16, int piece) {
  const int t0 = tile * TT + wave * 8;
  if (piece < 8) {
    // one row: the clamp is on the scalar row index, every lane at lane16 = 16 * lane
    const char *cb = reinterpret_cast<const char *>(p.ckv + (size_t)b * p.ckv_bstride);
    const int t = min(t0 + piece, T - 1);
    __builtin_amdgcn_global_load_lds(cb + (size_t)t * (LORA * 2) + lane16,
                                     LDS_PTR(stage + (wave * 8 + piece) * (KROW * 2)), 16, 0, 2);
    return;
  }
  const int t0c = min(t0, T - 1);
  // lane-derived offsets are unsigned (scalar base + 32-bit lane offset
  // addressing) and recomputed per copy, not held across the loop
  uint32_t ln;
  asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
  if (piece == 8) {
    const char *kb = reinterpret_cast<const char *>(p.kpe + (size_t)b * p.kpe_bstride) + (size_t)t0c * (ROPE * 2);
    const uint32_t row = static_cast<uint32_t>(min(t0 + static_cast<int>(ln >> 3), T - 1) - t0c);
    __builtin_amdgcn_global_load_lds(kb + row * (ROPE * 2) + (ln & 7u) * 16u, LDS_PTR(stage + K_BYTES + wave * 1024), 16,
                                     0, 2);
  } else {
    const char *tb = reinterpret_cast<const char *>(p.rope_table) + (size_t)t0c * (ROPE * 4);
    const uint32_t e = static_cast<uint32_t>(piece - 9) * 64u + ln;
    const uint32_t row = static_cast<uint32_t>(min(t0 + static_cast<int>(e >> 4), T - 1) - t0c);
    __builtin_amdgcn_global_load_lds(
        tb + row * (ROPE * 4) + (e & 15u) * 16u,
        LDS_PTR(smem + TAB_OFF + (parity & 1) * TAB_BYTES + wave * 2048 + (piece - 9) * 1024), 16, 0, 0);
  }
}

AMLA_DEV void dma_tile(const AttnParams &p, int b, int tile, int T, uint8_t *smem, uint8_t *stage, int wave, int lane) {
#pragma unroll
  for (int piece = 0; piece < TILE_DMA; ++piece)
    dma_piece(p, b, tile, tile, T, smem, stage, wave, lane, static_cast<uint32_t>(lane) * 16u, piece);
}

AMLA_DEV uint32_t rot_pair(uint32_t x, float c, float s) {
  const float a = lo_bf(x), b = hi_bf(x);
  return pack_bf16(__fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s)), __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c)));
}


AMLA_DEV float dot2_bf16(uint32_t a, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = __builtin_bit_cast(bf16x2, a);
  return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
}

template <int CTRL>
AMLA_DEV float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Wave w prepares the 8 rows it copied, 8 lanes per row (lane q of a row
// reads 16 B chunks q, q+8, ..: eight lanes cover 128 contiguous bytes):
//   r_t = rsqrt(mean(c_t^2) + eps) (rms_norm's factor, inference/ops.py:10-12)
//     goes to the stage's rt array; the latent row stays raw;
//   the rope key is rotated in fp32 and rounded to bf16 (inference/ops.py:93-97).
AMLA_DEV void prepare_own_rows(uint8_t *stage, const uint8_t *tab, int wave, int lane, float eps) {
  int ln;  // lane-derived addresses are recomputed here, not held across the tile loop
  asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
  const int row = wave * 8 + (ln >> 3), q = ln & 7;
  uint8_t *rp = stage + row * (KROW * 2);
  // two batches of four 16-byte reads keep the register footprint small
  float ss = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const u32x4 *>(rp + (q + 8 * (4 * h + i)) * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ss = dot2_bf16(v[i].x, ss);
      ss = dot2_bf16(v[i].y, ss);
      ss = dot2_bf16(v[i].z, ss);
      ss = dot2_bf16(v[i].w, ss);
    }
    asm volatile("" ::: "memory");
  }
  const u32x4 raw = *reinterpret_cast<const u32x4 *>(stage + K_BYTES + row * (ROPE * 2) + q * 16);
  const f32x4 c0 = *reinterpret_cast<const f32x4 *>(tab + row * (ROPE * 4) + q * 32);
  const f32x4 c1 = *reinterpret_cast<const f32x4 *>(tab + row * (ROPE * 4) + q * 32 + 16);
  // sum over the 8 lanes of the row: quad xor 1, xor 2, then the other quad
  ss += dpp_f32<0xB1>(ss);   // quad_perm [1,0,3,2]
  ss += dpp_f32<0x4E>(ss);   // quad_perm [2,3,0,1]
  ss += dpp_f32<0x141>(ss);  // row_half_mirror
  // v_rsq_f32 directly: the argument is at least eps, far from the denormal range
  if (q == 0) *reinterpret_cast<float *>(stage + RT_OFF + row * 4) = __builtin_amdgcn_rsqf(ss * (1.f / LORA) + eps);
  u32x4 k;
  k.x = rot_pair(raw.x, c0.x, c0.y);
  k.y = rot_pair(raw.y, c0.z, c0.w);
  k.z = rot_pair(raw.z, c1.x, c1.y);
  k.w = rot_pair(raw.w, c1.z, c1.w);
  *reinterpret_cast<u32x4 *>(rp + (LORA + q * 8) * 2) = k;
}


// sum / max over the four lanes l, l^16, l^32, l^48 (lane swaps, no LDS)
AMLA_DEV float sum_lane_groups(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
AMLA_DEV float max_lane_groups(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}


// Grid: one workgroup per split slot (seq_splits) and group of HG = 64 NTW
// heads (NTW = 2: all 128 heads, grid (slots); NTW = 1: two head groups, grid
// (slots, 2), for launches with few slots, where the query load and the
// partial O store of a workgroup, both in proportion to its heads, dominate);
// 256 threads, one workgroup per CU (~150 KB of LDS).
// Scores: wave w owns heads 16 NTW w .. of the group; values: wave w owns
// latent columns 128w .. 128w+127 of every head of the group.  Per tile of 32
// cache rows:
//   each wave computes r_t of its 8 copied rows and rotates their rope keys,
//     one tile ahead of use;
//   S^T (t x head) = K_tile (32 x 576) . Q^T with the tile rows as the MFMA M
//     dimension, so each lane ends with 8 scores of one head (its column);
//     18 K steps of 32 (16 latent, then r_t applied, 2 rotated rope), A
//     fragments read from LDS three steps ahead;
//   p = 2^(s - m_ref): m_ref is the head's max over the split's first tile and
//     stays fixed, so O^T is only ever touched by MFMA (no rescaling); a head
//     whose sum of p reaches 2^64 (a later score far above m_ref) is flagged
//     instead and recomputed exactly by the combine;
//   P^T (p * r_t as bf16) of the wave's heads goes to LDS;
//   O^T (128 latent x HG heads, fp32) += C^T (128 x t) . P^T (t x HG), C^T
//     by transpose reads of the wave's 128 columns of the raw tile: first the
//     wave's own heads (P from registers), then, after a barrier, the other
//     waves' heads from LDS.
// Registers (NTW = 2): O^T takes 256 accumulators, the query fragments 144; the loop
// must not spill (a scratch reload would wait for every copy in flight),
// which is why the copies use scalar bases and there is no rescaling path.
//
// LDS reads of the score steps and the transpose reads are inline asm with
// explicit lgkmcnt waits: the compiler would otherwise wait for every read
// (and, for the transpose builtin, every LDS-DMA copy) before each use.  A
// wait names the registers it guards as in/out operands so no use is
// scheduled before it.  Counting only this code's own reads is safe: LDS
// operations complete in order, so any other LDS operation issued in between
// only makes a wait stricter; nothing in the loop uses scalar memory loads.
template <int NTW>
__global__ __launch_bounds__(256, 1) void attn_kernel(AttnParams p) {
  static_assert(NTW == 1 || NTW == 2, "16 or 32 heads per wave");
  constexpr int HPW = 16 * NTW;  // heads per wave (scores)
  constexpr int HG = 4 * HPW;    // heads of the workgroup
  constexpr int NH = HG / 16;    // 16-head blocks of the workgroup (PV)
  constexpr int NO = NH - NTW;   // blocks of the other waves
  const int slot = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  // this workgroup's (sequence, split) from the batch's split plan; slots past
  // the plan have no work
  int b, split, ns;
  const int2 range = batch_tile_range(p.pos, p.tmax, p.batch);
  if (range.x == range.y) {
    ns = uniform_splits(range.x, p.units, p.batch);
    b = slot / ns;
    split = slot % ns;
    if (b >= p.batch) return;
  } else {
    b = __builtin_amdgcn_readfirstlane(p.plan[PLAN_HDR + 2 * p.batch + slot]);
    if (b < 0) return;
    const int2 fs = *reinterpret_cast<const int2 *>(p.plan + PLAN_HDR + 2 * b);
    split = slot - __builtin_amdgcn_readfirstlane(fs.x);
    ns = __builtin_amdgcn_readfirstlane(fs.y);
  }
  const int nb = seq_tiles(p, b);
  const int T = min(p.pos[b] + 1, p.tmax);
  const int tb = split_tile(nb, ns, split);
  const int te = split_tile(nb, ns, split + 1);
  extern __shared__ __align__(16) uint8_t smem[];
  const int hl0 = wave * HPW;                     // the wave's first head in the group
  const int head0 = blockIdx.y * HG + hl0;
  const uint32_t lane16 = static_cast<uint32_t>(lane) * 16u;  // the copies' lane offset inside the context

  // the first tile's copies, then the query fragments (B operand: head =
  // column l%16, K = 8*lg .. of each 32-wide step); the first tile starts
  // once both have landed (the compiler's wait before the first fragment use
  // is for every load issued so far), the second tile's copies go out during
  // its score steps
  if (tb < te) dma_tile(p, b, tb, T, smem, smem, wave, lane);
  __builtin_amdgcn_sched_barrier(0);
  constexpr int QLOADS = NTW * (QKD / 32);  // per wave, after the copies
  static_assert(TILE_DMA + QLOADS <= 63, "vmcnt range");
  bf16x8 qf[NTW][QKD / 32];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    const uint16_t *qr = p.qbuf + qfrag_index(b, head0 + nt * 16, 0) + lane * 8;
#pragma unroll
    for (int ks = 0; ks < QKD / 32; ++ks) qf[nt][ks] = as_bf16x8(ldg16(qr + ks * 512));
  }
  __builtin_amdgcn_sched_barrier(0);

  f32x4 o[8][NH];  // O^T: latent 128*wave + 16*mt + .., head block (NTW*wave + j) % NH of the group
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) o[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_ref[NTW], l_run[NTW];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    m_ref[nt] = -INFINITY;
    l_run[nt] = 0.f;
  }

  if (tb < te) {
    // the first tile's copies landed (the query loads, issued after them, may
    // still be in flight: loads complete in order)
    wait_vmcnt<QLOADS>();
    prepare_own_rows(smem, smem + TAB_OFF + (tb & 1) * TAB_BYTES, wave, lane, p.eps);
    // LDS-only barrier: __syncthreads would also wait for the second tile's
    // copies (each wave waited for its own first-tile copies above; the second
    // tile is waited for after the first one)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    bool have_ref = false;
    // One tile.  FIRST (the split's first tile) prepares no next tile inside
    // its score steps: it starts once its own copies have landed, and the
    // second tile, whose copies were issued with them, is prepared after it.
    auto tile_body = [&](const int tile, auto first_c) __attribute__((always_inline)) {
      constexpr bool FIRST = decltype(first_c)::value;
      const int it = tile - tb;
      uint8_t *const cur = smem + (it % NST) * STAGE_BYTES;
      // copies of the tile after next, one per score step below (its stage was
      // last read in the previous tile; the table block only ever holds this
      // wave's rows)
      uint8_t *const nst = smem + ((it + 2) % NST) * STAGE_BYTES;
      const uint16_t *K = reinterpret_cast<const uint16_t *>(cur);

      // ---- scores: 18 K steps, A fragments SD steps ahead.  The MFMAs are
      // inline asm with VGPR accumulators (the O accumulators own the AGPRs);
      // the compiler does not track their hazards, so the VALU touches of sc
      // below are preceded by explicit wait states.
      // The next tile's own-row preparation (r_t and the rope rotation, as
      // prepare_own_rows) runs inside this loop between the MFMAs: its 11 LDS
      // reads go out in three batches (iterations 0, 5, 10), are consumed five
      // iterations later, and its two LDS writes follow at iteration 15; the
      // current tile's r_t is read at iteration 12 for step 16.  Every
      // LDS operation here is inline asm issued in a fixed order, so the wait
      // for step k's A fragments is a fixed count (LDS operations complete in
      // order): kLgkm[k] = operations issued after step k's two reads.  The
      // preparation always runs (past the last tile it reads and writes a stage
      // nothing reads any more) so that the counts hold.
      constexpr int NSTEP = QKD / 32;
      constexpr int SD = 3;
      constexpr int F3 = NSTEP - TILE_DMA;  // the first tile's first step copying the third tile
      static_assert(F3 > 0 && F3 < TILE_DMA, "first-tile copy schedule");
      constexpr int kLgkmN[NSTEP] = {4, 8, 8, 8, 4, 4, 8, 8, 8, 4, 4, 7, 7, 9, 6, 6, 4, 2};
      // the first tile: only the fragment reads and the r_t reads of step 12
      constexpr int kLgkmF[NSTEP] = {4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 6, 6, 6, 2, 0};
      const uint32_t kaddr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) const uint16_t *)(K + li * KROW + 8 * lg)));
#define AMLA_RDA(dst, S, MT) \
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(kaddr), "i"(((MT) * 16 * KROW + (S) * 32) * 2))
#define AMLA_RD(dst, addr, off) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(off))
      f32x4 sc[2][NTW];
      // r_t of the lane's C-layout rows 4*lg + r (mt 0) and 16 + 4*lg + r (mt 1)
      // (read at iteration 12, needed from step 16 on)
      f32x4 rc[2];
      u32x4 ab[SD][2];
#pragma unroll
      for (int d = 0; d < SD; ++d) {
        AMLA_RDA(ab[d][0], d, 0);
        AMLA_RDA(ab[d][1], d, 1);
      }
      // next tile's rows: this wave's 8 rows, 8 lanes per row (lane q of a row
      // owns 16-byte chunks q, q+8, .. of the latent row)
      uint8_t *const nxt = smem + ((it + 1) % NST) * STAGE_BYTES;
      const uint8_t *const tabn = smem + TAB_OFF + ((tile + 1) & 1) * TAB_BYTES;
      int pln;
      asm volatile("v_mov_b32 %0, %1" : "=v"(pln) : "v"(lane));  // recomputed per tile, not held
      const int prow = wave * 8 + (pln >> 3), pq = pln & 7;
      const uint32_t rpa = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) const uint8_t *)(nxt + prow * (KROW * 2) + pq * 16)));
      u32x4 pv4[4], praw, pc0, pc1;
      float pss = 0.f;
#pragma unroll
      for (int ks = 0; ks < NSTEP; ++ks) {
        const int c = ks % SD;
        switch (FIRST ? kLgkmF[ks] : kLgkmN[ks]) {
          case 9: asm volatile("s_waitcnt lgkmcnt(9)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
          case 8: asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
          case 7: asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
          case 6: asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
          case 4: asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
          case 2: asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
          default: asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ab[c][0]), "+v"(ab[c][1])::"memory"); break;
        }
        if (ks == LORA / 32) {
          // latent part complete: apply r_t before the rope K steps (MFMA
          // write -> VALU read, then VALU write -> MFMA read wait states)
          asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(rc[0]), "+v"(rc[1])::"memory");
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) sc[mt][nt] *= rc[mt];
          if constexpr (NTW == 2)
            asm volatile("s_nop 4" : "+v"(sc[0][0]), "+v"(sc[0][1]), "+v"(sc[1][0]), "+v"(sc[1][1])::"memory");
          else
            asm volatile("s_nop 4" : "+v"(sc[0][0]), "+v"(sc[1][0])::"memory");
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) {
            if (ks == 0)
              asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=v"(sc[mt][nt]) : "v"(ab[c][mt]), "v"(qf[nt][ks]));
            else
              asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(sc[mt][nt]) : "v"(ab[c][mt]), "v"(qf[nt][ks]));
          }
        // consume a batch of the next tile's rows (landed: this step's wait
        // covers every operation issued before step ks's reads).  The empty
        // asm names the registers, so the compiler cannot hoist their use
        // above the wait: a wait orders memory operations, not register uses.
        if (!FIRST && (ks == 5 || ks == 10)) {
          asm volatile("" : "+v"(pv4[0]), "+v"(pv4[1]), "+v"(pv4[2]), "+v"(pv4[3]));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pss = dot2_bf16(pv4[i].x, pss);
            pss = dot2_bf16(pv4[i].y, pss);
            pss = dot2_bf16(pv4[i].z, pss);
            pss = dot2_bf16(pv4[i].w, pss);
          }
        }
        if (!FIRST && ks == 15) {
          // r_t = rsqrt(mean(c_t^2) + eps): sum over the row's 8 lanes (every
          // lane of the row ends with the total); rope key rotated in fp32,
          // rounded to bf16 (inference/ops.py:10-12, :93-97); the reads of
          // iteration 10 are pinned after this step's wait like pv4 above
          asm volatile("" : "+v"(praw), "+v"(pc0), "+v"(pc1));
          pss += dpp_f32<0xB1>(pss);   // quad_perm [1,0,3,2]
          pss += dpp_f32<0x4E>(pss);   // quad_perm [2,3,0,1]
          pss += dpp_f32<0x141>(pss);  // row_half_mirror
          const float rt = __builtin_amdgcn_rsqf(pss * (1.f / LORA) + p.eps);
          const f32x4 c0 = __builtin_bit_cast(f32x4, pc0), c1 = __builtin_bit_cast(f32x4, pc1);
          u32x4 kr;
          kr.x = rot_pair(praw.x, c0.x, c0.y);
          kr.y = rot_pair(praw.y, c0.z, c0.w);
          kr.z = rot_pair(praw.z, c1.x, c1.y);
          kr.w = rot_pair(praw.w, c1.z, c1.w);
          const uint32_t rta = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
              (__attribute__((address_space(3))) const uint8_t *)(nxt + RT_OFF + prow * 4)));
          asm volatile("ds_write_b32 %0, %1\n\tds_write_b128 %2, %3 offset:%4"
                       :
                       : "v"(rta), "v"(rt), "v"(rpa), "v"(kr), "i"(LORA * 2 - 0)
                       : "memory");
        }
        if (ks + SD < NSTEP) {
          AMLA_RDA(ab[c][0], ks + SD, 0);
          AMLA_RDA(ab[c][1], ks + SD, 1);
        }
        if (!FIRST && ks == 0) {
          // the next tile's copies landed (issued during the previous tile;
          // this tile's own copies start below)
          wait_vmcnt<0>();
          AMLA_RD(pv4[0], rpa, 0);
          AMLA_RD(pv4[1], rpa, 128);
          AMLA_RD(pv4[2], rpa, 256);
          AMLA_RD(pv4[3], rpa, 384);
        } else if (!FIRST && ks == 5) {
          AMLA_RD(pv4[0], rpa, 512);
          AMLA_RD(pv4[1], rpa, 640);
          AMLA_RD(pv4[2], rpa, 768);
          AMLA_RD(pv4[3], rpa, 896);
        } else if (!FIRST && ks == 10) {
          const uint32_t rawa = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
              (__attribute__((address_space(3))) const uint8_t *)(nxt + K_BYTES + prow * (ROPE * 2) + pq * 16)));
          const uint32_t taba = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
              (__attribute__((address_space(3))) const uint8_t *)(tabn + prow * (ROPE * 4) + pq * 32)));
          AMLA_RD(praw, rawa, 0);
          AMLA_RD(pc0, taba, 0);
          AMLA_RD(pc1, taba, 16);
        } else if (ks == 12) {
          const uint32_t ra = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
              (__attribute__((address_space(3))) const uint8_t *)(cur + RT_OFF + (4 * lg) * 4)));
          // early-clobber outputs: the second read still needs the address register
          asm volatile("ds_read_b128 %0, %2 offset:0\n\tds_read_b128 %1, %2 offset:64" : "=&v"(rc[0]), "=&v"(rc[1]) : "v"(ra));
        }
        // unconditional (no branch per copy): past the split's end the last
        // tile is copied again (an L2 hit) into a stage nothing reads any more;
        // the table block is the parity of tile + 2, never the one the
        // preparation of tile + 1 reads
        if constexpr (FIRST) {
          // the second tile's copies (steps 0 .. 10), then the third tile's
          // (steps 7 .. 17, after the second tile's piece of the same step)
          if (ks < TILE_DMA)
            dma_piece(p, b, min(tile + 1, te - 1), tile + 1, T, smem, smem + STAGE_BYTES, wave, lane, lane16, ks);
          if (ks >= F3)
            dma_piece(p, b, min(tile + 2, te - 1), tile + 2, T, smem, nst, wave, lane, lane16, ks - F3);
        } else {
          if (ks < TILE_DMA) dma_piece(p, b, min(tile + 2, te - 1), tile + 2, T, smem, nst, wave, lane, lane16, ks);
        }
      }
      // the softmax reads sc: MFMA write -> VALU read wait states
      if constexpr (NTW == 2)
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(sc[0][0]), "+v"(sc[0][1]), "+v"(sc[1][0]), "+v"(sc[1][1])::"memory");
      else
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(sc[0][0]), "+v"(sc[1][0])::"memory");
#undef AMLA_RD
#undef AMLA_RDA
      __builtin_amdgcn_sched_barrier(0);

      // ---- probabilities relative to the head's fixed reference max; r_t of
      // the lane's rows 4*lg + r (mt 0) and 16 + 4*lg + r (mt 1)
      // (the scale is positive: the max is taken on the raw scores, and
      // 2^(scale*s - m_ref) is one fma and one exp per score; rows past the
      // context exist only in the last tile of a sequence)
      const int tbase = tile * TT;
      const bool partial = tbase + TT > T;
      u32x4 pk[NTW];
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        float sv[8];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[mt * 4 + r] = sc[mt][nt][r];
        if (partial) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (tbase + (e >> 2) * 16 + 4 * lg + (e & 3) >= T) sv[e] = -INFINITY;
        }
        if (!have_ref) {  // the split's first tile fixes the reference max (a wave-uniform branch)
          const float mx =
              fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
          m_ref[nt] = p.scale_log2 * max_lane_groups(mx);
        }
        float pv[8];
        float lsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(p.scale_log2, sv[e], -m_ref[nt]));  // 2^-inf = 0
          lsum += pe;
          pv[e] = pe * rc[e >> 2][e & 3];
        }
        l_run[nt] += lsum;
        pk[nt] = u32x4{pack_bf16(pv[0], pv[1]), pack_bf16(pv[2], pv[3]), pack_bf16(pv[4], pv[5]),
                       pack_bf16(pv[6], pv[7])};
      }
      have_ref = true;

      // ---- P^T of this wave's heads to LDS, for the other waves: row = head,
      // bf16 slot 8*lg + j holds t = 4*lg + j (j < 4) or 16 + 4*lg + j - 4:
      // exactly this lane's eight scores, and the k order of the transpose
      // reads below (so pk[nt] is also this wave's own B fragment)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
        asm volatile("ds_write_b128 %0, %1" ::"v"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                         (__attribute__((address_space(3))) uint8_t *)(smem + P_OFF + (hl0 + nt * 16 + li) * PROW +
                                                                       lg * 16)))),
                     "v"(pk[nt])
                     : "memory");

      // ---- O^T (latent x head) += C^T (latent x t) . P^T (t x head).  C^T by
      // transpose reads: within a 16-lane group, lane s addresses row
      // t0 + s/4, columns c0 + 4(s%4) .. +3 and lane L receives
      // C[t0 .. t0+3][c0 + L]; t0 = 4*lg and 16 + 4*lg match P^T's k order.
      // All eight column blocks of this wave's 128 latent columns are read
      // once and kept for both passes (outputs early-clobber: two reads share
      // one address).  Accumulator block j holds head block (NTW*wave + j) % NH
      // of the group, so blocks j < NTW are this wave's own heads: their MFMAs
      // run on P straight from registers while the other waves' P^T is
      // written, and only the other NO blocks wait for the barrier.
      const int s16 = lane & 15;
      const uint32_t a0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) const uint16_t *)(K + (4 * lg + (s16 >> 2)) * KROW + wave * 128 +
                                                                4 * (s16 & 3))));
      u32x2 ta[8], tb[8];
#define AMLA_TR(MT)                                                                                        \
  asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"               \
               : "=&v"(ta[MT]), "=&v"(tb[MT])                                                            \
               : "v"(a0), "i"((MT) * 32), "i"((MT) * 32 + 16 * KROW * 2))
      AMLA_TR(0); AMLA_TR(1); AMLA_TR(2); AMLA_TR(3); AMLA_TR(4); AMLA_TR(5); AMLA_TR(6); AMLA_TR(7);
#undef AMLA_TR
      // wait for column block MT's reads (LDS operations complete in order:
      // 2 * (7 - MT) reads were issued after them); the P^T writes before them
      // are then complete too
#define AMLA_WTR(MT, N) \
  asm volatile("s_waitcnt lgkmcnt(" #N ")" : "+v"(ta[MT]), "+v"(tb[MT])::"memory")
      // the own-head MFMAs read pk, written by VALU (the cvt/pack above): cover
      // the VALU write -> MFMA read wait states the compiler does not see
      if constexpr (NTW == 2)
        asm volatile("s_nop 4" : "+v"(pk[0]), "+v"(pk[1])::"memory");
      else
        asm volatile("s_nop 4" : "+v"(pk[0])::"memory");
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        switch (mt) {
          case 0: AMLA_WTR(0, 14); break;
          case 1: AMLA_WTR(1, 12); break;
          case 2: AMLA_WTR(2, 10); break;
          case 3: AMLA_WTR(3, 8); break;
          case 4: AMLA_WTR(4, 6); break;
          case 5: AMLA_WTR(5, 4); break;
          case 6: AMLA_WTR(6, 2); break;
          default: AMLA_WTR(7, 0); break;
        }
        const bf16x8 a = as_bf16x8(u32x4{ta[mt].x, ta[mt].y, tb[mt].x, tb[mt].y});
#pragma unroll
        for (int j = 0; j < NTW; ++j)
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(o[mt][j]) : "v"(a), "v"(pk[j]));
      }
#undef AMLA_WTR
      // every LDS operation of this wave is complete (lgkmcnt(0) above): after
      // the barrier all waves' P^T is visible
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      u32x4 pb[NO];
      {
        const uint32_t paddr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
            (__attribute__((address_space(3))) const uint8_t *)(smem + P_OFF + li * PROW + lg * 16)));
#pragma unroll
        for (int j = 0; j < NO; ++j) {
          const uint32_t off = static_cast<uint32_t>((((NTW * wave + NTW + j) % NH) * 16) * PROW);  // wave-uniform
          asm volatile("ds_read_b128 %0, %1" : "=v"(pb[j]) : "v"(paddr + off));
        }
      }
      // wait for block j's read: NO - 1 - j reads were issued after it
#define AMLA_WPB(J, N) asm volatile("s_waitcnt lgkmcnt(" #N ")" : "+v"(pb[J])::"memory")
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        switch (NO - 1 - j) {
          case 5: AMLA_WPB(j, 5); break;
          case 4: AMLA_WPB(j, 4); break;
          case 3: AMLA_WPB(j, 3); break;
          case 2: AMLA_WPB(j, 2); break;
          case 1: AMLA_WPB(j, 1); break;
          default: AMLA_WPB(j, 0); break;
        }
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) {  // accumulators pinned to AGPRs (only these MFMAs touch them in the loop)
          const bf16x8 a = as_bf16x8(u32x4{ta[mt].x, ta[mt].y, tb[mt].x, tb[mt].y});
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(o[mt][NTW + j]) : "v"(a), "v"(pb[j]));
        }
      }
#undef AMLA_WPB
      __builtin_amdgcn_sched_barrier(0);

      // barrier without a memory fence: a fence would also wait for the copy
      // of the tile after next; LDS writes (rotated keys) are drained by hand
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    tile_body(tb, BoolC<true>{});
    if (tb + 1 < te) {
      // the second tile's copies landed (the third tile's pieces issued after
      // its last one may still be in flight); prepared here, then the steady loop
      wait_vmcnt<QKD / 32 - TILE_DMA + 1>();
      prepare_own_rows(smem + STAGE_BYTES, smem + TAB_OFF + ((tb + 1) & 1) * TAB_BYTES, wave, lane, p.eps);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    for (int tile = tb + 1; tile < te; ++tile) tile_body(tile, BoolC<false>{});
  }

  // the accumulators' last MFMA writes are read by VALU code below: cover the
  // MFMA write-to-read wait states the compiler does not see for inline asm
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  // ---- partial results of this split: (m, l) of the wave's heads, O of its
  // latent columns for every head of the group
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) {
    float l = l_run[nt];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int head = head0 + nt * 16 + li;
    const size_t row = (size_t)slot * HEADS + head;
    // a sum at or above 2^64 (or inf / NaN) means a score rose far above the
    // reference max: the combine recomputes this (split, head) exactly
    const bool bad = !(l < REF_HEADROOM_SUM);
    if (lg == 0) {
      p.part_ml[row * 2] = m_ref[nt];
      p.part_ml[row * 2 + 1] = bad ? -1.f : l;
    }
  }
  // O goes out through LDS, over the stages and table blocks: the copies the
  // last iterations issued (into stages nothing reads) must have landed in
  // every wave before any wave writes there; then head rows of 512 bf16, and
  // 1 KB contiguous per wave-wide store
  wait_vmcnt<0>();
  __syncthreads();
#pragma unroll
  for (int nt = 0; nt < NH; ++nt)
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
      *reinterpret_cast<u32x2 *>(smem + ((((NTW * wave + nt) % NH) * 16) + li) * OROW +
                                 (wave * 128 + mt * 16 + 4 * lg) * 2) =
          u32x2{pack_bf16(o[mt][nt].x, o[mt][nt].y), pack_bf16(o[mt][nt].z, o[mt][nt].w)};
  __syncthreads();
  uint8_t *const dst = reinterpret_cast<uint8_t *>(p.part_o + ((size_t)slot * HEADS + blockIdx.y * HG) * LORA);
#pragma unroll 8
  for (int i = 0; i < HG * LORA * 2 / (256 * 16); ++i) {
    const int chunk = i * 256 + tid, head = chunk >> 6, c16 = chunk & 63;
    *reinterpret_cast<u32x4 *>(dst + (size_t)chunk * 16) = *reinterpret_cast<const u32x4 *>(smem + head * OROW + c16 * 16);
  }
}

constexpr size_t ATTN_LDS = ATTN_LDS_BYTES;

// ---------------------------------------------------------------- combine + W_UV

AMLA_DEV float block_reduce(float v, float *red, bool is_max) {
  // 512 threads (8 waves), in wave order
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = is_max ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < 8; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

// Exact online-softmax recomputation of one (split, head) in fp32, used only
// for heads attn_kernel flagged (a sum of p = 2^(s - m_ref) at or above 2^64:
// scores far above the split's reference max).  Thread tid < 256 owns latent
// columns 2*tid and 2*tid+1 and one row of each 256-row block; the other
// threads of the 512 take part in the reductions only.
AMLA_DEV void recompute_split(const AttnParams &p, int b, int h, const SeqSplits &sp, int split, float *qs,
                              float *ps, float *red, float &m_out, float &l_out, float &o0, float &o1) {
  const int tid = threadIdx.x;
  const bool act = tid < 256;
  const int T = min(p.pos[b] + 1, p.tmax);
  const int t0 = split_tile(sp.ntiles, sp.count, split) * TT;
  const int t1 = min(split_tile(sp.ntiles, sp.count, split + 1) * TT, T);
  __syncthreads();
  for (int c = tid; c < QKD; c += 512) qs[c] = bf2f(p.qbuf[qfrag_index(b, h, c)]);
  __syncthreads();
  const uint16_t *cb = p.ckv + (size_t)b * p.ckv_bstride;
  const uint16_t *kb = p.kpe + (size_t)b * p.kpe_bstride;
  float M = -INFINITY, L = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c0 = t0; c0 < t1; c0 += 256) {
    const int t = c0 + tid;
    float sv = -INFINITY, rt = 0.f;
    if (act && t < t1) {
      const uint16_t *row = cb + (size_t)t * LORA;
      float ss = 0.f, dl = 0.f;
      for (int c = 0; c < LORA; ++c) {
        const float x = bf2f(row[c]);
        ss += x * x;
        dl += x * qs[c];
      }
      float dp = 0.f;
      for (int i = 0; i < ROPE / 2; ++i) {
        const uint32_t kv = *reinterpret_cast<const uint32_t *>(kb + (size_t)t * ROPE + 2 * i);
        const float cs = p.rope_table[((size_t)t * (ROPE / 2) + i) * 2];
        const float sn = p.rope_table[((size_t)t * (ROPE / 2) + i) * 2 + 1];
        const uint32_t rk = rot_pair(kv, cs, sn);
        dp += lo_bf(rk) * qs[LORA + 2 * i] + hi_bf(rk) * qs[LORA + 2 * i + 1];
      }
      rt = __builtin_amdgcn_rsqf(ss * (1.f / LORA) + p.eps);
      sv = p.scale_log2 * (rt * dl + dp);
    }
    const float mc = block_reduce(sv, red, true);
    const float Mn = fmaxf(M, mc);
    const float f = (M == -INFINITY) ? 0.f : exp2f(M - Mn);
    const float pe = (sv == -INFINITY) ? 0.f : exp2f(sv - Mn);
    if (act) ps[tid] = pe * rt;
    const float ls = block_reduce(pe, red, false);
    L = L * f + ls;
    a0 *= f;
    a1 *= f;
    M = Mn;
    const int n = min(256, t1 - c0);
    if (act) {
      for (int j = 0; j < n; ++j) {
        const float w = ps[j];
        const uint32_t pr = reinterpret_cast<const uint32_t *>(cb + (size_t)(c0 + j) * LORA)[tid];  // columns 2tid, 2tid+1
        a0 += w * lo_bf(pr);
        a1 += w * hi_bf(pr);
      }
    }
    __syncthreads();
  }
  m_out = M;
  l_out = L;
  o0 = a0;
  o1 = a1;
}

// Grid (VH H, ceil(B / SQ)), 512 threads: workgroup (VH h + i, g) finishes
// sequences SQ g .. SQ g + SQ - 1 of head h, output rows 128 i / VH .. of
// 128 / VH, so W_UV[h] is read once per SQ sequences (SQ = 4 up to batch 8,
// else 16: the MFMA's 16 columns; VH = 2 for one sequence group, where two
// workgroups per head halve each one's weight stream and both merge).
//   merge units (sequence, part of its splits), WPS parts per sequence (2 up
//     to batch 8, else 1), go to the 8 waves in turn (lane: latent columns
//     8l .. 8l+7, one 16-byte load per split, up to XB splits in flight);
//     every part takes the max over all the sequence's splits and sums its
//     own with exp2(m_s - M); the parts' sums meet in LDS in part order;
//   a sequence with a flagged split is merged by the whole workgroup with
//     exact recomputation of the flagged splits (rare);
//   lat = O / l times kv_a_layernorm gamma and W_UV's block scale, as bf16;
//   out[b][v] = W_UV[h][v] . lat[b] by 16x16x32 MFMAs: A = W_UV rows (fp8
//     converted exactly), B = lat of the SQ sequences (columns past them
//     zero); wave w produces rows v = 16w .. 16w+15.
template <int SQ, int WPS, int VH>
__global__ __launch_bounds__(512) void combine_uv_kernel(AttnParams ap, const uint8_t *__restrict__ wkvb,
                                                         const float *__restrict__ skvb,
                                                         const uint16_t *__restrict__ gamma, int B,
                                                         uint16_t *__restrict__ attn) {
  constexpr int NU = SQ * WPS;    // merge units
  constexpr int XB = SQ > 4 ? 8 : 20;  // splits in flight per wave (a batch)
  constexpr int WMAX = 256;       // splits per sequence
  constexpr int MLR = WMAX / 64;  // (m, l) loads per lane
  constexpr int LROW = LORA + 8;  // bf16 per lat row in LDS (16 B pad)
  static_assert(SQ <= 16 && NU <= 16, "one MFMA column per sequence; at most two units per wave");
  static_assert(VH == 1 || VH == 2, "whole or half W_UV[h] per workgroup");
  constexpr int VW = 8 / VH;  // waves with W_UV rows
  const int h = blockIdx.x / VH, b0 = blockIdx.y * SQ;
  const int vbase = (blockIdx.x % VH) * (VD / VH);  // first output row of this workgroup
  const int nb = min(SQ, B - b0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ __align__(16) uint16_t latb[SQ][LROW];
  __shared__ float wsp[8][WMAX + XB];  // weight of split s, zero past the last split
  __shared__ float xacc[NU][8][64];  // each unit's sums, [column e][lane]
  __shared__ float xl[NU];
  __shared__ float qs[QKD];
  __shared__ float ps[256];
  __shared__ float red[8];
  __shared__ int s_flag[SQ];
  float bsc[4];  // W_UV block scales of the four 128-column blocks
#pragma unroll
  for (int q = 0; q < 4; ++q) bsc[q] = skvb[(size_t)(2 * h + 1) * (LORA / 128) + q];

  // W_UV rows of this wave (rows v = vbase + 16w .. +15, 8 bytes per lane and
  // K step; waves w < VW) are loaded first: nothing they feed depends on the
  // merge
  const int li = lane & 15, lg = lane >> 4;
  const bool vwave = wave < VW;
  const uint8_t *wr = wkvb + ((size_t)h * (NOPE + VD) + NOPE + vbase + 16 * (wave % VW) + li) * LORA + 8 * lg;
  u32x2 wa[LORA / 32];
  // non-temporal when this is the only workgroup reading these weight rows
  if (vwave) {
    if (gridDim.y == 1) {
#pragma unroll
      for (int ks = 0; ks < LORA / 32; ++ks) wa[ks] = ldg8_nt(wr + ks * 32);
    } else {
#pragma unroll
      for (int ks = 0; ks < LORA / 32; ++ks) wa[ks] = ldg8(wr + ks * 32);
    }
  }

  // ---- fast merge: unit u = (sequence b0 + u / WPS, part u % WPS).  A
  // unit's first batch of partial rows and every split's (m, l) are loaded
  // together (lane l: splits l, l + 64, ..); the max and the weights are
  // formed from those registers while the rows are in flight.
  for (int u = wave; u < NU; u += 8) {
    const int su = u / WPS, pu = u % WPS;
    if (su >= nb) {
      if (pu == 0 && lane == 0) s_flag[su] = 0;
      continue;
    }
    const SeqSplits sp = seq_splits(ap, b0 + su);
    const size_t base = (size_t)sp.first * HEADS + h;
    const u32x4 *po = reinterpret_cast<const u32x4 *>(ap.part_o + base * LORA) + lane;
    const size_t stride = (size_t)HEADS * LORA / 8;
    const int nsp = sp.count;
    const int chunk = (nsp + WPS - 1) / WPS;
    const int s0 = min(pu * chunk, nsp), s1 = min(s0 + chunk, nsp);  // this unit's splits [s0, s1)
    u32x4 v[XB];
#pragma unroll
    for (int j = 0; j < XB; ++j) v[j] = po[(size_t)min(s0 + j, nsp - 1) * stride];
    float2 ml[MLR];
#pragma unroll
    for (int r = 0; r < MLR; ++r) {
      ml[r] = float2{-INFINITY, 0.f};
      if (64 * r < nsp) {
        const int s = min(lane + 64 * r, nsp - 1);
        const float2 e = *reinterpret_cast<const float2 *>(ap.part_ml + (base + (size_t)s * HEADS) * 2);
        if (lane + 64 * r < nsp) ml[r] = e;
      }
    }
    float mloc = -INFINITY;
    bool badl = false;
#pragma unroll
    for (int r = 0; r < MLR; ++r) {
      mloc = fmaxf(mloc, ml[r].x);
      badl = badl || ml[r].y < 0.f;
    }
    const float M = wave_max(mloc);
    const bool flagged = __builtin_amdgcn_ballot_w64(badl) != 0;
    if (pu == 0 && lane == 0) s_flag[su] = flagged;
    if (flagged) continue;
    // weights of this unit's splits (by split index), zero past its last
    // split up to a whole batch
    float lloc = 0.f;
#pragma unroll
    for (int r = 0; r < MLR; ++r) {
      const int s = lane + 64 * r;
      if (64 * r < s0 + ((s1 - s0 + XB - 1) / XB) * XB) {
        float w = 0.f;
        if (s >= s0 && s < s1 && ml[r].x != -INFINITY) {
          w = exp2f(ml[r].x - M);
          lloc += w * ml[r].y;
        }
        wsp[wave][s] = w;
      }
    }
    if (lane < XB) wsp[wave][WMAX + lane] = 0.f;
    const float L = wave_sum(lloc);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < s1 - s0; k += XB) {
#pragma unroll
      for (int j = 0; j < XB; ++j) {
        const float w = wsp[wave][s0 + k + j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += w * lo_bf(v[j][e]);
          acc[2 * e + 1] += w * hi_bf(v[j][e]);
        }
      }
      if (k + XB < s1 - s0) {
#pragma unroll
        for (int j = 0; j < XB; ++j) v[j] = po[(size_t)min(s0 + k + XB + j, nsp - 1) * stride];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) xacc[u][e][lane] = acc[e];
    if (lane == 0) xl[u] = L;
  }
  __syncthreads();
  for (int sq = wave; sq < nb; sq += 8) {
    if (s_flag[sq]) continue;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = xacc[sq * WPS][e][lane];
    float L = xl[sq * WPS];
#pragma unroll
    for (int pu = 1; pu < WPS; ++pu) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += xacc[sq * WPS + pu][e][lane];
      L += xl[sq * WPS + pu];
    }
    const float inv = 1.f / L;
    const float sc = bsc[(8 * lane) / 128];
    const u32x4 gm = *reinterpret_cast<const u32x4 *>(gamma + 8 * lane);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16(acc[2 * e] * inv * lo_bf(gm[e]) * sc, acc[2 * e + 1] * inv * hi_bf(gm[e]) * sc);
    *reinterpret_cast<u32x4 *>(&latb[sq][8 * lane]) = o;
  }
  __syncthreads();

  // ---- rare path: sequences with a flagged split, merged by the whole
  // workgroup (thread tid < 256: latent columns 2 tid, 2 tid + 1)
  for (int bb = 0; bb < nb; ++bb) {
    if (!s_flag[bb]) continue;
    const int b = b0 + bb;
    const SeqSplits sp = seq_splits(ap, b);
    const size_t base = (size_t)sp.first * HEADS + h;
    float M = -INFINITY, Ls = 0.f, a0 = 0.f, a1 = 0.f;
    for (int s = 0; s < sp.count; ++s) {
      const size_t row = base + (size_t)s * HEADS;
      float m1 = ap.part_ml[row * 2], l1 = ap.part_ml[row * 2 + 1], o0 = 0.f, o1 = 0.f;
      if (l1 < 0.f) {
        recompute_split(ap, b, h, sp, s, qs, ps, red, m1, l1, o0, o1);
      } else if (tid < 256) {
        const uint32_t v = reinterpret_cast<const uint32_t *>(ap.part_o + row * LORA)[tid];
        o0 = lo_bf(v);
        o1 = hi_bf(v);
      }
      if (m1 == -INFINITY) continue;  // split past this sequence's context
      const float Mn = fmaxf(M, m1);
      const float fo = (M == -INFINITY) ? 0.f : exp2f(M - Mn);
      const float fn = exp2f(m1 - Mn);
      a0 = a0 * fo + o0 * fn;
      a1 = a1 * fo + o1 * fn;
      Ls = Ls * fo + l1 * fn;
      M = Mn;
    }
    if (tid < 256) {
      const float inv = 1.f / Ls;
      const float sc = bsc[(2 * tid) / 128];
      const uint32_t gm = reinterpret_cast<const uint32_t *>(gamma)[tid];
      reinterpret_cast<uint32_t *>(&latb[bb][0])[tid] = pack_bf16(a0 * inv * lo_bf(gm) * sc, a1 * inv * hi_bf(gm) * sc);
    }
    __syncthreads();
  }

  // ---- out = W_UV[h] . lat: wave w < VW, rows vbase + 16w .. +15, 16 K steps of 32
  if (!vwave) return;
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  const bool bvalid = li < nb;
  const uint16_t *lr = &latb[bvalid ? li : 0][8 * lg];
#pragma unroll
  for (int ks = 0; ks < LORA / 32; ++ks) {
    const u32x4 bl = bvalid ? *reinterpret_cast<const u32x4 *>(lr + ks * 32) : u32x4{0, 0, 0, 0};
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[ks].x, 1.f, false);
    const bf16x2_t c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[ks].x, 1.f, true);
    const bf16x2_t c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[ks].y, 1.f, false);
    const bf16x2_t c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[ks].y, 1.f, true);
    const bf16x8 a = {c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
    c = mfma16(a, as_bf16x8(bl), c);
  }
  // C: lane holds sequence b0 + li, rows v = 16w + 4 lg .. +3
  if (bvalid) {
    uint16_t *dst = attn + (size_t)(b0 + li) * HEADS * VD + h * VD + vbase + 16 * wave + 4 * lg;
    *reinterpret_cast<u32x2 *>(dst) = u32x2{pack_bf16(c.x, c.y), pack_bf16(c.z, c.w)};
  }
}

// ---------------------------------------------------------------- orchestration

struct DecodeLayout {
  size_t plan, xn, qa, q, qbuf, part_ml, part_o, attn, lin, total;
  GemvPlan pa, pb, po;
  int units, slots;  // split budget (build_split_plan) and partial slots
};

// Sequences per decode launch sequence: a larger batch runs in chunks of this
// many, one after another on the stream, sharing one workspace.
constexpr int DECODE_MAX_BATCH = 64;

// Head groups of the attention launch: two (64 heads per workgroup) while the
// split slots fill at most half the CUs, so that a workgroup's fixed cost (the
// query fragments in, the partial O out, both in proportion to its heads)
// halves and twice the CUs share it; else one (all 128 heads).
static int attn_head_groups(const DecodeLayout &L) { return L.slots <= 128 ? 2 : 1; }

static DecodeLayout decode_layout(const amla_mla_args &a) {
  DecodeLayout L = {};
  const int B = std::min(a.batch, DECODE_MAX_BATCH);
  const int HD = a.qk_nope + a.qk_rope;
  L.pa = plan_linear(B, a.q_lora + a.kv_lora + a.qk_rope, a.hidden);
  L.pb = plan_linear(B, a.heads * HD, a.q_lora);
  L.po = plan_linear(B, a.hidden, a.heads * a.v_dim);
  // splits over the batch: one per CU, at least two tiles each for the
  // longest possible context, or one tile each while the batch holds at most
  // 64 tiles (a split's fixed cost then outweighs its second tile); the plan
  // itself is made on the device from the positions (build_split_plan)
  const int maxT = mla_context_bound(a);
  const int ntiles = (maxT + TT - 1) / TT;
  const int bt = B * ntiles;
  L.units = std::max(1, std::min(256, bt <= 64 ? bt : B * std::max(1, ntiles / 2)));
  L.slots = L.units + B;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes, 256); return o; };
  L.plan = take(plan_ints(B, L.slots) * 4);  // first: a test reads the table back
  L.xn = take((size_t)B * a.hidden * 2);
  L.qa = take((size_t)B * a.q_lora * 2);
  L.q = take((size_t)B * a.heads * HD * 2);
  L.qbuf = take((size_t)B * a.heads * QKD * 2);
  L.part_ml = take((size_t)L.slots * a.heads * 2 * 4);
  L.part_o = take((size_t)L.slots * a.heads * LORA * 2);
  L.attn = take((size_t)B * a.heads * a.v_dim * 2);
  L.lin = take(std::max(L.pa.part_bytes, std::max(L.pb.part_bytes, L.po.part_bytes)));  // K-part sums of the linears
  L.total = off;
  return L;
}

int check_mla_common(const amla_mla_args *a, const char *who) {
  if (!a) return fail(AMLA_EINVAL, "%s: null args", who);
  if (a->heads != HEADS || a->kv_lora != LORA || a->qk_rope != ROPE || a->qk_nope != NOPE || a->v_dim != VD)
    return fail(AMLA_EUNSUPPORTED,
                "%s: kernels are built for heads=128 kv_lora=512 rope=64 nope=128 v=128 (got %d/%d/%d/%d/%d)",
                who, a->heads, a->kv_lora, a->qk_rope, a->qk_nope, a->v_dim);
  if (a->hidden <= 0 || a->hidden % 128 || a->q_lora <= 0 || a->q_lora % 128)
    return fail(AMLA_EUNSUPPORTED, "%s: hidden and q_lora must be positive multiples of 128", who);
  if (a->batch <= 0 || a->seq_len <= 0) return fail(AMLA_EINVAL, "%s: batch and seq_len must be >= 1", who);
  if (a->max_seq <= 0 || a->rope_rows <= 0) return fail(AMLA_EINVAL, "%s: max_seq / rope_rows must be >= 1", who);
  if (a->max_context < 0) return fail(AMLA_EINVAL, "%s: max_context must be >= 0 (0: max_seq)", who);
  const int bound = mla_context_bound(*a);
  if (bound > a->max_seq || bound > a->rope_rows)
    return fail(AMLA_EINVAL, "%s: context bound %d exceeds the cache (%d rows) or the rope table (%d rows)", who,
                bound, a->max_seq, a->rope_rows);
  if (bound < a->seq_len)
    return fail(AMLA_EINVAL, "%s: context bound %d is below seq_len %d", who, bound, a->seq_len);
  const void *ptrs[] = {a->positions, a->hidden_states, a->out, a->w_q_a, a->s_q_a, a->w_q_b, a->s_q_b,
                        a->w_kv_a, a->s_kv_a, a->w_kv_b, a->s_kv_b, a->w_o, a->s_o, a->gamma_q,
                        a->gamma_kv, a->ckv_cache, a->kpe_cache, a->rope_table, a->workspace};
  for (const void *q : ptrs)
    if (!q) return fail(AMLA_EINVAL, "%s: a required pointer is null", who);
  if (!aligned16(a->hidden_states) || !aligned16(a->ckv_cache) || !aligned16(a->kpe_cache) ||
      !aligned16(a->rope_table) || !aligned16(a->out) || !aligned16(a->workspace) || !aligned16(a->attn_out))
    return fail(AMLA_EINVAL, "%s: activations, caches, rope table and workspace must be 16-byte aligned", who);
  return AMLA_OK;
}

// Optional stage events (bench instrumentation): ev[i] is recorded before
// stage i and ev[NSTAGE] after the last one.
constexpr int NSTAGE = 7;  // qkva, q_a norm, q_b, absorb, attention, combine, o_proj

static inline void mark(hipEvent_t const *ev, int i, hipStream_t st) {
  if (ev) (void)hipEventRecord(ev[i], st);
}

static int decode_chunk(const amla_mla_args *a, hipStream_t st, hipEvent_t const *ev, int attn_repeat);

static int decode_impl(const amla_mla_args *a, hipStream_t st, hipEvent_t const *ev = nullptr, int attn_repeat = 1) {
  int rc = check_mla_common(a, "mla_decode");
  if (rc) return rc;
  if (a->seq_len != 1) return fail(AMLA_EINVAL, "mla_decode: seq_len must be 1 (use mla_prefill)");
  if (a->batch <= DECODE_MAX_BATCH) return decode_chunk(a, st, ev, attn_repeat);
  // inference/ops.py:119 takes any batch: chunks of DECODE_MAX_BATCH sequences
  // in order on the stream (each chunk's launches finish before the next
  // chunk's reuse the workspace)
  for (int b0 = 0; b0 < a->batch; b0 += DECODE_MAX_BATCH) {
    amla_mla_args c = *a;
    c.batch = std::min(DECODE_MAX_BATCH, a->batch - b0);
    const size_t row = (size_t)a->hidden * 2;
    c.positions = a->positions + b0;
    c.hidden_states = static_cast<const char *>(a->hidden_states) + (size_t)b0 * row;
    c.out = static_cast<char *>(a->out) + (size_t)b0 * row;
    if (a->residual) c.residual = static_cast<const char *>(a->residual) + (size_t)b0 * row;
    if (a->attn_out) c.attn_out = static_cast<char *>(a->attn_out) + (size_t)b0 * a->heads * a->v_dim * 2;
    c.ckv_cache = static_cast<char *>(a->ckv_cache) + (size_t)b0 * a->max_seq * a->kv_lora * 2;
    c.kpe_cache = static_cast<char *>(a->kpe_cache) + (size_t)b0 * a->max_seq * a->qk_rope * 2;
    if ((rc = decode_chunk(&c, st, ev, attn_repeat))) return rc;
  }
  return AMLA_OK;
}

// One launch sequence for at most DECODE_MAX_BATCH sequences (args checked).
// attn_repeat > 1 (measurement only) launches the attention kernel that many
// times back to back: it reads the same inputs and rewrites the same partials.
static int decode_chunk(const amla_mla_args *a, hipStream_t st, hipEvent_t const *ev, int attn_repeat) {
  int rc = AMLA_OK;
  const DecodeLayout L = decode_layout(*a);
  if (a->workspace_bytes < L.total)
    return fail(AMLA_EWORKSPACE, "mla_decode: workspace %zu bytes < %zu needed", a->workspace_bytes, L.total);
  char *ws = reinterpret_cast<char *>(a->workspace);
  const int B = a->batch;
  const int HD = a->qk_nope + a->qk_rope;

  const uint16_t *x = reinterpret_cast<const uint16_t *>(a->hidden_states);
  uint16_t *qa = reinterpret_cast<uint16_t *>(ws + L.qa);
  uint16_t *q = reinterpret_cast<uint16_t *>(ws + L.q);
  uint16_t *qbuf = reinterpret_cast<uint16_t *>(ws + L.qbuf);

  // 1. [input RMSNorm, layer mode] q_a | kv_a  (kv_a written raw into the
  //    caches, inference/ops.py:136-141; forward.py:92).  The streaming GEMV
  //    (batch 1) normalises its x row itself, exactly as rms_norm; with K
  //    parts the norm is folded: the GEMM reads bf16(x * input_gamma) and the
  //    K-part finish multiplies each sum by the row's rsqrt(mean(x^2) + eps)
  //    (one bf16 rounding fewer than the reference's); otherwise it is its
  //    own launch first.
  mark(ev, 0, st);
  const uint16_t *xin = x;
  const uint16_t *gin = reinterpret_cast<const uint16_t *>(a->input_gamma);
  const bool fold_norm = gin && (L.pa.kparts > 1 || L.pa.vec) && a->hidden <= 8192;
  if (gin && !fold_norm) {
    uint16_t *xn = reinterpret_cast<uint16_t *>(ws + L.xn);
    if ((rc = launch_rms_norm(x, B, a->hidden, a->hidden, gin, a->eps, xn, a->hidden, st))) return rc;
    xin = xn;
  }
  GemvParams pa = {};
  pa.x = xin; pa.M = B; pa.ldx = a->hidden;
  pa.xg = fold_norm ? gin : nullptr;
  pa.xnorm = fold_norm && L.pa.vec;
  pa.eps_in = a->eps;
  pa.w0 = reinterpret_cast<const uint8_t *>(a->w_q_a); pa.s0 = a->s_q_a;
  pa.w1 = reinterpret_cast<const uint8_t *>(a->w_kv_a); pa.s1 = a->s_kv_a;
  pa.N = a->q_lora + LORA + ROPE; pa.K = a->hidden; pa.n_split = a->q_lora;
  pa.y = qa; pa.ldy = a->q_lora;
  pa.ckv = reinterpret_cast<uint16_t *>(a->ckv_cache);
  pa.kpe = reinterpret_cast<uint16_t *>(a->kpe_cache);
  pa.ckv_bstride = (int64_t)a->max_seq * LORA; pa.kpe_bstride = (int64_t)a->max_seq * ROPE;
  pa.kv_lora = LORA; pa.rope = ROPE; pa.pos = a->positions; pa.seq_len = 1; pa.max_rows = a->max_seq;
  pa.part = reinterpret_cast<float *>(ws + L.lin);
  if ((rc = launch_gemv(pa, GEMV_QKVA, L.pa, st, false))) return rc;  // K parts are summed below
  // 2. q_a_layernorm (inference/ops.py:130): fused into the K-part finish;
  //    done by q_b's streaming GEMV on its x row (batch 1); else a row norm
  //    in place
  mark(ev, 1, st);
  const uint16_t *gq = reinterpret_cast<const uint16_t *>(a->gamma_q);
  const bool fold_qnorm = L.pa.kparts == 1 && L.pb.vec;
  if (L.pa.kparts > 1) {
    if ((rc = launch_qkva_finish_norm(pa, L.pa.kparts, gq, a->eps, st, fold_norm ? x : nullptr, a->eps))) return rc;
  } else if (!fold_qnorm && (rc = launch_rms_norm(qa, B, a->q_lora, a->q_lora, gq, a->eps, qa, a->q_lora, st))) {
    return rc;
  }

  // 3. q = q_a_norm W_qb^T, RoPE on q_pe at pos[b] (inference/ops.py:131-133, :156)
  mark(ev, 2, st);
  GemvParams pb = {};
  pb.x = qa; pb.M = B; pb.ldx = a->q_lora;
  pb.xg = fold_qnorm ? gq : nullptr;
  pb.xnorm = fold_qnorm;
  pb.eps_in = a->eps;
  pb.w0 = reinterpret_cast<const uint8_t *>(a->w_q_b); pb.s0 = a->s_q_b;
  pb.N = a->heads * HD; pb.K = a->q_lora; pb.n_split = pb.N;
  pb.y = q; pb.ldy = pb.N;
  pb.pos = a->positions; pb.seq_len = 1; pb.rope = ROPE; pb.rope_table = a->rope_table; pb.rope_rows = a->rope_rows;
  pb.head_dim = HD; pb.nope = a->qk_nope;
  pb.part = reinterpret_cast<float *>(ws + L.lin);
  if ((rc = launch_gemv(pb, GEMV_QROPE, L.pb, st))) return rc;

  // 4. absorb W_UK into the query
  mark(ev, 3, st);
  int32_t *plan = reinterpret_cast<int32_t *>(ws + L.plan);
  const int tmax = mla_context_bound(*a);
  if (B <= AB_SEQ)
    absorb_kernel<1><<<dim3(HEADS + 1, LORA / 128, 1), 256, 0, st>>>(
        q, reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b, reinterpret_cast<const uint16_t *>(a->gamma_kv), B,
        qbuf, a->positions, tmax, L.units, L.slots, plan);
  else
    absorb_kernel<2><<<dim3(HEADS + 1, LORA / 128, (B + 2 * AB_SEQ - 1) / (2 * AB_SEQ)), 256, 0, st>>>(
        q, reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b, reinterpret_cast<const uint16_t *>(a->gamma_kv), B,
        qbuf, a->positions, tmax, L.units, L.slots, plan);
  if ((rc = check_launch("mla absorb"))) return rc;

  // 5. attention over the latent cache, split over context
  mark(ev, 4, st);
  AttnParams ap = {};
  ap.qbuf = qbuf;
  ap.ckv = reinterpret_cast<const uint16_t *>(a->ckv_cache);
  ap.kpe = reinterpret_cast<const uint16_t *>(a->kpe_cache);
  ap.ckv_bstride = (int64_t)a->max_seq * LORA; ap.kpe_bstride = (int64_t)a->max_seq * ROPE;
  ap.rope_table = a->rope_table; ap.pos = a->positions; ap.tmax = tmax;
  ap.units = L.units; ap.batch = B; ap.plan = plan;
  ap.scale_log2 = a->softmax_scale * 1.4426950408889634f;
  ap.eps = a->eps;
  ap.part_o = reinterpret_cast<uint16_t *>(ws + L.part_o);
  ap.part_ml = reinterpret_cast<float *>(ws + L.part_ml);
  for (int r = 0; r < attn_repeat; ++r) {
    if (attn_head_groups(L) == 2)
      attn_kernel<1><<<dim3(L.slots, 2), 256, ATTN_LDS, st>>>(ap);
    else
      attn_kernel<2><<<dim3(L.slots), 256, ATTN_LDS, st>>>(ap);
    if ((rc = check_launch("mla attention"))) return rc;
  }

  // 6. merge splits, W_UV
  mark(ev, 5, st);
  uint16_t *attn = reinterpret_cast<uint16_t *>(a->attn_out ? a->attn_out : ws + L.attn);
  if (B <= 2)  // one sequence group: W_UV[h] split over two workgroups
    combine_uv_kernel<4, 2, 2><<<dim3(2 * HEADS, 1), 512, 0, st>>>(
        ap, reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b, reinterpret_cast<const uint16_t *>(a->gamma_kv), B,
        attn);
  else if (B <= 8)
    combine_uv_kernel<4, 2, 1><<<dim3(HEADS, (B + 3) / 4), 512, 0, st>>>(
        ap, reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b, reinterpret_cast<const uint16_t *>(a->gamma_kv), B,
        attn);
  else
    combine_uv_kernel<16, 1, 1><<<dim3(HEADS, (B + 15) / 16), 512, 0, st>>>(
        ap, reinterpret_cast<const uint8_t *>(a->w_kv_b), a->s_kv_b, reinterpret_cast<const uint16_t *>(a->gamma_kv), B,
        attn);
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
  po.part = reinterpret_cast<float *>(ws + L.lin);
  rc = launch_gemv(po, a->residual ? GEMV_RESID : GEMV_PLAIN, L.po, st);
  mark(ev, NSTAGE, st);
  return rc;
}

static bool g_attr_set = false;

static void set_attn_attr() {
  if (!g_attr_set) {
    // Opt in to more than 64 KB of dynamic LDS (gfx950 has 160 KB per CU).
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_kernel<1>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)ATTN_LDS);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_kernel<2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)ATTN_LDS);
    (void)hipGetLastError();
    g_attr_set = true;
  }
}

// ---------------------------------------------------------------- no-allocation decode

// Scratch of amla_mla_decode_noalloc: one array per device (each GPU the
// library runs on holds its own copy, at its own address, until the process
// ends).  In host code `scratch` names a host-side stand-in, never the
// device memory: the device address comes from hipGetSymbolAddress, per
// device, and only that address is passed to kernels.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)AMLA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static void *g_scratch_ptr[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch array (looked up once per
// device, with that device current); nullptr and a message on failure.
static void *noalloc_scratch(int *rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = fail((int)e, "mla_decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    *rc = fail(AMLA_EUNSUPPORTED, "mla_decode_noalloc: device %d beyond %d", dev, NOALLOC_MAX_DEVICES);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *rc = fail(e != hipSuccess ? (int)e : AMLA_EINVAL, "mla_decode_noalloc: hipGetSymbolAddress failed: %s",
                 hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *rc = AMLA_OK;
  return g_scratch_ptr[dev];
}

}  // namespace amla

using namespace amla;

extern "C" {

size_t amla_mla_decode_workspace_bytes(const amla_mla_args *a) {
  if (!a || a->batch <= 0) return 0;
  return decode_layout(*a).total;
}

int amla_mla_decode(const amla_mla_args *a, void *stream) {
  set_attn_attr();
  return decode_impl(a, reinterpret_cast<hipStream_t>(stream));
}

int amla_mla_decode_noalloc(const amla_mla_args *a, void *stream) {
  if (!a) return fail(AMLA_EINVAL, "mla_decode_noalloc: null args");
  if (a->batch <= 0) return fail(AMLA_EINVAL, "mla_decode_noalloc: batch must be >= 1");
  const size_t need = decode_layout(*a).total;
  if (need > NOALLOC_SCRATCH_BYTES)
    return fail(AMLA_EWORKSPACE, "mla_decode_noalloc: needs %zu bytes of scratch, the static array holds %zu",
                need, NOALLOC_SCRATCH_BYTES);
  int rc = AMLA_OK;
  void *ptr = noalloc_scratch(&rc);
  if (!ptr) return rc;
  amla_mla_args b = *a;
  b.workspace = ptr;
  b.workspace_bytes = NOALLOC_SCRATCH_BYTES;
  set_attn_attr();
  return decode_impl(&b, reinterpret_cast<hipStream_t>(stream));
}

int amla_mla_decode_profiled_repeat(const amla_mla_args *a, void *stream, void *const *events, int attn_repeat) {
  if (!events) return fail(AMLA_EINVAL, "mla_decode_profiled: null events");
  for (int i = 0; i <= NSTAGE; ++i)
    if (!events[i]) return fail(AMLA_EINVAL, "mla_decode_profiled: null event %d", i);
  if (attn_repeat < 1 || attn_repeat > 64)
    return fail(AMLA_EINVAL, "mla_decode_profiled: attention repeat %d outside 1..64", attn_repeat);
  set_attn_attr();
  return decode_impl(a, reinterpret_cast<hipStream_t>(stream), reinterpret_cast<hipEvent_t const *>(events),
                     attn_repeat);
}

int amla_mla_decode_profiled(const amla_mla_args *a, void *stream, void *const *events) {
  return amla_mla_decode_profiled_repeat(a, stream, events, 1);
}

}  // extern "C"
