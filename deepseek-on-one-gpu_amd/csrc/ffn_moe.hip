// FFN / MoE entry points for gfx950, built on the block-FP8 linear kernels:
//
//   amla_silu_mul     <- F.silu(gate) * up inside swiglu, inference/ops.py:189-191
//   amla_swiglu       <- swiglu / dense_ffn / expert_ffn, inference/ops.py:186-206
//   amla_moe_route    <- route, inference/ops.py:209-257
//   amla_moe_experts  <- the routed-expert loop of moe_block, inference/forward.py:139-151
//   amla_moe_experts_dev <- the same loop with the slots grouped by expert on the
//                        device (the reference's host read of the indices,
//                        gpu_transfer.py:60, has no counterpart)
//   amla_moe_combine  <- the combine of moe_block, inference/forward.py:138-153
//
// swiglu runs gate and up as one skinny (M <= 64) or large fp8 GEMM over the
// two stacked weights, one elementwise pass for silu * up over the stacked
// rows, and the down projection; the rounding points are the reference's (bf16
// after every linear, after silu and after the product).  The routed experts
// of a MoE layer run as grouped skinny GEMMs (up to 32 experts per launch).
// Routing computes the fp32 logits with bf16 MFMAs (exact products, fp32
// sums), then one wave per token does the sigmoid, the group ranking and the
// top-k in fp32.
#include <math.h>

#include <algorithm>
#include <vector>

#include "amla_common.h"
#include "amla_internal.h"

namespace amla {

// ---------------------------------------------------------------- silu * up

AMLA_DEV float silu_bf16(float g) { return round_bf16(g / (1.f + expf(-g))); }

// h[i] = bf16( bf16(silu(g[i])) * u[i] ); eight elements per thread step.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ g, const uint16_t *__restrict__ u,
                                                       int64_t n8, int64_t n, uint16_t *__restrict__ h) {
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < n8; c += (int64_t)gridDim.x * blockDim.x) {
    const u32x4 gv = *reinterpret_cast<const u32x4 *>(g + c * 8);
    const u32x4 uv = *reinterpret_cast<const u32x4 *>(u + c * 8);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = pack_bf16(silu_bf16(lo_bf(gv[i])) * lo_bf(uv[i]), silu_bf16(hi_bf(gv[i])) * hi_bf(uv[i]));
    *reinterpret_cast<u32x4 *>(h + c * 8) = o;
  }
  // elements past the last full group of 8 (all of them when a pointer is not 16-byte aligned)
  for (int64_t t = n8 * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n;
       t += (int64_t)gridDim.x * blockDim.x)
    h[t] = f2bf(silu_bf16(bf2f(g[t])) * bf2f(u[t]));
}

// The K-part sums of [gate | up] (fp32, [part][m][2n]) added in part order
// and rounded to bf16 as gemv_finish stores them, then
// h[m, j] = bf16( bf16(silu(gate)) * up ): gemv_finish and silu_mul_rows_kernel
// in one pass.  Thread: 4 consecutive columns of one row.
__global__ __launch_bounds__(64) void gu_finish_silu_kernel(const float *__restrict__ part, int M, int n, int kparts,
                                                            uint16_t *__restrict__ h) {
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (i >= (int64_t)M * (n >> 2)) return;
  const int m = (int)(i / (n >> 2)), j = (int)(i % (n >> 2)) * 4;
  const size_t N = 2 * (size_t)n;
  f32x4 g[GEMV_MAX_PARTS], u[GEMV_MAX_PARTS];
#pragma unroll
  for (int q = 0; q < GEMV_MAX_PARTS; ++q)
    if (q < kparts) {
      const float *row = part + ((size_t)q * M + m) * N;
      g[q] = *reinterpret_cast<const f32x4 *>(row + j);
      u[q] = *reinterpret_cast<const f32x4 *>(row + n + j);
    }
  f32x4 gs = g[0], us = u[0];
#pragma unroll
  for (int q = 1; q < GEMV_MAX_PARTS; ++q)
    if (q < kparts) {
      gs += g[q];
      us += u[q];
    }
  u32x2 o = {pack_bf16(silu_bf16(round_bf16(gs.x)) * round_bf16(us.x), silu_bf16(round_bf16(gs.y)) * round_bf16(us.y)),
             pack_bf16(silu_bf16(round_bf16(gs.z)) * round_bf16(us.z), silu_bf16(round_bf16(gs.w)) * round_bf16(us.w))};
  *reinterpret_cast<u32x2 *>(h + (size_t)m * n + j) = o;
}

static int launch_silu_mul(const uint16_t *g, const uint16_t *u, int64_t n, uint16_t *h, hipStream_t st) {
  const int64_t n8 = (aligned16(g) && aligned16(u) && aligned16(h)) ? n / 8 : 0;
  const int64_t work = std::max<int64_t>(n8, n - n8 * 8);
  const int blocks = (int)std::min<int64_t>((work + 255) / 256, 4096);
  silu_mul_kernel<<<std::max(blocks, 1), 256, 0, st>>>(g, u, n8, n, h);
  return check_launch("silu_mul");
}

// h[r, j] = bf16( bf16(silu(gu[r, j])) * gu[r, n + j] ) for rows r of [gate | up]
// (drows: the row count in device memory, else rows)
__global__ __launch_bounds__(256) void silu_mul_rows_kernel(const uint16_t *__restrict__ gu, int rows, int n,
                                                            uint16_t *__restrict__ h,
                                                            const int32_t *__restrict__ drows = nullptr) {
  if (drows) rows = *drows;
  for (int r = blockIdx.y; r < rows; r += gridDim.y) {
    const uint16_t *g = gu + (size_t)r * 2 * n, *u = g + n;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < n / 8; c += gridDim.x * blockDim.x) {
      const u32x4 gv = *reinterpret_cast<const u32x4 *>(g + c * 8);
      const u32x4 uv = *reinterpret_cast<const u32x4 *>(u + c * 8);
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = pack_bf16(silu_bf16(lo_bf(gv[i])) * lo_bf(uv[i]), silu_bf16(hi_bf(gv[i])) * hi_bf(uv[i]));
      *reinterpret_cast<u32x4 *>(h + (size_t)r * n + c * 8) = o;
    }
  }
}

// ---------------------------------------------------------------- swiglu

// One fp8 linear (y = bf16(x W^T)), skinny or large-M path.
static int fp8_linear_into(const uint16_t *x, int m, int k, const uint8_t *w, const float *s, int n, uint16_t *y,
                           float *part, hipStream_t st) {
  GemvParams p = {};
  p.x = x;
  p.M = m;
  p.ldx = k;
  p.w0 = w;
  p.s0 = s;
  p.N = n;
  p.K = k;
  p.n_split = n;
  p.y = y;
  p.ldy = n;
  p.seq_len = 1;
  if (m > 64) return launch_gemm(p, GEMV_PLAIN, st);
  const GemvPlan pl = plan_linear(m, n, k);
  p.part = part;
  return launch_gemv(p, GEMV_PLAIN, pl, st);
}

struct SwigluLayout {
  size_t gu, h, part, total;
};

// [gate | up] rows (m, 2n), then h (m, n), then the K-part sums of the skinny path
static SwigluLayout swiglu_layout(int64_t m, int64_t k, int64_t n) {
  SwigluLayout L;
  size_t off = 0;
  L.gu = off;
  off = align_up(off + (size_t)m * 2 * n * 2, 256);
  L.h = off;
  off = align_up(off + (size_t)m * n * 2, 256);
  size_t part = 0;
  if (m <= 64 && m > 0)
    part = std::max(plan_linear((int)m, (int)(2 * n), (int)k).part_bytes, plan_linear((int)m, (int)k, (int)n).part_bytes);
  L.part = off;
  off = align_up(off + part, 256);
  L.total = off;
  return L;
}

}  // namespace amla

using namespace amla;

extern "C" {

int amla_silu_mul(const void *gate, const void *up, int64_t numel, void *out, void *stream) {
  if (!gate || !up || !out) return fail(AMLA_EINVAL, "silu_mul: null pointer");
  if (numel < 0) return fail(AMLA_EINVAL, "silu_mul: numel < 0");
  if (numel == 0) return AMLA_OK;
  return launch_silu_mul(static_cast<const uint16_t *>(gate), static_cast<const uint16_t *>(up), numel,
                         static_cast<uint16_t *>(out), reinterpret_cast<hipStream_t>(stream));
}

size_t amla_swiglu_workspace_bytes(int64_t m, int64_t k, int64_t n) {
  if (m <= 0 || k <= 0 || n <= 0) return 0;
  return swiglu_layout(m, k, n).total;
}

int amla_swiglu(const void *x, int64_t m, int64_t k, const void *gate_w, const float *gate_s, const void *up_w,
                const float *up_s, int64_t n, const void *down_w, const float *down_s, void *y, void *workspace,
                size_t workspace_bytes, void *stream) {
  if (!x || !gate_w || !gate_s || !up_w || !up_s || !down_w || !down_s || !y)
    return fail(AMLA_EINVAL, "swiglu: null pointer");
  if (m < 0 || k <= 0 || n <= 0) return fail(AMLA_EINVAL, "swiglu: bad shape m=%lld k=%lld n=%lld", (long long)m,
                                             (long long)k, (long long)n);
  if (m == 0) return AMLA_OK;
  if (k % 128 || n % 128 || !aligned16(x) || !aligned16(y) || !aligned16(gate_w) || !aligned16(up_w) ||
      !aligned16(down_w))
    return fail(AMLA_EUNSUPPORTED,
                "swiglu: needs hidden and intermediate sizes that are multiples of 128 and 16-byte aligned "
                "x, y and weights (k=%lld n=%lld)",
                (long long)k, (long long)n);
  if (m > INT32_MAX || k > INT32_MAX || n > INT32_MAX) return fail(AMLA_EUNSUPPORTED, "swiglu: sizes above 2^31");
  const SwigluLayout L = swiglu_layout(m, k, n);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
    return fail(AMLA_EWORKSPACE, "swiglu: needs %zu bytes of 16-byte aligned workspace (got %zu)", L.total,
                workspace ? workspace_bytes : (size_t)0);
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  uint16_t *gu = reinterpret_cast<uint16_t *>(ws + L.gu);
  uint16_t *h = reinterpret_cast<uint16_t *>(ws + L.h);
  float *part = reinterpret_cast<float *>(ws + L.part);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  // gate and up as one GEMM over the two stacked weights: rows (m, [gate | up])
  GemvParams p = {};
  p.x = static_cast<const uint16_t *>(x);
  p.M = (int)m;
  p.ldx = (int)k;
  p.w0 = static_cast<const uint8_t *>(gate_w);
  p.s0 = gate_s;
  p.w1 = static_cast<const uint8_t *>(up_w);
  p.s1 = up_s;
  p.N = (int)(2 * n);
  p.K = (int)k;
  p.n_split = (int)n;
  p.y = gu;
  p.ldy = (int)(2 * n);
  p.seq_len = 1;
  p.part = part;
  if (m > 64 && n % 256 == 0) rc = launch_gemm(p, GEMV_PLAIN, st);
  else if (m > 64) {
    // the large-M GEMM tiles 256 rows: a 128-row split point takes two launches
    GemvParams a = p, b = p;
    a.w1 = nullptr;
    a.N = (int)n;
    a.n_split = (int)n;
    b.w0 = p.w1;
    b.s0 = p.s1;
    b.w1 = nullptr;
    b.N = (int)n;
    b.n_split = (int)n;
    b.y = gu + n;
    rc = launch_gemm(a, GEMV_PLAIN, st);
    if (!rc) rc = launch_gemm(b, GEMV_PLAIN, st);
  } else {
    const GemvPlan pl = plan_linear((int)m, (int)(2 * n), (int)k);
    if (pl.kparts > 1) {
      // the K-part finish and silu * up in one pass (n % 128 == 0)
      if ((rc = launch_gemv(p, GEMV_PLAIN, pl, st, false))) return rc;
      const int64_t items = m * (n / 4);
      gu_finish_silu_kernel<<<(unsigned)((items + 63) / 64), 64, 0, st>>>(part, (int)m, (int)n, pl.kparts, h);
      if ((rc = check_launch("swiglu gate|up finish + silu_mul"))) return rc;
      return fp8_linear_into(h, (int)m, (int)n, static_cast<const uint8_t *>(down_w), down_s, (int)k,
                             static_cast<uint16_t *>(y), part, st);
    }
    rc = launch_gemv(p, GEMV_PLAIN, pl, st);
  }
  if (rc) return rc;
  silu_mul_rows_kernel<<<dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>(n / 8 / 256, 16)),
                              (unsigned)std::min<int64_t>(m, 65535)),
                         256, 0, st>>>(gu, (int)m, (int)n, h);
  if ((rc = check_launch("swiglu silu_mul"))) return rc;
  return fp8_linear_into(h, (int)m, (int)n, static_cast<const uint8_t *>(down_w), down_s, (int)k,
                         static_cast<uint16_t *>(y), part, st);
}

}  // extern "C"

namespace amla {

// ---------------------------------------------------------------- routing

// Partial logits part[z][m, e] = sum over the K steps of split z of
// f32(hidden[m, k]) * f32(gate_w[e, k]) for a 16-token x 16-expert tile per
// workgroup; the four waves take interleaved 32-wide K steps and add their
// partial tiles in wave order through LDS.  route_select adds the splits in
// order.
__global__ __launch_bounds__(256) void route_logits_kernel(const uint16_t *__restrict__ hidden,
                                                           const uint16_t *__restrict__ gw, int M, int D, int E,
                                                           float *__restrict__ part) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e0 = blockIdx.x * 16, m0 = blockIdx.y * 16, z = blockIdx.z, nz = gridDim.z;
  float *logits = part + (size_t)z * M * E;
  const int r = lane & 15, kq = lane >> 4;
  const uint16_t *hp = hidden + (size_t)min(m0 + r, M - 1) * D + 8 * kq;
  const uint16_t *wp = gw + (size_t)min(e0 + r, E - 1) * D + 8 * kq;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int steps = D / 32;
  for (int ks = wave + 4 * z; ks < steps; ks += 4 * nz)
    acc = mfma16(as_bf16x8(ldg16(hp + ks * 32)), as_bf16x8(ldg16(wp + ks * 32)), acc);
  __shared__ f32x4 red[4][64];
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4 v = red[0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) v += red[w][lane];
    // C layout: lane holds rows (tokens) 4 (lane/16) .. +3 of column (expert) lane % 16
    const int e = e0 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 4 * (lane >> 4) + i;
      if (m < M && e < E) logits[(size_t)m * E + e] = v[i];
    }
  }
}

constexpr int ROUTE_MAX_E = 1024;           // experts per token handled by one wave
constexpr int ROUTE_EPL = ROUTE_MAX_E / 64;  // experts per lane (lane l: l, l + 64, ..)
constexpr int ROUTE_MAX_Z = 8;               // K splits of the logits (route_ksplit)

// One wave per token: scores = sigmoid(logits); rank the n_group groups by
// their maximum score and keep topk_group of them; take the top_k experts of
// the kept groups by score (ties to the lower index); weights are the scores,
// divided by (sum + 1e-9) when norm is set.  The scores stay in registers:
// every split's partial logit is loaded at once and the splits are added in
// order; a group is kept when fewer than topk_group groups rank above it (a
// larger maximum, or an equal one at a lower index: the order of picking the
// best remaining group topk_group times); the top_k rounds are wave
// reductions.
__global__ __launch_bounds__(64) void route_select_kernel(const float *__restrict__ part, int M, int ksplit, int E,
                                                          int n_group, int topk_group, int top_k, int norm,
                                                          int64_t *__restrict__ idx_out, float *__restrict__ w_out) {
  __shared__ int gmax[64];  // group maxima as the bits of non-negative floats (ordered like the values)
  const int lane = threadIdx.x, m = blockIdx.x;
  const int gs = E / n_group;
  float sc[ROUTE_EPL];
#pragma unroll
  for (int i = 0; i < ROUTE_EPL; ++i) {
    const int e = lane + 64 * i;
    float v[ROUTE_MAX_Z];
#pragma unroll
    for (int z = 0; z < ROUTE_MAX_Z; ++z) v[z] = e < E && z < ksplit ? part[((size_t)z * M + m) * E + e] : 0.f;
    float l = v[0];
#pragma unroll
    for (int z = 1; z < ROUTE_MAX_Z; ++z)
      if (z < ksplit) l += v[z];
    sc[i] = e < E ? 1.f / (1.f + expf(-l)) : -4.f;  // -4: below every candidate and the initial best
  }
  if (lane < n_group) gmax[lane] = 0;  // +0.0f: every score is >= 0
  __syncthreads();
#pragma unroll
  for (int i = 0; i < ROUTE_EPL; ++i) {
    const int e = lane + 64 * i;
    if (e < E) atomicMax(&gmax[e / gs], __float_as_int(sc[i]));
  }
  __syncthreads();
  bool keep_g = false;
  if (lane < n_group) {
    const float gv = __int_as_float(gmax[lane]);
    int rank = 0;
    for (int g = 0; g < n_group; ++g) {
      const float ov = __int_as_float(gmax[g]);
      rank += ov > gv || (ov == gv && g < lane);
    }
    keep_g = rank < topk_group;
  }
  const uint64_t keep = __ballot(keep_g);
  // candidate scores: experts of dropped groups take part as 0.0 (the
  // reference's masked_scores), chosen ones are removed as -1
#pragma unroll
  for (int i = 0; i < ROUTE_EPL; ++i) {
    const int e = lane + 64 * i;
    if (e < E && !((keep >> (e / gs)) & 1)) sc[i] = 0.f;
  }
  float sum = 0.f, my_w = 0.f;
  int my_idx = 0;
  for (int t = 0; t < top_k; ++t) {
    float bv = -2.f;
    int bi = E;
#pragma unroll
    for (int i = 0; i < ROUTE_EPL; ++i)
      if (sc[i] > bv) {  // ascending e per lane: ties keep the lower index
        bv = sc[i];
        bi = lane + 64 * i;
      }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
#pragma unroll
    for (int i = 0; i < ROUTE_EPL; ++i)
      if (lane + 64 * i == bi) sc[i] = -1.f;
    if (lane == t) {
      my_idx = bi;
      my_w = bv;
    }
    sum += bv;
  }
  if (lane < top_k) {
    idx_out[(size_t)m * top_k + lane] = my_idx;
    w_out[(size_t)m * top_k + lane] = norm ? my_w / (sum + 1e-9f) : my_w;
  }
}

// ---------------------------------------------------------------- combine

// out[m] = bf16( shared[m] + bf16( acc * scale ) ),  acc = bf16 running sum
// over k of bf16( bf16(w[m, k]) * expert_out[m, k] ), in k order.
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t *__restrict__ shared,
                                                          const uint16_t *__restrict__ eout,
                                                          const float *__restrict__ w, int top_k, int64_t D,
                                                          float scale, uint16_t *__restrict__ out) {
  const int m = blockIdx.y;
  for (int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; d < D; d += (int64_t)gridDim.x * blockDim.x) {
    float acc = 0.f;
    for (int k = 0; k < top_k; ++k) {
      const float wk = round_bf16(w[(size_t)m * top_k + k]);
      acc = round_bf16(acc + round_bf16(wk * bf2f(eout[((size_t)m * top_k + k) * D + d])));
    }
    out[(size_t)m * D + d] = f2bf(bf2f(shared[(size_t)m * D + d]) + round_bf16(acc * scale));
  }
}

}  // namespace amla

extern "C" {

// K splits of the router logits: about 128 workgroups for decode-sized batches
static int route_ksplit(int64_t m, int64_t n_experts) {
  const int64_t tiles = ((n_experts + 15) / 16) * ((m + 15) / 16);
  return (int)std::max<int64_t>(1, std::min<int64_t>(ROUTE_MAX_Z, 128 / std::max<int64_t>(tiles, 1)));
}

size_t amla_moe_route_workspace_bytes(int64_t m, int64_t n_experts) {
  if (m <= 0 || n_experts <= 0) return 0;
  return align_up((size_t)route_ksplit(m, n_experts) * m * n_experts * 4, 256);
}

int amla_moe_route(const void *hidden, int64_t m, int64_t d, const void *gate_weight, int64_t n_experts,
                   int n_group, int topk_group, int top_k, int norm_topk_prob, int64_t *indices, float *weights,
                   void *workspace, size_t workspace_bytes, void *stream) {
  if (!hidden || !gate_weight || !indices || !weights) return fail(AMLA_EINVAL, "moe_route: null pointer");
  if (m < 0 || d <= 0 || n_experts <= 0 || n_group <= 0 || topk_group <= 0 || top_k <= 0)
    return fail(AMLA_EINVAL, "moe_route: bad sizes");
  if (m == 0) return AMLA_OK;
  if (n_experts % n_group || topk_group > n_group || n_group > 64 || n_experts > ROUTE_MAX_E ||
      (int64_t)topk_group * (n_experts / n_group) < top_k)
    return fail(AMLA_EINVAL,
                "moe_route: needs n_experts %% n_group == 0, topk_group <= n_group <= 64, n_experts <= %d and "
                "top_k <= topk_group * group size",
                ROUTE_MAX_E);
  if (top_k > 64) return fail(AMLA_EUNSUPPORTED, "moe_route: top_k > 64");
  if (d % 32 || !aligned16(hidden) || !aligned16(gate_weight) || m > (int64_t)65535 * 16 || d > INT32_MAX)
    return fail(AMLA_EUNSUPPORTED, "moe_route: needs hidden size %% 32 == 0 and 16-byte aligned inputs");
  const size_t need = amla_moe_route_workspace_bytes(m, n_experts);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(AMLA_EWORKSPACE, "moe_route: needs %zu bytes of 16-byte aligned workspace", need);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float *part = static_cast<float *>(workspace);
  const int ks = route_ksplit(m, n_experts);
  route_logits_kernel<<<dim3((unsigned)((n_experts + 15) / 16), (unsigned)((m + 15) / 16), (unsigned)ks), 256, 0,
                        st>>>(static_cast<const uint16_t *>(hidden), static_cast<const uint16_t *>(gate_weight),
                              (int)m, (int)d, (int)n_experts, part);
  int rc;
  if ((rc = check_launch("moe_route logits"))) return rc;
  route_select_kernel<<<dim3((unsigned)m), 64, 0, st>>>(part, (int)m, ks, (int)n_experts, n_group, topk_group, top_k,
                                                        norm_topk_prob, indices, weights);
  return check_launch("moe_route select");
}

int amla_moe_combine(const void *shared_out, const void *expert_out, const float *weights, int64_t m, int top_k,
                     int64_t d, float routed_scaling_factor, void *out, void *stream) {
  if (!shared_out || !expert_out || !weights || !out) return fail(AMLA_EINVAL, "moe_combine: null pointer");
  if (m < 0 || top_k <= 0 || d <= 0) return fail(AMLA_EINVAL, "moe_combine: bad sizes");
  if (m == 0) return AMLA_OK;
  if (m > 65535) return fail(AMLA_EUNSUPPORTED, "moe_combine: at most 65535 tokens per call");
  const unsigned bx = (unsigned)std::min<int64_t>((d + 255) / 256, 64);
  moe_combine_kernel<<<dim3(bx, (unsigned)m), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t *>(shared_out), static_cast<const uint16_t *>(expert_out), weights, top_k, d,
      routed_scaling_factor, static_cast<uint16_t *>(out));
  return check_launch("moe_combine");
}

}  // extern "C"

namespace amla {

// ---------------------------------------------------------------- routed experts

// (token, k) slots whose row lists travel as kernel arguments; larger chunks
// copy their lists into the workspace
constexpr int MOE_ARG_SLOTS = 512;
constexpr int MOE_MAX_SLOTS = 65536;  // slots per chunk

struct RowList {
  int32_t row[MOE_ARG_SLOTS];
};

// dst row i (of `rows`) = src row L[i]  (gather), or dst row L[i] = src row i
// (scatter); L = dlist when given (device memory), else the by-value list
// (drows: the row count in device memory, else rows)
template <bool SCATTER>
__global__ __launch_bounds__(256) void move_rows_kernel(const uint16_t *__restrict__ src, int64_t d, int rows,
                                                        RowList list, const int32_t *__restrict__ dlist,
                                                        uint16_t *__restrict__ dst,
                                                        const int32_t *__restrict__ drows = nullptr) {
  const int i = blockIdx.x;
  if (i >= (drows ? *drows : rows)) return;
  const int li = dlist ? dlist[i] : list.row[i];
  const uint16_t *s = src + (size_t)(SCATTER ? i : li) * d;
  uint16_t *t = dst + (size_t)(SCATTER ? li : i) * d;
  for (int64_t c = threadIdx.x; c < d / 8; c += blockDim.x)
    *reinterpret_cast<u32x4 *>(t + c * 8) = *reinterpret_cast<const u32x4 *>(s + c * 8);
}

struct MoeLayout {
  int chunk_tokens;
  size_t lists, xs, ys, gu, h, part, part_bytes, total;
};

static MoeLayout moe_layout(int64_t m, int64_t d, int top_k, int64_t n) {
  MoeLayout L;
  L.chunk_tokens = (int)std::min<int64_t>(m, (m * top_k <= MOE_ARG_SLOTS ? MOE_ARG_SLOTS : MOE_MAX_SLOTS) / top_k);
  const size_t slots = (size_t)L.chunk_tokens * top_k;
  // largest expert group on the skinny path: any run of one expert up to 64
  // slots (a token may list an expert more than once, so a run can be longer
  // than the chunk's token count); the K-part count grows with the group size
  const int mg = (int)std::min<size_t>(slots, 64);
  size_t off = 0;
  L.lists = off;
  off = align_up(off + (slots > MOE_ARG_SLOTS ? 2 * slots * 4 : 0), 256);
  L.xs = off;
  off = align_up(off + slots * d * 2, 256);
  L.ys = off;
  off = align_up(off + slots * d * 2, 256);
  L.gu = off;
  off = align_up(off + slots * 2 * n * 2, 256);
  L.h = off;
  off = align_up(off + slots * n * 2, 256);
  L.part = off;
  // partial sums of every group of one grouped launch, each sized for its own rows
  const GemvPlan a = plan_gemv(mg, (int)(2 * n), (int)d), b = plan_gemv(mg, (int)d, (int)n);
  const size_t pa = a.kparts > 1 ? (size_t)a.kparts * slots * 2 * n * 4 : 0;
  const size_t pb = b.kparts > 1 ? (size_t)b.kparts * slots * d * 4 : 0;
  L.part_bytes = std::max(pa, pb);
  off = align_up(off + L.part_bytes, 256);
  L.total = off;
  return L;
}

}  // namespace amla

extern "C" {

size_t amla_moe_experts_workspace_bytes(int64_t m, int64_t d, int top_k, int64_t n_inter) {
  if (m <= 0 || d <= 0 || top_k <= 0 || top_k > 64 || n_inter <= 0) return 0;
  return moe_layout(m, d, top_k, n_inter).total;
}

int amla_moe_experts(const void *hidden, int64_t m, int64_t d, int top_k, const int64_t *indices, int64_t n_inter,
                     int64_t n_experts, const void *const *gate_w, const float *const *gate_s,
                     const void *const *up_w, const float *const *up_s, const void *const *down_w,
                     const float *const *down_s, void *expert_out, void *workspace, size_t workspace_bytes,
                     void *stream) {
  if (!hidden || !indices || !gate_w || !gate_s || !up_w || !up_s || !down_w || !down_s || !expert_out)
    return fail(AMLA_EINVAL, "moe_experts: null pointer");
  if (m < 0 || d <= 0 || top_k <= 0 || n_inter <= 0 || n_experts <= 0) return fail(AMLA_EINVAL, "moe_experts: bad sizes");
  if (m == 0) return AMLA_OK;
  if (top_k > 64) return fail(AMLA_EUNSUPPORTED, "moe_experts: top_k > 64");
  if (d % 128 || n_inter % 256 || d > INT32_MAX || n_inter > INT32_MAX / 2 || !aligned16(hidden) ||
      !aligned16(expert_out))
    return fail(AMLA_EUNSUPPORTED,
                "moe_experts: needs hidden %% 128 == 0, intermediate %% 256 == 0 and 16-byte aligned rows");
  for (int64_t i = 0; i < m * top_k; ++i) {
    const int64_t e = indices[i];
    if (e < 0) continue;  // a slot left to another call (its expert_out row is not written)
    if (e >= n_experts) return fail(AMLA_EINVAL, "moe_experts: expert index %lld out of range", (long long)e);
    if (!gate_w[e] || !gate_s[e] || !up_w[e] || !up_s[e] || !down_w[e] || !down_s[e] || !aligned16(gate_w[e]) ||
        !aligned16(up_w[e]) || !aligned16(down_w[e]))
      return fail(AMLA_EINVAL, "moe_experts: expert %lld has a null or misaligned weight", (long long)e);
  }
  const MoeLayout L = moe_layout(m, d, top_k, n_inter);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
    return fail(AMLA_EWORKSPACE, "moe_experts: needs %zu bytes of 16-byte aligned workspace (got %zu)", L.total,
                workspace ? workspace_bytes : (size_t)0);
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  uint16_t *xs = reinterpret_cast<uint16_t *>(ws + L.xs), *ys = reinterpret_cast<uint16_t *>(ws + L.ys);
  uint16_t *gu = reinterpret_cast<uint16_t *>(ws + L.gu), *hb = reinterpret_cast<uint16_t *>(ws + L.h);
  float *part = reinterpret_cast<float *>(ws + L.part);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint16_t *hid = static_cast<const uint16_t *>(hidden);
  uint16_t *eout = static_cast<uint16_t *>(expert_out);
  const int n = (int)n_inter, D = (int)d;
  int rc;
  std::vector<int32_t> order;
  for (int64_t t0 = 0; t0 < m; t0 += L.chunk_tokens) {
    const int nt = (int)std::min<int64_t>(L.chunk_tokens, m - t0);
    // slots of this chunk with an expert (index >= 0), sorted by expert
    // (stable: token-major within an expert)
    const int64_t *ix = indices + t0 * top_k;
    order.clear();
    for (int i = 0; i < nt * top_k; ++i)
      if (ix[i] >= 0) order.push_back(i);
    const int ns = (int)order.size();
    if (ns == 0) continue;
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return ix[a] < ix[b]; });
    RowList gather, scatter;
    int32_t *dg = nullptr, *dsc = nullptr;
    if (ns <= MOE_ARG_SLOTS) {
      for (int i = 0; i < ns; ++i) {
        gather.row[i] = (int32_t)(t0 + order[i] / top_k);
        scatter.row[i] = (int32_t)(t0 * top_k + order[i]);
      }
    } else {
      // long lists go through the workspace; the host array must outlive the
      // copy, so this path waits for the stream once
      std::vector<int32_t> hl(2 * (size_t)ns);
      for (int i = 0; i < ns; ++i) {
        hl[i] = (int32_t)(t0 + order[i] / top_k);
        hl[ns + i] = (int32_t)(t0 * top_k + order[i]);
      }
      dg = reinterpret_cast<int32_t *>(ws + L.lists);
      dsc = dg + ns;
      hipError_t e = hipMemcpyAsync(dg, hl.data(), hl.size() * 4, hipMemcpyHostToDevice, st);
      if (e == hipSuccess) e = hipStreamSynchronize(st);
      if (e != hipSuccess) return fail((int)e, "moe_experts: row list copy failed: %s", hipGetErrorString(e));
    }
    move_rows_kernel<false><<<ns, 256, 0, st>>>(hid, d, ns, gather, dg, xs);
    if ((rc = check_launch("moe_experts gather"))) return rc;
    // runs of one expert: [run_begin[r], run_begin[r + 1])
    std::vector<int> run_begin;
    for (int i = 0; i < ns; ++i)
      if (i == 0 || ix[order[i]] != ix[order[i - 1]]) run_begin.push_back(i);
    run_begin.push_back(ns);
    const int nruns = (int)run_begin.size() - 1;
    int max_small = 0;
    for (int r = 0; r < nruns; ++r)
      if (run_begin[r + 1] - run_begin[r] <= 64) max_small = std::max(max_small, run_begin[r + 1] - run_begin[r]);
    GemvParams pg = {};  // [gate | up] x (cnt, D) -> gu (cnt, 2n)
    pg.ldx = D;
    pg.N = 2 * n;
    pg.K = D;
    pg.n_split = n;
    pg.ldy = 2 * n;
    pg.seq_len = 1;
    GemvParams pd = {};  // down h (cnt, n) -> ys (cnt, D)
    pd.ldx = n;
    pd.N = D;
    pd.K = n;
    pd.n_split = D;
    pd.ldy = D;
    pd.seq_len = 1;
    const GemvPlan plan_g = plan_gemv_grouped(std::max(max_small, 1), 2 * n, D);
    const GemvPlan plan_d = plan_gemv_grouped(std::max(max_small, 1), D, n);
    // experts with more than 64 of these tokens: one large-M GEMM each
    for (int r = 0; r < nruns; ++r) {
      const int i0 = run_begin[r], cnt = run_begin[r + 1] - i0;
      if (cnt <= 64) continue;
      const int64_t e = ix[order[i0]];
      GemvParams p = pg;
      p.x = xs + (size_t)i0 * D;
      p.M = cnt;
      p.w0 = static_cast<const uint8_t *>(gate_w[e]);
      p.s0 = gate_s[e];
      p.w1 = static_cast<const uint8_t *>(up_w[e]);
      p.s1 = up_s[e];
      p.y = gu + (size_t)i0 * 2 * n;
      if ((rc = launch_gemm(p, GEMV_PLAIN, st))) return rc;
    }
    // the others: grouped skinny GEMMs, GEMV_MAX_GROUPS experts per launch
    for (int pass = 0; pass < 2; ++pass) {
      if (pass == 1) {
        // silu * up over every row of [gate | up]
        silu_mul_rows_kernel<<<dim3((unsigned)std::max(1, std::min(n / 8 / 256, 16)), (unsigned)ns), 256, 0, st>>>(
            gu, ns, n, hb);
        if ((rc = check_launch("moe_experts silu_mul"))) return rc;
      }
      const GemvPlan &pl = pass == 0 ? plan_g : plan_d;
      const GemvParams &base = pass == 0 ? pg : pd;
      if (pl.kparts > 1 && (size_t)pl.kparts * ns * base.N * 4 > L.part_bytes)
        return fail(AMLA_EWORKSPACE, "moe_experts: K-part sums (%d parts x %d slots x %d) exceed the workspace plan",
                    pl.kparts, ns, base.N);
      GemvGroups gr;
      gr.n = 0;
      gr.units = 0;
      for (int r = 0; r <= nruns; ++r) {
        const bool flush = r == nruns || gr.n == GEMV_MAX_GROUPS;
        if (flush && gr.n) {
          if ((rc = launch_gemv_grouped(base, gr, pl, st))) return rc;
          gr.n = 0;
        }
        if (r == nruns) break;
        const int i0 = run_begin[r], cnt = run_begin[r + 1] - i0;
        if (cnt > 64) continue;
        const int64_t e = ix[order[i0]];
        GemvGroup &g = gr.g[gr.n++];
        g.M = cnt;
        g.pad = 0;
        if (pass == 0) {
          g.x = xs + (size_t)i0 * D;
          g.w0 = static_cast<const uint8_t *>(gate_w[e]);
          g.s0 = gate_s[e];
          g.w1 = static_cast<const uint8_t *>(up_w[e]);
          g.s1 = up_s[e];
          g.y = gu + (size_t)i0 * 2 * n;
          g.part = pl.kparts > 1 ? part + (size_t)pl.kparts * i0 * 2 * n : nullptr;
        } else {
          g.x = hb + (size_t)i0 * n;
          g.w0 = static_cast<const uint8_t *>(down_w[e]);
          g.s0 = down_s[e];
          g.w1 = nullptr;
          g.s1 = nullptr;
          g.y = ys + (size_t)i0 * D;
          g.part = pl.kparts > 1 ? part + (size_t)pl.kparts * i0 * D : nullptr;
        }
      }
    }
    for (int r = 0; r < nruns; ++r) {
      const int i0 = run_begin[r], cnt = run_begin[r + 1] - i0;
      if (cnt <= 64) continue;
      const int64_t e = ix[order[i0]];
      GemvParams q = pd;
      q.x = hb + (size_t)i0 * n;
      q.M = cnt;
      q.w0 = static_cast<const uint8_t *>(down_w[e]);
      q.s0 = down_s[e];
      q.y = ys + (size_t)i0 * D;
      if ((rc = launch_gemm(q, GEMV_PLAIN, st))) return rc;
    }
    move_rows_kernel<true><<<ns, 256, 0, st>>>(ys, d, ns, scatter, dsc, eout);
    if ((rc = check_launch("moe_experts scatter"))) return rc;
  }
  return AMLA_OK;
}

}  // extern "C"

namespace amla {

// ---------------------------------------------------------------- routed experts, device schedule

// amla_moe_experts_dev: the (token, k) slots are grouped by expert on the
// device, so the call needs no host copy of the indices and no stream
// synchronisation (a HIP graph can hold it).  moe_sort_kernel (one workgroup)
// makes the schedule; every later launch has a grid for the worst case and
// its workgroups past the device counts return at once.
constexpr int MSORT_WAVES = 16;     // 1024 threads
constexpr int MSORT_MAXE = 512;     // experts per layer
constexpr int MSORT_EBITS = 9;      // bits of an expert index
constexpr int MOE_DEV_MAX_SLOTS = 65536;
constexpr int MOE_TILE_ROWS = 256;  // rows of a GEMM tile entry

struct MoeDevLayout {
  int sb;                      // largest group on the skinny path
  int sb1;                     // largest group of the one-tile skinny launch (<= 16 rows)
  int max_small, max_small4, max_tiles;  // schedule entries (worst case)
  size_t hdr, cls, gather, scatter, small, small4, tiles, xs, ys, gu, h, part, total;
};

static MoeDevLayout moe_dev_layout(int64_t m, int64_t d, int top_k, int64_t n, int64_t E) {
  MoeDevLayout L;
  const int64_t S = m * top_k;
  // a token names an expert once in a routing, so a group has at most m rows;
  // larger groups (repeated indices) and groups over 64 rows take the GEMM
  L.sb = (int)std::min<int64_t>(std::min<int64_t>(m, 64), S);
  // skinny groups of up to 16 rows and of 17..sb rows take separate launches
  // (one x tile, or the tiles the largest needs), each sized for its own worst case
  L.sb1 = std::min(L.sb, 16);
  L.max_small = (int)std::min<int64_t>(E, S);
  L.max_small4 = L.sb > L.sb1 ? (int)std::min<int64_t>(E, S / (L.sb1 + 1)) : 0;
  L.max_tiles = (int)((S + MOE_TILE_ROWS - 1) / MOE_TILE_ROWS + std::min<int64_t>(E, S / (L.sb + 1)));
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes, 256); return o; };
  L.hdr = take(16);
  L.cls = take(8);
  L.gather = take((size_t)S * 4);
  L.scatter = take((size_t)S * 4);
  L.small = take((size_t)L.max_small * 16);
  L.small4 = take((size_t)std::max(L.max_small4, 1) * 16);
  L.tiles = take((size_t)std::max(L.max_tiles, 1) * 16);
  L.xs = take((size_t)S * d * 2);
  L.ys = take((size_t)S * d * 2);
  L.gu = take((size_t)S * 2 * n * 2);
  L.h = take((size_t)S * n * 2);
  const GemvPlan a = plan_gemv_grouped(L.sb, (int)(2 * n), (int)d), b = plan_gemv_grouped(L.sb, (int)d, (int)n);
  const size_t pa = a.kparts > 1 ? (size_t)a.kparts * S * 2 * n * 4 : 0;
  const size_t pb = b.kparts > 1 ? (size_t)b.kparts * S * d * 4 : 0;
  L.part = take(std::max<size_t>(std::max(pa, pb), 16));
  L.total = off;
  return L;
}

AMLA_DEV int block_scan_incl(int v, int *wsum, int lane, int wave) {
  // inclusive prefix sum over the first MSORT_WAVES * 64 threads (all take part)
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  if (lane == 63) wsum[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; ++w) v += wsum[w];
  __syncthreads();
  return v;
}

// Schedule of the routed slots.  Wave w walks slots [w S/16, (w+1) S/16) in
// order: first counting them per expert (its own row of counts), then, with
// every expert's start known, placing each slot at its expert's next free
// position (rank among equal experts of the 64-slot step by ballots), so the
// order is slot order within each expert whatever the timing.  Outputs:
//   gather[p] = token of position p, scatter[p] = slot of position p;
//   small[]   = (expert, first position, rows) of experts with 1..sb1 slots;
//   small4[]  = the same for experts with sb1+1..sb slots;
//   tiles[]   = (expert, first position, rows <= 256) of the larger ones;
//   hdr       = {routed slots, small + small4 entries, tile entries, skipped slots};
//   cls       = {small entries, small4 entries}.
// Slots with a negative index are left out; an index >= E, or an expert with a
// null or misaligned weight, is left out and counted as skipped.
__global__ __launch_bounds__(1024) void moe_sort_kernel(const int64_t *__restrict__ idx, int S, int top_k, int E,
                                                        int sb, int sb1, const void *const *__restrict__ wtab,
                                                        int32_t *__restrict__ hdr, int32_t *__restrict__ cls,
                                                        int32_t *__restrict__ gather, int32_t *__restrict__ scatter,
                                                        int32_t *__restrict__ small, int32_t *__restrict__ small4,
                                                        int32_t *__restrict__ tiles) {
  __shared__ int32_t cur[MSORT_WAVES][MSORT_MAXE];  // per-wave counts, then per-wave next positions
  __shared__ int32_t eok[MSORT_MAXE];
  __shared__ int32_t wsum[4][MSORT_WAVES];
  __shared__ int32_t skipped;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < MSORT_WAVES * MSORT_MAXE; i += 1024) (&cur[0][0])[i] = 0;
  for (int e = tid; e < E; e += 1024) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(wtab[j * E + e]);
      ok = ok && a != 0 && (a & ((j & 1) ? 3 : 15)) == 0;
    }
    eok[e] = ok;
  }
  if (tid == 0) skipped = 0;
  __syncthreads();
  const int b0 = (int)((int64_t)S * wave / MSORT_WAVES), b1 = (int)((int64_t)S * (wave + 1) / MSORT_WAVES);
  auto expert_of = [&](int i) -> int {  // -1: left out, -2: skipped
    if (i >= b1) return -1;
    const int64_t v = idx[i];
    if (v < 0) return -1;
    if (v >= E || !eok[(int)v]) return -2;
    return (int)v;
  };
  for (int base = b0; base < b1; base += 64) {
    const int e = expert_of(base + lane);
    if (e >= 0) atomicAdd(&cur[wave][e], 1);
    else if (e == -2) atomicAdd(&skipped, 1);
  }
  __syncthreads();
  // per expert: waves' counts -> offsets inside the expert; schedule sizes
  int tot = 0;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < MSORT_WAVES; ++w) {
      const int c = cur[w][tid];
      cur[w][tid] = tot;
      tot += c;
    }
  }
  const int is_small = tot >= 1 && tot <= sb1;
  const int is_small4 = tot > sb1 && tot <= sb;
  const int ntile = tot > sb ? (tot + MOE_TILE_ROWS - 1) / MOE_TILE_ROWS : 0;
  const int pos_incl = block_scan_incl(tot, wsum[0], lane, wave);
  const int small_incl = block_scan_incl(is_small, wsum[1], lane, wave);
  const int small4_incl = block_scan_incl(is_small4, wsum[3], lane, wave);
  const int tile_incl = block_scan_incl(ntile, wsum[2], lane, wave);
  const int first = pos_incl - tot;
  if (tid < E) {
#pragma unroll
    for (int w = 0; w < MSORT_WAVES; ++w) cur[w][tid] += first;
    if (is_small) {
      int32_t *en = small + 4 * (small_incl - 1);
      en[0] = tid; en[1] = first; en[2] = tot; en[3] = 0;
    }
    if (is_small4) {
      int32_t *en = small4 + 4 * (small4_incl - 1);
      en[0] = tid; en[1] = first; en[2] = tot; en[3] = 0;
    }
    for (int j = 0; j < ntile; ++j) {
      int32_t *en = tiles + 4 * (tile_incl - ntile + j);
      en[0] = tid; en[1] = first + j * MOE_TILE_ROWS; en[2] = min(MOE_TILE_ROWS, tot - j * MOE_TILE_ROWS); en[3] = 0;
    }
  }
  if (tid == 1023) {
    hdr[0] = pos_incl;
    hdr[1] = small_incl + small4_incl;
    hdr[2] = tile_incl;
    cls[0] = small_incl;
    cls[1] = small4_incl;
  }
  __syncthreads();
  if (tid == 0) hdr[3] = skipped;
  // placement, in slot order per wave
  for (int base = b0; base < b1; base += 64) {
    const int i = base + lane;
    const int e = expert_of(i);
    const bool act = e >= 0;
    uint64_t peers = __ballot(act);
#pragma unroll
    for (int bit = 0; bit < MSORT_EBITS; ++bit) {
      const bool on = act && ((e >> bit) & 1);
      const uint64_t bm = __ballot(on);
      peers &= on ? bm : ~bm;
    }
    const uint64_t lower = peers & ((1ull << lane) - 1);
    if (act) {
      const int p = cur[wave][e] + __popcll(lower);
      gather[p] = i / top_k;
      scatter[p] = i;
    }
    // every lane of the wave has read its position: the lowest lane of each
    // expert advances that expert's next position
    if (act && lower == 0) cur[wave][e] += __popcll(peers);
  }
}

}  // namespace amla

extern "C" {

size_t amla_moe_experts_dev_workspace_bytes(int64_t m, int64_t d, int top_k, int64_t n_inter, int64_t n_experts) {
  if (m <= 0 || d <= 0 || top_k <= 0 || top_k > 64 || n_inter <= 0 || n_experts <= 0 ||
      n_experts > MSORT_MAXE || m * top_k > MOE_DEV_MAX_SLOTS)
    return 0;
  return moe_dev_layout(m, d, top_k, n_inter, n_experts).total;
}

int amla_moe_experts_dev(const void *hidden, int64_t m, int64_t d, int top_k, const int64_t *indices,
                         int64_t n_inter, int64_t n_experts, const void *const *weight_table, void *expert_out,
                         void *workspace, size_t workspace_bytes, void *stream) {
  if (!hidden || !indices || !weight_table || !expert_out) return fail(AMLA_EINVAL, "moe_experts_dev: null pointer");
  if (m < 0 || d <= 0 || top_k <= 0 || n_inter <= 0 || n_experts <= 0)
    return fail(AMLA_EINVAL, "moe_experts_dev: bad sizes");
  if (m == 0) return AMLA_OK;
  if (top_k > 64 || n_experts > MSORT_MAXE || m * top_k > MOE_DEV_MAX_SLOTS)
    return fail(AMLA_EUNSUPPORTED, "moe_experts_dev: needs top_k <= 64, at most %d experts and %d slots per call",
                MSORT_MAXE, MOE_DEV_MAX_SLOTS);
  if (d % 128 || n_inter % 256 || d > INT32_MAX || n_inter > INT32_MAX / 2 || !aligned16(hidden) ||
      !aligned16(expert_out))
    return fail(AMLA_EUNSUPPORTED,
                "moe_experts_dev: needs hidden %% 128 == 0, intermediate %% 256 == 0 and 16-byte aligned rows");
  const MoeDevLayout L = moe_dev_layout(m, d, top_k, n_inter, n_experts);
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
    return fail(AMLA_EWORKSPACE, "moe_experts_dev: needs %zu bytes of 16-byte aligned workspace (got %zu)", L.total,
                workspace ? workspace_bytes : (size_t)0);
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  int32_t *hdr = reinterpret_cast<int32_t *>(ws + L.hdr);
  int32_t *gather = reinterpret_cast<int32_t *>(ws + L.gather), *scatter = reinterpret_cast<int32_t *>(ws + L.scatter);
  int32_t *small = reinterpret_cast<int32_t *>(ws + L.small), *tiles = reinterpret_cast<int32_t *>(ws + L.tiles);
  uint16_t *xs = reinterpret_cast<uint16_t *>(ws + L.xs), *ys = reinterpret_cast<uint16_t *>(ws + L.ys);
  uint16_t *gu = reinterpret_cast<uint16_t *>(ws + L.gu), *hb = reinterpret_cast<uint16_t *>(ws + L.h);
  float *part = reinterpret_cast<float *>(ws + L.part);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int S = (int)(m * top_k), n = (int)n_inter, D = (int)d, E = (int)n_experts;
  int rc;
  int32_t *cls = reinterpret_cast<int32_t *>(ws + L.cls), *small4 = reinterpret_cast<int32_t *>(ws + L.small4);
  moe_sort_kernel<<<1, 1024, 0, st>>>(indices, S, top_k, E, L.sb, L.sb1, weight_table, hdr, cls, gather, scatter,
                                      small, small4, tiles);
  if ((rc = check_launch("moe_experts_dev schedule"))) return rc;
  RowList none = {};
  move_rows_kernel<false><<<S, 256, 0, st>>>(static_cast<const uint16_t *>(hidden), d, S, none, gather, xs, hdr);
  if ((rc = check_launch("moe_experts_dev gather"))) return rc;
  const MoeSched small_gu = {weight_table, small, cls, E, 0}, tiles_gu = {weight_table, tiles, hdr + 2, E, 0};
  const MoeSched small_dn = {weight_table, small, cls, E, 1}, tiles_dn = {weight_table, tiles, hdr + 2, E, 1};
  const MoeSched small4_gu = {weight_table, small4, cls + 1, E, 0}, small4_dn = {weight_table, small4, cls + 1, E, 1};
  GemvParams pg = {};  // [gate | up] x (rows, D) -> gu (rows, 2n)
  pg.x = xs; pg.ldx = D; pg.N = 2 * n; pg.K = D; pg.n_split = n; pg.y = gu; pg.ldy = 2 * n; pg.seq_len = 1;
  pg.part = part;
  GemvParams pd = {};  // down h (rows, n) -> ys (rows, D)
  pd.x = hb; pd.ldx = n; pd.N = D; pd.K = n; pd.n_split = D; pd.y = ys; pd.ldy = D; pd.seq_len = 1;
  pd.part = part;
  if ((rc = launch_gemm_sched(pg, tiles_gu, L.max_tiles, st))) return rc;
  if ((rc = launch_gemv_sched(pg, small_gu, L.max_small, L.sb1, plan_gemv_grouped(L.sb1, 2 * n, D), st))) return rc;
  if ((rc = launch_gemv_sched(pg, small4_gu, L.max_small4, L.sb, plan_gemv_grouped(L.sb, 2 * n, D), st))) return rc;
  silu_mul_rows_kernel<<<dim3((unsigned)std::max(1, std::min(n / 8 / 256, 16)), (unsigned)std::min(S, 65535)), 256,
                         0, st>>>(gu, S, n, hb, hdr);
  if ((rc = check_launch("moe_experts_dev silu_mul"))) return rc;
  if ((rc = launch_gemm_sched(pd, tiles_dn, L.max_tiles, st))) return rc;
  if ((rc = launch_gemv_sched(pd, small_dn, L.max_small, L.sb1, plan_gemv_grouped(L.sb1, D, n), st))) return rc;
  if ((rc = launch_gemv_sched(pd, small4_dn, L.max_small4, L.sb, plan_gemv_grouped(L.sb, D, n), st))) return rc;
  move_rows_kernel<true><<<S, 256, 0, st>>>(ys, d, S, none, scatter, static_cast<uint16_t *>(expert_out), hdr);
  return check_launch("moe_experts_dev scatter");
}

}  // extern "C"
