// Host-side plumbing shared by the translation units of libamla.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "amla.h"

namespace amla {

// Records a message for amla_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char *what);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------- skinny fp8 GEMM

enum GemvMode : int {
  GEMV_PLAIN = 0,  // y[m, n] = bf16(acc)
  GEMV_RESID = 1,  // y[m, n] = bf16(res[m, n] + bf16(acc))
  GEMV_QKVA = 2,   // rows < n_split -> y; the rest -> latent / rope-key cache rows
  GEMV_QROPE = 3,  // y = bf16(acc); rows with (n % head_dim) >= nope rotated by RoPE at pos(m)
  GEMV_F32 = 4,    // y[m, n] = acc as fp32 (y is a float buffer, ldy counted in floats)
};

struct GemvParams {
  const uint16_t *x;  // (M, K) bf16, row stride ldx
  int M, ldx;
  const uint16_t *xg;  // optional (K) bf16 per-column factor: the GEMM takes bf16(x * xg) as its input
  const uint8_t *w0;  // rows [0, n_split) (all rows unless QKVA)
  const float *s0;
  const uint8_t *w1;  // rows [n_split, N) for QKVA, or for any mode when set (two stacked weights)
  const float *s1;
  int N, K, n_split;
  uint16_t *y;
  int ldy;
  const uint16_t *res;  // RESID
  int ldr;
  uint16_t *ckv, *kpe;  // QKVA destinations
  int64_t ckv_bstride, kpe_bstride;
  int kv_lora, rope;
  const int32_t *pos;   // per-m positions (QKVA, QROPE); m indexes (b * S + s)
  int seq_len;          // S: position of row m is pos[m / S] + m % S
  int max_rows;         // QKVA: cache rows per sequence (stores to rows >= max_rows are dropped)
  int rope_rows;        // QROPE: rows of rope_table (positions are clamped to rope_rows - 1)
  const float *rope_table;
  int head_dim, nope;   // QROPE
  float *part;          // fp32 partial sums of the K parts (GemvPlan::part_bytes), else unused
  int xnorm;            // streaming GEMV only: x is the raw input, projected as rms_norm(x, xg, eps_in)
  float eps_in;         // (bf16(bf16(x * rsqrt(mean(x^2) + eps_in)) * xg), the norm's own rounding)
};

struct GemvPlan {
  int kpb;           // 128-wide K blocks per K part
  int kparts;        // K parts (workgroups per row group); > 1 needs GemvParams::part
  int rg;            // 16-row tiles per workgroup
  int groups;        // workgroups
  size_t lds;        // dynamic LDS bytes per workgroup
  size_t part_bytes; // fp32 partial sums (kparts * M * N * 4) when kparts > 1
  int vec;           // streaming GEMV: 1 vgemv_kernel, 2 vgemv_short_kernel (one row of x),
                     // 3 xgemv_kernel (2 .. 8 rows of x in LDS), 4 mgemv_kernel (9 .. 64 rows of x,
                     // kparts K parts summed by a finish as for gemv_kernel)
};

GemvPlan plan_gemv(int M, int N, int K);
// plan_gemv, or a streaming GEMV where one applies: one row of x, N % 8 == 0,
// and 4096 <= K <= 16384 (K % 128 == 0; vec = 1) or K = 1536 (one weight
// segment, not the cache-row epilogue; vec = 2); or 2 .. 8 rows of x at the
// attention projections' shapes (vec = 3); or 9 .. 64 rows of x at the MLA
// projections' shapes (vec = 4).  For launch_gemv only (the grouped and
// scheduled launches take plan_gemv plans).
GemvPlan plan_linear(int M, int N, int K);
size_t gemv_lds_bytes(int MT, int kpb, int rg, int kparts);  // MT = 16-row tiles of x (1, 2 or 4)
// Launches the skinny GEMM for M <= 64 (N % 16 == 0, K % 128 == 0, 16-byte aligned rows);
// p.part must hold plan.part_bytes when plan.kparts > 1.
// finish = false leaves the fp32 K-part sums in p.part (plan.kparts > 1) for
// the caller's own finishing kernel.
int launch_gemv(const GemvParams &p, int mode, const GemvPlan &plan, hipStream_t stream, bool finish = true);
// QKVA finish with the q_a RMSNorm fused: sums the K parts, writes the kv_a
// rows into the caches and rms_norm(q_a, gamma, eps) (both roundings of
// inference/ops.py:12) into p.y; one workgroup per row.  With x_raw (the
// GEMM ran on bf16(x * input_gamma), p.xg), every sum is first multiplied by
// the row's input RMSNorm factor rsqrt(mean(x_raw^2) + eps_in).
int launch_qkva_finish_norm(const GemvParams &p, int kparts, const uint16_t *gamma, float eps, hipStream_t stream,
                            const uint16_t *x_raw = nullptr, float eps_in = 0.f);

// Independent skinny GEMMs of one shape in one launch (GEMV_PLAIN): the
// fields below replace those of the shared GemvParams for group g.
constexpr int GEMV_MAX_GROUPS = 32;
struct GemvGroup {
  const uint16_t *x;
  const uint8_t *w0;
  const float *s0;
  const uint8_t *w1;
  const float *s1;
  uint16_t *y;
  float *part;  // plan.kparts * M * N fp32 of this group when plan.kparts > 1
  int M, pad;
};
struct GemvGroups {
  int n;      // groups in use
  int units;  // workgroups per group (set by launch_gemv_grouped)
  GemvGroup g[GEMV_MAX_GROUPS];
};
// plan: plan_gemv_grouped(max M of the groups, N, K) (or plan_gemv).
GemvPlan plan_gemv_grouped(int M, int N, int K);
int launch_gemv_grouped(const GemvParams &p, GemvGroups groups, const GemvPlan &plan, hipStream_t stream);
// Routed-expert work scheduled on the device (amla_moe_experts_dev): entries
// of (expert, first row, rows, unused) int32, their count in device memory,
// and the device table of expert weights [6][E]: gate_w, gate_s, up_w, up_s,
// down_w, down_s.  Row r of an entry's x / y is row (first row + r) of the
// gathered buffers.
struct MoeSched {
  const void *const *wtab;
  const int32_t *ent;
  const int32_t *count;
  int E;
  int down;  // 0: [gate | up] as two weight segments (n_split = gate rows), 1: down
};
AMLA_DEV void moe_sched_weights(GemvParams &p, const MoeSched &s, int e) {
  const void *const *t = s.wtab + (s.down ? 4 : 0) * s.E;
  p.w0 = static_cast<const uint8_t *>(t[e]);
  p.s0 = static_cast<const float *>(t[s.E + e]);
  p.w1 = s.down ? nullptr : static_cast<const uint8_t *>(t[2 * s.E + e]);
  p.s1 = s.down ? nullptr : static_cast<const float *>(t[3 * s.E + e]);
}
// Skinny GEMMs (GEMV_PLAIN) of the scheduled entries, each with at most max_m
// rows; grid max_entries x plan.groups.  plan: plan_gemv_grouped(max_m, N, K);
// p.part holds plan.kparts * (rows of all entries) * N fp32 when kparts > 1
// (entry at first row r0 uses part + kparts * r0 * N).
int launch_gemv_sched(const GemvParams &p, const MoeSched &s, int max_entries, int max_m, const GemvPlan &plan,
                      hipStream_t stream);
// Large-M fp8 GEMM tiles of the scheduled entries (rows <= 256 each).
int launch_gemm_sched(const GemvParams &p, const MoeSched &s, int max_entries, hipStream_t stream);
// Large-M fp8 GEMM with the same modes (M > 64).  With split_ws of at least
// gemm_ws_bytes(M, N, K) bytes, tiles past the last full round of 256
// workgroups are cut into K parts (fp32 partial sums in split_ws, summed in
// part order by a finishing kernel); without it every tile takes the whole K.
constexpr int GEMV_MAX_PARTS = 32;  // K parts of the skinny GEMM (summed by its finishing passes)
constexpr int GEMM_MAX_PARTS = 8;
struct GemmSplit {
  int full;        // tiles with the whole K
  int parts;       // K parts of each later tile
  int n_tiles;     // 256-column tiles
  int items;       // workgroups
  float *partial;  // [split tile][part][256 x 256] fp32 in the workgroup's lane order
  size_t bytes;    // of partial
};
GemmSplit plan_gemm_split(int M, int N, int K);
size_t gemm_ws_bytes(int M, int N, int K);
int launch_gemm(const GemvParams &p, int mode, hipStream_t stream, float *split_ws = nullptr,
                size_t split_ws_bytes = 0);

int launch_rms_norm(const uint16_t *x, int64_t rows, int64_t dim, int64_t ldx, const uint16_t *gamma,
                    float eps, uint16_t *y, int64_t ldy, hipStream_t stream);

// Host checks shared by the MLA entry points (dimensions, null pointers,
// alignment, context bounds); returns AMLA_OK or the failure code.
int check_mla_common(const amla_mla_args *a, const char *who);
// Rows of context the kernels may read for these args: max_context when set
// (> 0), else max_seq.
inline int mla_context_bound(const amla_mla_args &a) { return a.max_context > 0 ? a.max_context : a.max_seq; }

}  // namespace amla
