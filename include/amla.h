/* amla: MI355X (gfx950) absorbed-MLA + block-FP8 linear kernels, C ABI.
 *
 * Plain pointers and sizes only.  Every pointer argument is a device pointer
 * unless noted; bf16 tensors are passed as raw 16-bit storage, fp8 weights as
 * raw OCP e4m3fn bytes (torch.float8_e4m3fn), scales as fp32.  All calls are
 * asynchronous on `stream` (a hipStream_t; NULL = the default stream), never
 * synchronise the host and never allocate: outputs and workspaces belong to the
 * caller.  Return value: 0 on success, < 0 for a bad argument (nothing is
 * launched), > 0 a hipError_t from a launch.  amla_last_error() gives the
 * message of the last failing call on the calling thread.
 *
 * The reference (sushruta/deepseek-on-one-gpu) has no FFI: its path is the set
 * of Python functions in inference/ops.py.  Each entry point below names the
 * function it replaces.
 */
#ifndef AMLA_H_
#define AMLA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AMLA_OK 0
#define AMLA_EINVAL (-1)
#define AMLA_EWORKSPACE (-2)
#define AMLA_EUNSUPPORTED (-3)

/* Version of this ABI (major * 100 + minor). */
int amla_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *amla_last_error(void);

/* Replaces the dequantisation half of fp8_linear, inference/ops.py:30-43:
 *   out[i*k + j] = f32(weight[i*k + j]) * scale_inv[(i/128) * ceil(k/128) + j/128]
 * Bit-exact fp32 (exact e4m3 convert, one RNE multiply).
 * weight (n, k) e4m3fn row-major; scale_inv (ceil(n/128), ceil(k/128)) fp32;
 * out (n, k) fp32. */
int amla_fp8_block_dequant(const void *weight, const float *scale_inv, int64_t n, int64_t k,
                           float *out, void *stream);

/* Replaces fp8_linear(x, weight, scale_inv, out_dtype=bf16), inference/ops.py:15-44:
 *   y[i, j] = bf16( sum_k x[i, k] * f32(weight[j, k]) * scale_inv[j/128, k/128] )
 * fp32 accumulation; x (m, k) bf16 with row stride ldx; y (m, n) bf16 with row
 * stride ldy.  For m <= 64 a long K is split over workgroups whose fp32
 * partial sums need `workspace` (16-byte aligned) of
 * amla_fp8_linear_workspace_bytes(m, n, k) bytes; when that is 0, NULL is
 * accepted.  Scratch only: no contents carry between calls. */
int amla_fp8_linear(const void *x, int64_t m, int64_t k, int64_t ldx, const void *weight,
                    const float *scale_inv, int64_t n, void *y, int64_t ldy, void *workspace,
                    size_t workspace_bytes, void *stream);
size_t amla_fp8_linear_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* Replaces fp8_linear(x, weight, scale_inv, out_dtype=torch.float32),
 * inference/ops.py:15-44 (the fp32 result before `.to(out_dtype)`, :44):
 *   y[i, j] = sum_k x[i, k] * f32(weight[j, k]) * scale_inv[j/128, k/128]
 * as amla_fp8_linear, with y (m, n) fp32, row stride ldy (in floats, ldy % 4
 * == 0, y 16-byte aligned).  Same workspace (amla_fp8_linear_workspace_bytes).
 * Any other out_dtype is this result cast by the caller, as in the reference. */
int amla_fp8_linear_f32(const void *x, int64_t m, int64_t k, int64_t ldx, const void *weight,
                        const float *scale_inv, int64_t n, float *y, int64_t ldy, void *workspace,
                        size_t workspace_bytes, void *stream);

/* Replaces rms_norm(x, weight, eps), inference/ops.py:10-12:
 *   r = rsqrt(mean(f32(x)^2) + eps);  y = bf16( bf16(f32(x) * r) * gamma )
 * x (rows, dim) bf16, row stride ldx; gamma (dim) bf16; y (rows, dim), ldy. */
int amla_rms_norm(const void *x, int64_t rows, int64_t dim, int64_t ldx, const void *gamma,
                  float eps, void *y, int64_t ldy, void *stream);

/* Replaces apply_rope(x, freqs), inference/ops.py:86-97, for x laid out as
 * (groups, s, dim) bf16 (dim even, pairs (2i, 2i+1) interleaved) and freqs as
 * (s, dim/2) complex64 viewed as fp32 (cos, sin) pairs:
 *   (y0, y1) = bf16( x0*cos - x1*sin, x0*sin + x1*cos )  in fp32. */
int amla_apply_rope(const void *x, int64_t groups, int64_t s, int64_t dim, const float *freqs,
                    void *y, void *stream);

/* Arguments of one MLA call (decode or prefill) for DeepSeek-R1 dimensions.
 * Mirrors the arguments of mla_attention(hidden, attn_weights, kv_cache,
 * position, rope_freqs, config), inference/ops.py:100-107, unpacked:
 * attn_weights keys (inference/weight_store.py:208-226) become w_* / s_* / gamma_*,
 * kv_cache the two cache pointers, rope_freqs the fp32 (cos, sin) table. */
typedef struct amla_mla_args {
  /* dimensions (config fields, inference/config.py:8-20) */
  int32_t batch;        /* B */
  int32_t seq_len;      /* S new tokens per sequence (1 = decode) */
  int32_t hidden;       /* 7168 */
  int32_t heads;        /* 128 */
  int32_t q_lora;       /* 1536 */
  int32_t kv_lora;      /* 512 */
  int32_t qk_nope;      /* 128 */
  int32_t qk_rope;      /* 64 */
  int32_t v_dim;        /* 128 */
  int32_t max_seq;      /* cache rows per sequence */
  int32_t rope_rows;    /* rows of the rope table */
  int32_t max_context;  /* upper bound of position+S over the batch (scheduling) */
  float eps;            /* rms_norm_eps */
  float softmax_scale;  /* yarn_get_mscale(factor, mscale_all_dim) / sqrt(qk_head_dim) */
  /* first new position of each sequence: positions[b] (device int32, length
   * batch); the reference's scalar `position` is the case of all-equal entries */
  const int32_t *positions;
  /* activations */
  const void *hidden_states;  /* (B, S, hidden) bf16, already input-normed unless input_gamma */
  void *out;                  /* (B, S, hidden) bf16 */
  /* optional transformer_layer attention half (inference/forward.py:92-94):
   * if input_gamma != NULL, hidden_states is normed with it first (in decode
   * folded into the q_a|kv_a projection: bf16(x * input_gamma) projected, the
   * sums scaled by the row's rsqrt(mean(x^2) + eps)); if residual != NULL,
   * out = residual + attention (bf16 add). */
  const void *input_gamma;
  const void *residual;
  /* block-FP8 projections (weight e4m3fn row-major, scale_inv fp32) */
  const void *w_q_a;  const float *s_q_a;   /* (q_lora, hidden) */
  const void *w_q_b;  const float *s_q_b;   /* (heads*(nope+rope), q_lora) */
  const void *w_kv_a; const float *s_kv_a;  /* (kv_lora+rope, hidden) */
  const void *w_kv_b; const float *s_kv_b;  /* (heads*(nope+v), kv_lora) */
  const void *w_o;    const float *s_o;     /* (hidden, heads*v) */
  const void *gamma_q;   /* q_a_layernorm (q_lora) bf16 */
  const void *gamma_kv;  /* kv_a_layernorm (kv_lora) bf16 */
  /* latent cache (B_alloc, max_seq, kv_lora) and rope-key cache
   * (B_alloc, max_seq, qk_rope), bf16, raw (pre-norm, pre-RoPE) rows;
   * rows [positions[b], positions[b]+S) of sequence b are written. */
  void *ckv_cache;
  void *kpe_cache;
  const float *rope_table;  /* (rope_rows, qk_rope/2, 2) fp32 cos/sin */
  void *workspace;
  size_t workspace_bytes;
  /* optional (B, S, heads * v_dim) bf16, 16-byte aligned: when set, the
   * per-head attention output before o_proj (the `out` of inference/ops.py:182,
   * heads-major columns h * v_dim + d) is written here instead of the workspace,
   * and o_proj reads it from here. */
  void *attn_out;
} amla_mla_args;

/* Replaces mla_attention(...) for S == 1, inference/ops.py:100-183, computed in
 * absorbed form (q_nope.W_UK into latent space, scores on the raw latent +
 * rope cache, online softmax split over context, latent.W_UV back to heads).
 * Any batch (ops.py:119): more than 64 sequences run as chunks of 64, one after
 * another on the stream, in one workspace sized for 64. */
int amla_mla_decode(const amla_mla_args *args, void *stream);

/* Measurement hook with no counterpart in the reference: amla_mla_decode that
 * also records events[i] (hipEvent_t) on `stream` before each of its 7 stages
 * (q_a|kv_a projection, preceded by the input RMSNorm in layer mode; q_a norm
 * with the projection's K-part finish; q_b projection + RoPE; W_UK absorption;
 * attention; split merge + W_UV; o_proj) and events[7] after the last, so a
 * benchmark can time each kernel on the stream it runs on. */
int amla_mla_decode_profiled(const amla_mla_args *args, void *stream, void *const *events);
/* The same hook with the attention kernel launched attn_repeat (1..64) times
 * back to back between events[4] and events[5] (it reads the same inputs and
 * rewrites the same partial results, so the output is unchanged): the
 * per-launch time (events[5] - events[4]) / attn_repeat then carries only a
 * 1/attn_repeat share of the event and dispatch overhead around one launch. */
int amla_mla_decode_profiled_repeat(const amla_mla_args *args, void *stream, void *const *events, int attn_repeat);

/* No counterpart in the reference: for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * amla_mla_decode with its scratch taken from a per-device static device array
 * of AMLA_NOALLOC_SCRATCH_BYTES (enough for batch <= 32 at any context);
 * args->workspace and args->workspace_bytes are ignored.  Calls no allocating
 * routine.  Every call on one device shares that device's array (it holds the
 * last call's intermediates; nothing in it needs to start at zero): calls that
 * overlap in time on one device (two streams, two threads) race and must be
 * serialised by the caller.  Returns AMLA_EWORKSPACE, launching nothing, when
 * amla_mla_decode_workspace_bytes(args) exceeds the array. */
#define AMLA_NOALLOC_SCRATCH_BYTES (48u << 20)
int amla_mla_decode_noalloc(const amla_mla_args *args, void *stream);

/* Replaces mla_attention(...) for S >= 1 with a causal mask over the new rows
 * (inference/ops.py:100-183 incl. :172-177): kv_b decompression of the cached
 * rows and flash attention with bf16 MFMA. */
int amla_mla_prefill(const amla_mla_args *args, void *stream);

/* Workspace bytes amla_mla_decode / amla_mla_prefill need for these args
 * (pointer fields are ignored).  Scratch only: no contents carry between calls. */
size_t amla_mla_decode_workspace_bytes(const amla_mla_args *args);
size_t amla_mla_prefill_workspace_bytes(const amla_mla_args *args);

/* ---- FFN / MoE on the same fp8 kernels ---- */

/* The elementwise half of swiglu, inference/ops.py:189-191 (F.silu(gate) * up):
 *   out[i] = bf16( bf16( g / (1 + exp(-g)) ) * up[i] ),  g = f32(gate[i])
 * gate, up, out: numel bf16 values (out may alias gate). */
int amla_silu_mul(const void *gate, const void *up, int64_t numel, void *out, void *stream);

/* Replaces swiglu(x, gate_proj, gate_scale, up_proj, up_scale, down_proj,
 * down_scale), inference/ops.py:186-192, and so dense_ffn / expert_ffn
 * (:195-206):  y = fp8_linear( bf16(silu(fp8_linear(x, gate))) * fp8_linear(x, up), down )
 * x (m, k) bf16; gate_w, up_w (n, k) e4m3fn with (ceil(n/128), ceil(k/128))
 * fp32 scales; down_w (k, n) with (ceil(k/128), ceil(n/128)) scales; y (m, k)
 * bf16.  k and n multiples of 128.  Workspace (16-byte aligned) of
 * amla_swiglu_workspace_bytes(m, k, n) bytes; scratch only. */
int amla_swiglu(const void *x, int64_t m, int64_t k, const void *gate_w, const float *gate_s, const void *up_w,
                const float *up_s, int64_t n, const void *down_w, const float *down_s, void *y, void *workspace,
                size_t workspace_bytes, void *stream);
size_t amla_swiglu_workspace_bytes(int64_t m, int64_t k, int64_t n);

/* Replaces route(hidden, gate_weight, config), inference/ops.py:209-257:
 *   scores = sigmoid(f32(hidden) @ f32(gate_weight)^T); keep the topk_group
 *   groups (n_experts / n_group experts each) with the largest maximum score;
 *   indices = the top_k experts by score with the other groups' scores at 0.0
 *   (ties to the lower index); weights = their scores, / (sum + 1e-9) when
 *   norm_topk_prob.
 * hidden (m, d) bf16 (d % 32 == 0); gate_weight (n_experts, d) bf16;
 * indices (m, top_k) int64, weights (m, top_k) fp32.  Workspace of
 * amla_moe_route_workspace_bytes(m, n_experts) bytes (the fp32 logits). */
int amla_moe_route(const void *hidden, int64_t m, int64_t d, const void *gate_weight, int64_t n_experts,
                   int n_group, int topk_group, int top_k, int norm_topk_prob, int64_t *indices, float *weights,
                   void *workspace, size_t workspace_bytes, void *stream);
size_t amla_moe_route_workspace_bytes(int64_t m, int64_t n_experts);

/* Replaces the routed-expert loop of moe_block, inference/forward.py:139-151
 * (expert_ffn of every (token, k) pair), with the experts already on the device:
 *   expert_out[t, k] = swiglu(hidden[t], expert indices[t, k])
 * indices (m, top_k) int64 in HOST memory (the reference also brings them to
 * the host); an index < 0 skips its (token, k) slot, whose expert_out row is
 * then left as it was (a caller that holds only some experts on the device
 * runs them in several calls); gate_w .. down_s: HOST arrays of n_experts
 * device pointers (only the chosen experts' entries are read; others may be
 * NULL), the weights of
 * expert e laid out as for amla_swiglu with intermediate size n_inter.  Each
 * chosen expert runs once over all of its tokens (gather, [gate | up] in one
 * skinny GEMM, silu * up, down, scatter).  hidden (m, d) bf16, expert_out
 * (m, top_k, d) bf16; d % 128 == 0, n_inter % 256 == 0, top_k <= 64.
 * Workspace of amla_moe_experts_workspace_bytes(m, d, top_k, n_inter) bytes.
 * Up to 512 (token, k) slots the call is asynchronous like the others; above
 * that the slot lists are copied from host memory and the call waits for
 * `stream` once per 65536 slots. */
int amla_moe_experts(const void *hidden, int64_t m, int64_t d, int top_k, const int64_t *indices, int64_t n_inter,
                     int64_t n_experts, const void *const *gate_w, const float *const *gate_s,
                     const void *const *up_w, const float *const *up_s, const void *const *down_w,
                     const float *const *down_s, void *expert_out, void *workspace, size_t workspace_bytes,
                     void *stream);
size_t amla_moe_experts_workspace_bytes(int64_t m, int64_t d, int top_k, int64_t n_inter);

/* amla_moe_experts with the indices left on the device: the same computation
 * (forward.py:139-151, each chosen expert once over all of its tokens), with
 * the (token, k) slots grouped by expert on the device, so the call copies
 * nothing from the host, never waits for the stream and can be captured in a
 * HIP graph.  The reference brings the indices to the host (gpu_transfer.py:60,
 * `.tolist()`) before its expert loop; this entry point has no counterpart
 * there.  It is for callers that hold every expert of the layer on the device.
 *   indices (m, top_k) int64 in DEVICE memory; an index < 0 skips its slot
 *     (expert_out row left as it was);
 *   weight_table: DEVICE array of 6 * n_experts pointers, [gate_w | gate_s |
 *     up_w | up_s | down_w | down_s] x n_experts (weights 16-byte aligned,
 *     scales 4-byte aligned), laid out per expert as for amla_swiglu;
 *   m * top_k <= 65536, n_experts <= 512, top_k <= 64, d % 128 == 0,
 *   n_inter % 256 == 0.
 * A slot whose index is >= n_experts, or whose expert has a NULL or misaligned
 * pointer in the table, is skipped like a negative one and counted: after the
 * call the first 16 bytes of the workspace hold int32 {routed slots, skinny
 * groups, GEMM tiles, skipped slots}.  Workspace of
 * amla_moe_experts_dev_workspace_bytes(m, d, top_k, n_inter, n_experts) bytes
 * (0 for unsupported sizes); calls that share a workspace must not overlap. */
int amla_moe_experts_dev(const void *hidden, int64_t m, int64_t d, int top_k, const int64_t *indices,
                         int64_t n_inter, int64_t n_experts, const void *const *weight_table, void *expert_out,
                         void *workspace, size_t workspace_bytes, void *stream);
size_t amla_moe_experts_dev_workspace_bytes(int64_t m, int64_t d, int top_k, int64_t n_inter, int64_t n_experts);

/* The combine of moe_block, inference/forward.py:138-153, for m tokens:
 *   acc = 0;  for k in 0..top_k-1:  acc = bf16( acc + bf16( bf16(w[t, k]) * expert_out[t, k] ) )
 *   out[t] = bf16( shared_out[t] + bf16( acc * routed_scaling_factor ) )
 * shared_out, out (m, d) bf16; expert_out (m, top_k, d) bf16; weights (m, top_k) fp32. */
int amla_moe_combine(const void *shared_out, const void *expert_out, const float *weights, int64_t m, int top_k,
                     int64_t d, float routed_scaling_factor, void *out, void *stream);

/* ---- output head ---- */

/* The lm_head projection of forward.py:70-72 (hidden.float() @ lm_head_w.float().T):
 *   logits[i, j] = sum_k f32(x[i, k]) * f32(weight[j, k])   (fp32 sums of exact products)
 * x (m, k) bf16; weight (n, k) bf16 (k % 32 == 0); logits (m, n) fp32 with row stride ld_logits. */
int amla_bf16_logits(const void *x, int64_t m, int64_t k, const void *weight, int64_t n, float *logits,
                     int64_t ld_logits, void *stream);

/* sample(logits, temperature=0, ...) of engine.py:166-173: out[r] = index of the largest
 * logits[r, :] (ties to the lower index).  logits (rows, n) fp32, row stride ld; out int64. */
int amla_argmax(const float *logits, int64_t rows, int64_t n, int64_t ld, int64_t *out, void *stream);

/* sample(logits, temperature, top_p) of engine.py:166-186 for temperature > 0:
 * p = softmax(logits / temperature); sorted by p descending, a token is dropped when the
 * mass strictly before it exceeds top_p (equal probabilities in vocabulary order, the order of
 * a stable sort: of the tokens tied at the threshold, the first ones are kept);
 * one token is drawn from the renormalised kept p with a counter-based generator keyed
 * by (seed, row).  Same distribution as the reference's torch.multinomial, not the same
 * random stream: the masses are summed in 2^-40 fixed point (integer sums, independent of
 * the order of the additions), u = floor(K * r / 2^64) for the kept mass K and a 64-bit
 * random r, and the token is the first kept one in vocabulary order whose running kept
 * mass exceeds u.  One workgroup per row. */
int amla_sample_top_p(const float *logits, int64_t rows, int64_t n, int64_t ld, float temperature, float top_p,
                      uint64_t seed, int64_t *out, void *stream);

/* sample(logits, temperature, top_p) of engine.py:166-186 with each row cut into chunks
 * (rows x chunks workgroups fill the device): temperature 0 gives amla_argmax's result,
 * temperature > 0 amla_sample_top_p's result for the same seed (the same token).
 * Workspace of amla_sample_workspace_bytes(rows, n) bytes, 256-byte aligned; scratch only,
 * nothing needs clearing; calls that share a workspace must be ordered on one stream. */
int amla_sample(const float *logits, int64_t rows, int64_t n, int64_t ld, float temperature, float top_p,
                uint64_t seed, int64_t *out, void *workspace, size_t workspace_bytes, void *stream);
size_t amla_sample_workspace_bytes(int64_t rows, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* AMLA_H_ */
