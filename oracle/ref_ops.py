"""CPU oracle for the MLA + block-FP8 path: a restatement of inference/ops.py:10-183.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module;
it is used by tests/, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline``
leg of bench.py, and there only to check results (or as the timed CPU baseline),
never as a fallback for the GPU path.

Each function follows the reference's torch op sequence step by step, because
the reference's numerics are defined by its rounding points (bf16 after every
fp8 linear, two roundings in rms_norm, bf16 RoPE output, bf16 scores rounded
again by the scale multiply, fp32 mask add for S>1, fp32 softmax stored as bf16,
bf16 P@V).  Layout changes that the reference makes with einops.rearrange are
made here with view/permute, which is what rearrange lowers to.

Pinning (checked by tests/test_oracle.py):
* fp8_block_dequant: brute force over all 256 e4m3fn codes against the C
  restatement of the OCP decode table (oracle/fp8_ref.c), bit patterns compared.
* fp8_linear: fp64 brute force; identity / one-hot weights give exact outputs.
* rms_norm: closed form; constant rows; gamma = 1.
* yarn_get_mscale: closed form 0.1*ln(40)+1.
* precompute_rope_freqs / apply_rope / mla_attention: golden vectors written by
  tests/golden/make_golden.py from the reference's own functions, plus closed
  forms (factor 1 -> textbook RoPE, |z| = 1, position 0 is the identity) and the
  invariants of truth.py (naive == absorbed in fp64, T = 1, uniform rows).
"""
from __future__ import annotations

import math

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """inference/ops.py:10-12: fp32 mean-square -> rsqrt -> x*r rounded to x.dtype -> *weight."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    normed = (xf * inv).to(x.dtype)
    return normed * weight


def fp8_block_dequant(weight: torch.Tensor, scale_inv: torch.Tensor, block: int = 128) -> torch.Tensor:
    """inference/ops.py:30-43: w_f32[i, j] = f32(weight[i, j]) * scale_inv[i // 128, j // 128].

    The reference expands scale_inv with repeat_interleave and trims to the
    weight shape; indexing with i // 128, j // 128 selects the same entries.
    """
    n, k = weight.shape
    r = torch.arange(n) // block
    c = torch.arange(k) // block
    expanded = scale_inv[r][:, c]
    return weight.float() * expanded


def fp8_linear(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor,
               out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """inference/ops.py:15-44: fp32 GEMM against the dequantised weight, output cast to out_dtype."""
    w = fp8_block_dequant(weight, scale_inv)
    return (x.float() @ w.T).to(out_dtype)


def yarn_get_mscale(scale: float = 1.0, mscale: float = 1.0) -> float:
    """inference/ops.py:47-50."""
    return 1.0 if scale <= 1.0 else 0.1 * mscale * math.log(scale) + 1.0


def yarn_ramp_bounds(cfg) -> tuple[int, int]:
    """The integer ramp ends of inference/ops.py:69-70 (R1: low 10, high 23)."""
    dim = cfg.qk_rope_head_dim
    base = cfg.rope_theta
    omax = cfg.original_max_position_embeddings

    def edge(beta):
        return dim * math.log(omax / (beta * 2 * math.pi)) / (2 * math.log(base))

    low = max(math.floor(edge(cfg.rope_scaling_beta_fast)), 0)
    high = min(math.ceil(edge(cfg.rope_scaling_beta_slow)), dim // 2 - 1)
    return low, high


def yarn_inv_freq(cfg) -> torch.Tensor:
    """fp32 per-pair frequencies after the YaRN blend (inference/ops.py:66-78)."""
    dim = cfg.qk_rope_head_dim
    base = cfg.rope_theta
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    low, high = yarn_ramp_bounds(cfg)
    ramp = torch.ones(dim // 2, dtype=torch.float32)
    if high > low:
        idx = torch.arange(dim // 2, dtype=torch.float32)
        ramp = ((idx - low) / (high - low)).clamp(0.0, 1.0)
    return inv * (1.0 - ramp) + (inv / cfg.rope_scaling_factor) * ramp


def precompute_rope_freqs(cfg, seq_len: int, device="cpu") -> torch.Tensor:
    """inference/ops.py:53-83: complex64 (seq_len, dim/2) = polar(1, t * f_i)."""
    f = yarn_inv_freq(cfg)
    t = torch.arange(seq_len, dtype=torch.float32)
    ang = torch.outer(t, f)
    return torch.polar(torch.ones_like(ang), ang).to(device)


def apply_rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """inference/ops.py:86-97: rotate interleaved pairs (2i, 2i+1) by freqs, fp32 math, cast back."""
    pairs = torch.view_as_complex(x.float().reshape(*x.shape[:-1], -1, 2))
    rot = pairs * freqs[None, None]
    return torch.view_as_real(rot).flatten(-2).to(x.dtype)


def _split_heads(t: torch.Tensor, H: int) -> torch.Tensor:
    """'B S (H D) -> B H S D' as a view + permute."""
    B, S, HD = t.shape
    return t.view(B, S, H, HD // H).permute(0, 2, 1, 3)


def mla_attention(hidden, attn_weights, kv_cache, position: int, rope_freqs, cfg) -> torch.Tensor:
    """inference/ops.py:100-183 (naive MLA; mutates kv_cache rows [position, position+S))."""
    return mla_attention_parts(hidden, attn_weights, kv_cache, position, rope_freqs, cfg)[1]


def mla_attention_parts(hidden, attn_weights, kv_cache, position: int, rope_freqs, cfg):
    """inference/ops.py:100-183 returning (per-head output before o_proj (B, S, H*v), final output).

    The first tensor is the ``out`` of inference/ops.py:182 (heads-major
    columns h*v_head_dim + d), the input of the o_proj linear at :183.
    """
    B, S, _ = hidden.shape
    H = cfg.num_attention_heads
    nope, rope_d, vd, lora = cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.v_head_dim, cfg.kv_lora_rank
    ckv_cache, kpe_cache = kv_cache

    # query: q_a -> norm -> q_b, heads of (nope | rope)      ops.py:129-133
    qa = fp8_linear(hidden, *attn_weights["q_a_proj"])
    qa = rms_norm(qa, attn_weights["q_a_layernorm"], cfg.rms_norm_eps)
    q = _split_heads(fp8_linear(qa, *attn_weights["q_b_proj"]), H)
    q_nope, q_pe = q.split([nope, rope_d], dim=-1)

    # latent + rope key of the new tokens, stored raw          ops.py:136-141
    kva = fp8_linear(hidden, *attn_weights["kv_a_proj_with_mqa"])
    c_new, kpe_new = kva.split([lora, rope_d], dim=-1)
    ckv_cache[:B, position:position + S] = c_new
    kpe_cache[:B, position:position + S] = kpe_new
    T = position + S
    c_all = ckv_cache[:B, :T]
    kpe_all = kpe_cache[:B, :T]

    # decompress every cached row through kv_b                 ops.py:148-151
    c_normed = rms_norm(c_all, attn_weights["kv_a_layernorm"], cfg.rms_norm_eps)
    kvb = _split_heads(fp8_linear(c_normed, *attn_weights["kv_b_proj"]), H)
    k_nope, v = kvb.split([nope, vd], dim=-1)

    # RoPE on q at its positions and on every cached k_pe row   ops.py:154-159
    q_pe = apply_rope(q_pe, rope_freqs[position:T])
    kpe_heads = kpe_all.view(B, 1, T, rope_d).expand(-1, H, -1, -1)
    kpe_heads = apply_rope(kpe_heads, rope_freqs[:T])

    q_full = torch.cat([q_nope, q_pe], dim=-1)
    k_full = torch.cat([k_nope, kpe_heads], dim=-1)

    # scores in bf16, scaled once by mscale/sqrt(qk_head_dim)  ops.py:166-169
    scale = yarn_get_mscale(cfg.rope_scaling_factor, cfg.rope_scaling_mscale_all_dim) / math.sqrt(cfg.qk_head_dim)
    scores = torch.matmul(q_full, k_full.transpose(-2, -1)) * scale

    if S > 1:                                                  # ops.py:172-177
        mask = torch.triu(torch.full((S, T), float("-inf"), device=hidden.device), diagonal=position + 1)
        scores = scores + mask[None, None]

    probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(hidden.dtype)   # ops.py:179
    out = torch.matmul(probs, v)                                                 # ops.py:180
    out = out.permute(0, 2, 1, 3).reshape(B, S, H * vd)                          # ops.py:182
    return out, fp8_linear(out, *attn_weights["o_proj"])                         # ops.py:183


def mla_attention_per_sequence(hidden, attn_weights, kv_cache, positions, rope_freqs, cfg) -> torch.Tensor:
    """Ragged batch (one position per sequence) as a loop of B = 1 reference calls.

    The reference's ``position`` is one int for the whole batch
    (inference/ops.py:104, :140-145), so per-sequence positions can only be
    expressed as this loop.
    """
    return mla_attention_per_sequence_parts(hidden, attn_weights, kv_cache, positions, rope_freqs, cfg)[1]


def mla_attention_per_sequence_parts(hidden, attn_weights, kv_cache, positions, rope_freqs, cfg):
    """mla_attention_per_sequence returning (per-head output before o_proj, final output)."""
    ckv, kpe = kv_cache
    heads, outs = [], []
    for b, p in enumerate(positions):
        a, o = mla_attention_parts(hidden[b:b + 1], attn_weights, (ckv[b:b + 1], kpe[b:b + 1]), int(p),
                                   rope_freqs, cfg)
        heads.append(a)
        outs.append(o)
    return torch.cat(heads, dim=0), torch.cat(outs, dim=0)


def transformer_layer_attention(hidden, input_layernorm, attn_weights, kv_cache, position, rope_freqs, cfg):
    """inference/forward.py:92-94: hidden + mla_attention(rms_norm(hidden)) with a bf16 residual add."""
    normed = rms_norm(hidden, input_layernorm, cfg.rms_norm_eps)
    return hidden + mla_attention(normed, attn_weights, kv_cache, position, rope_freqs, cfg)
