"""Model hyper-parameters the MLA path reads.

Mirrors the frozen dataclass of inference/config.py:6-52 (same field names and
defaults, DeepSeek-R1-0528 values), so a caller may pass either that object or
this one to :func:`amla.ops.mla_attention`.  Only these fields are read on the
path: hidden_size, num_attention_heads, q_lora_rank, kv_lora_rank,
qk_nope_head_dim, qk_rope_head_dim, v_head_dim, qk_head_dim, rope_theta,
rope_scaling_factor, rope_scaling_beta_fast, rope_scaling_beta_slow,
rope_scaling_mscale_all_dim, original_max_position_embeddings, rms_norm_eps.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class DeepSeekConfig:
    hidden_size: int = 7168
    num_layers: int = 61
    num_attention_heads: int = 128
    num_key_value_heads: int = 128
    vocab_size: int = 129280

    q_lora_rank: int = 1536
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    qk_head_dim: int = 192

    rope_theta: float = 10000.0
    max_position_embeddings: int = 163840
    rope_scaling_factor: float = 40.0
    rope_scaling_beta_fast: int = 32
    rope_scaling_beta_slow: int = 1
    rope_scaling_mscale: float = 1.0
    rope_scaling_mscale_all_dim: float = 1.0
    original_max_position_embeddings: int = 4096

    n_routed_experts: int = 256
    num_experts_per_tok: int = 8
    n_group: int = 8
    topk_group: int = 4
    moe_intermediate_size: int = 2048
    routed_scaling_factor: float = 2.5
    norm_topk_prob: bool = True

    intermediate_size: int = 18432
    first_k_dense_replace: int = 3
    n_shared_experts: int = 1

    rms_norm_eps: float = 1e-6
    fp8_block_size: int = 128
