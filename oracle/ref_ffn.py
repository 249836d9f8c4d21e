"""CPU oracle for the FFN / MoE path: a restatement of inference/ops.py:186-257 and
inference/forward.py:112-153.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this module;
tests/ and the bench's CPU leg use it to check results, never as a fallback.

The reference's numerics are defined by its rounding points, so each function
follows its op sequence: every fp8 linear returns bf16, F.silu on a bf16 tensor
computes x / (1 + exp(-x)) in fp32 and rounds to bf16, the gate*up product is
rounded to bf16, routing runs in fp32 (logits, sigmoid, top-k, normalisation),
and the MoE combine accumulates each token's expert outputs into a bf16 buffer
one expert at a time (the fp32 routing weight is cast to the bf16 of the
expert output before the multiply, as a 0-dim device tensor is in the
reference's elementwise ops), then adds routed * routed_scaling_factor to the
shared expert's output in bf16.

Pinning (tests/test_oracle_ffn.py):
* swiglu: one-hot fp8 weights turn every linear into an exact selection, so the
  output is silu/mul of chosen inputs, checked against float64 closed forms.
* route: the chosen groups and experts are checked against an independent
  numpy float64 formulation (sort the groups by their maximum, then the experts
  of the chosen groups by score; no masking), on random logits and on
  constructed cases where the group limit changes the answer; normalised
  weights sum to one.
* moe_block: zero routed weights leave the shared expert's output; a single
  expert per token reduces to w * expert(x) + shared in the stated roundings.
"""
from __future__ import annotations

from typing import Callable, Mapping

import torch

from .ref_ops import fp8_linear

Pair = tuple[torch.Tensor, torch.Tensor]


def silu_bf16(x: torch.Tensor) -> torch.Tensor:
    """F.silu on a bf16 tensor: fp32 x / (1 + exp(-x)), rounded to bf16."""
    xf = x.float()
    return (xf / (1.0 + torch.exp(-xf))).to(x.dtype)


def swiglu(x, gate_proj, gate_scale, up_proj, up_scale, down_proj, down_scale) -> torch.Tensor:
    """inference/ops.py:186-192: down(silu(gate(x)) * up(x)), every linear rounded to bf16."""
    gate = silu_bf16(fp8_linear(x, gate_proj, gate_scale))
    up = fp8_linear(x, up_proj, up_scale)
    return fp8_linear(gate * up, down_proj, down_scale)


def dense_ffn(hidden: torch.Tensor, mlp_weights: Mapping[str, Pair]) -> torch.Tensor:
    """inference/ops.py:195-199."""
    return swiglu(hidden, *mlp_weights["gate_proj"], *mlp_weights["up_proj"], *mlp_weights["down_proj"])


def expert_ffn(hidden: torch.Tensor, expert_weights: Mapping[str, Pair]) -> torch.Tensor:
    """inference/ops.py:202-206."""
    return swiglu(hidden, *expert_weights["gate_proj"], *expert_weights["up_proj"], *expert_weights["down_proj"])


def route(hidden: torch.Tensor, gate_weight: torch.Tensor, cfg) -> tuple[torch.Tensor, torch.Tensor]:
    """inference/ops.py:209-257: sigmoid scores, group-limited top-k, optional normalisation."""
    logits = hidden.float() @ gate_weight.float().T                       # :224
    scores = torch.sigmoid(logits)                                         # :225
    n_experts, n_group = cfg.n_routed_experts, cfg.n_group
    group_size = n_experts // n_group
    grouped = scores.view(*scores.shape[:-1], n_group, group_size)         # :236
    group_scores = grouped.max(dim=-1).values                              # :239
    top_groups = group_scores.topk(cfg.topk_group, dim=-1).indices        # :240
    group_mask = torch.zeros_like(group_scores, dtype=torch.bool)
    group_mask.scatter_(-1, top_groups, True)                              # :244
    expert_mask = group_mask.unsqueeze(-1).expand_as(grouped)
    masked = grouped.where(expert_mask, torch.tensor(0.0)).view(*scores.shape[:-1], n_experts)  # :247-248
    topk_w, topk_i = masked.topk(cfg.num_experts_per_tok, dim=-1)          # :251
    if cfg.norm_topk_prob:
        topk_w = topk_w / (topk_w.sum(dim=-1, keepdim=True) + 1e-9)        # :254-255
    return topk_i, topk_w


def moe_block(hidden: torch.Tensor, gate_weight: torch.Tensor, shared_weights: Mapping[str, Pair],
              experts: Callable[[int], Mapping[str, Pair]], cfg) -> torch.Tensor:
    """inference/forward.py:112-153 with the experts handed in (no host streaming).

    experts(e) returns the weights of routed expert e.
    """
    idx, w = route(hidden, gate_weight, cfg)                               # :122
    shared_out = expert_ffn(hidden, shared_weights)                        # :134
    B, S, top_k = idx.shape
    routed = torch.zeros_like(hidden)                                      # :138
    for b in range(B):
        for s in range(S):
            tok = hidden[b, s].unsqueeze(0).unsqueeze(0)
            for k in range(top_k):
                e_out = expert_ffn(tok, experts(int(idx[b, s, k]))).squeeze(0).squeeze(0)
                wk = w[b, s, k].to(e_out.dtype)
                routed[b, s] += wk * e_out                                 # :151
    return shared_out + routed * cfg.routed_scaling_factor                 # :153
