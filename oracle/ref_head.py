"""CPU oracle for the output head: inference/forward.py:67-72 (final norm + lm_head) and
the deterministic part of inference/engine.py:166-186 (sample).

TEST INFRASTRUCTURE ONLY: used by tests/ to check results, never as a fallback.

``sample`` draws with torch.multinomial, so its random stream cannot be matched;
the oracle restates what the draw is taken from (``nucleus``: the kept tokens and
their renormalised probabilities) and the greedy path (temperature 0 -> argmax).

Pinning (tests/test_oracle_head.py): top_p = 0 keeps only the maximum, top_p >= 1
keeps every token, hand-worked four- and five-token examples (the second with tied
probabilities), and the kept set equals the "mass strictly before the token <= top_p"
rule computed in float64 on random rows, with and without ties.
"""
from __future__ import annotations

import torch

from .ref_ops import rms_norm


def lm_head_logits(hidden: torch.Tensor, final_norm: torch.Tensor, lm_head_w: torch.Tensor, eps: float) -> torch.Tensor:
    """forward.py:67-72: rms_norm then fp32 matmul against the bf16 lm_head."""
    h = rms_norm(hidden, final_norm, eps)
    return h.float() @ lm_head_w.float().T


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """engine.py:172-173."""
    return logits.argmax(dim=-1)


def nucleus(logits: torch.Tensor, temperature: float, top_p: float) -> tuple[torch.Tensor, torch.Tensor]:
    """engine.py:175-182: (kept mask in vocabulary order, renormalised probabilities in vocabulary order)."""
    probs = torch.softmax(logits / temperature, dim=-1)                     # :175
    # :178 calls sort without stable=True, which leaves the order of equal probabilities open
    # (torch's CPU sort does not keep them in vocabulary order); the oracle fixes it as the
    # vocabulary order, so that ties at the threshold keep a definite set of tokens
    sorted_probs, sorted_indices = probs.sort(dim=-1, descending=True, stable=True)
    cumulative = sorted_probs.cumsum(dim=-1)                                # :179
    mask = cumulative - sorted_probs > top_p                                # :180
    sorted_probs[mask] = 0.0                                                # :181
    sorted_probs /= sorted_probs.sum(dim=-1, keepdim=True)                  # :182
    kept = torch.zeros_like(probs, dtype=torch.bool).scatter(-1, sorted_indices, ~mask)
    p = torch.zeros_like(probs).scatter(-1, sorted_indices, sorted_probs)
    return kept, p
