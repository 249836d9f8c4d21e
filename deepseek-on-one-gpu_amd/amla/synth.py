"""Seeded synthetic inputs of DeepSeek-R1 MLA shape.

The reference loads real checkpoint tensors (inference/weight_store.py:208-226);
there is no network here, so every input is generated:

* weights N(0, 0.02) in fp32, quantised per 128x128 block to float8_e4m3fn with
  ``scale_inv = amax / 448`` (fp32) and ``clamp(w / scale_inv, -448, 448)`` cast
  with round-to-nearest-even (torch's cast maps |v| > 464 to NaN, hence the clamp);
* norm weights (gamma) bf16 ``1 + 0.1 N(0,1)`` (or all ones);
* hidden states and latent/rope cache rows N(0,1) rounded to bf16.

Every tensor has its own seed, derived from sha256 of a name path, so one layer's
tensors never depend on how many other tensors were drawn before.  CPU generation
(torch.Generator on "cpu") is deterministic across x86 hosts; GPU generation is
used only for large benchmark stacks where no CPU check reads the values.
"""
from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

import torch

from .config import DeepSeekConfig

FP8_MAX = 448.0
BLOCK = 128

# (name, rows, cols) of the five block-FP8 projections, in DeepSeek-R1 layout
# (weight is (out_features, in_features), as in inference/ops.py:23-24).
def projection_shapes(cfg: DeepSeekConfig) -> dict[str, tuple[int, int]]:
    H = cfg.num_attention_heads
    return {
        "q_a_proj": (cfg.q_lora_rank, cfg.hidden_size),
        "q_b_proj": (H * cfg.qk_head_dim, cfg.q_lora_rank),
        "kv_a_proj_with_mqa": (cfg.kv_lora_rank + cfg.qk_rope_head_dim, cfg.hidden_size),
        "kv_b_proj": (H * (cfg.qk_nope_head_dim + cfg.v_head_dim), cfg.kv_lora_rank),
        "o_proj": (cfg.hidden_size, H * cfg.v_head_dim),
    }


def seed_of(*parts) -> int:
    """63-bit seed from sha256 of the '/'-joined name path."""
    h = hashlib.sha256("/".join(str(p) for p in parts).encode()).digest()
    return int.from_bytes(h[:8], "little") & ((1 << 63) - 1)


def randn(shape, seed: int, std: float = 1.0, device="cpu") -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn(tuple(shape), generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t


def quantize_fp8_blocks(w: torch.Tensor, block: int = BLOCK):
    """fp32 (N, K) -> (float8_e4m3fn (N, K), fp32 scale_inv (ceil(N/b), ceil(K/b)))."""
    assert w.dim() == 2 and w.dtype == torch.float32
    N, K = w.shape
    nb, kb = math.ceil(N / block), math.ceil(K / block)
    pad = torch.zeros(nb * block, kb * block, dtype=torch.float32, device=w.device)
    pad[:N, :K] = w
    blocks = pad.view(nb, block, kb, block)
    amax = blocks.abs().amax(dim=(1, 3))                      # (nb, kb)
    scale = amax / FP8_MAX
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = (blocks / scale[:, None, :, None]).clamp_(-FP8_MAX, FP8_MAX)
    q = q.view(nb * block, kb * block)[:N, :K].to(torch.float8_e4m3fn).contiguous()
    return q, scale.contiguous()


def gamma(n: int, seed: int, mode: str = "perturbed", device="cpu") -> torch.Tensor:
    if mode == "ones":
        return torch.ones(n, dtype=torch.bfloat16, device=device)
    return (1.0 + randn((n,), seed, 0.1, device)).to(torch.bfloat16)


@dataclass
class LayerInputs:
    attn_weights: dict            # inference/weight_store.py:208-226 key contract
    input_layernorm: torch.Tensor


def make_layer(cfg: DeepSeekConfig, tag: str, layer: int = 0, device="cpu",
               gamma_mode: str = "perturbed", std: float = 0.02) -> LayerInputs:
    """One layer's MLA weights in the ``attn_weights`` dict format.

    Keys: q_a_proj, q_b_proj, kv_a_proj_with_mqa, kv_b_proj, o_proj ->
    (weight fp8, weight_scale_inv fp32); q_a_layernorm, kv_a_layernorm -> bf16.
    """
    aw = {}
    for name, (n, k) in projection_shapes(cfg).items():
        w = randn((n, k), seed_of(tag, layer, name), std, device)
        aw[name] = quantize_fp8_blocks(w)
        del w
    aw["q_a_layernorm"] = gamma(cfg.q_lora_rank, seed_of(tag, layer, "q_a_layernorm"), gamma_mode, device)
    aw["kv_a_layernorm"] = gamma(cfg.kv_lora_rank, seed_of(tag, layer, "kv_a_layernorm"), gamma_mode, device)
    ln = gamma(cfg.hidden_size, seed_of(tag, layer, "input_layernorm"), gamma_mode, device)
    return LayerInputs(aw, ln)


def make_hidden(cfg: DeepSeekConfig, B: int, S: int, tag: str, device="cpu") -> torch.Tensor:
    return randn((B, S, cfg.hidden_size), seed_of(tag, "hidden"), 1.0, device).to(torch.bfloat16)


def make_kv_cache(cfg: DeepSeekConfig, B: int, max_seq: int, filled, tag: str, layer: int = 0,
                  device="cpu"):
    """(ckv (B,max_seq,kv_lora), kpe (B,max_seq,rope)) bf16.

    Rows [0, filled[b]) of sequence b are N(0,1); the rest stay zero, as the
    engine's zero-initialised cache (inference/engine.py:72-87).
    """
    if isinstance(filled, int):
        filled = [filled] * B
    ckv = torch.zeros(B, max_seq, cfg.kv_lora_rank, dtype=torch.bfloat16, device=device)
    kpe = torch.zeros(B, max_seq, cfg.qk_rope_head_dim, dtype=torch.bfloat16, device=device)
    for b, L in enumerate(filled):
        if L > 0:
            ckv[b, :L] = randn((L, cfg.kv_lora_rank), seed_of(tag, layer, "ckv", b), 1.0, device).to(torch.bfloat16)
            kpe[b, :L] = randn((L, cfg.qk_rope_head_dim), seed_of(tag, layer, "kpe", b), 1.0, device).to(torch.bfloat16)
    return ckv, kpe


def ragged_lengths(B: int, lo: int, hi: int, tag: str) -> list[int]:
    """Per-sequence context lengths drawn uniform in [lo, hi] from a named seed."""
    g = torch.Generator().manual_seed(seed_of(tag, "lengths"))
    return torch.randint(lo, hi + 1, (B,), generator=g).tolist()


def sha256_of(t: torch.Tensor) -> str:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float8_e4m3fn):
        t = t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()
