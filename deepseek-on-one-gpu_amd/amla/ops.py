"""MLA-path operators with the reference's signatures, on gfx950 HIP kernels.

Drop-in for the MLA half of inference/ops.py: ``rms_norm`` (:10-12),
``fp8_linear`` (:15-44), ``yarn_get_mscale`` (:47-50), ``precompute_rope_freqs``
(:53-83), ``apply_rope`` (:86-97) and ``mla_attention`` (:100-183), plus the
attention half of ``transformer_layer`` (inference/forward.py:92-94) as
``mla_layer``; and the FFN / MoE functions on the same fp8 kernels: ``swiglu``
(:186-192), ``dense_ffn`` / ``expert_ffn`` (:195-206), ``route`` (:209-257) and
``moe_block`` (inference/forward.py:112-153, experts handed in).  Same argument
names, tensor layouts and dtypes; tensors must be
on a ROCm device.  Every compute call goes to libamla.so; there is no CPU or
PyTorch fallback (a missing library raises).

Superset over the reference: ``position`` of ``mla_attention`` may also be a
list of per-sequence start positions or an int32 device tensor of them (the
reference's scalar position cannot express a ragged batch).
"""
from __future__ import annotations

import ctypes
import math
from typing import Sequence

import torch

from . import _lib, torch_ops
from ._lib import check, lib

BF16 = torch.bfloat16
FP8 = torch.float8_e4m3fn


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a tensor on a ROCm device")


def _need(t: torch.Tensor, name: str, dtype, dev=None) -> None:
    _need_cuda(t, name)
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if dev is not None and t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ------------------------------------------------------------------ workspace

def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for one call, from torch's caching allocator on the current stream.

    A fresh buffer per call: inside a HIP graph capture it comes from the
    graph's private pool (a replay never touches memory another call owns),
    and calls on different streams never share it.
    """
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


# ------------------------------------------------------------------ elementwise / linear

def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """inference/ops.py:10-12: y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)."""
    _need_cuda(x, "x")
    if x.dtype != BF16 or weight.dtype != BF16:
        raise TypeError("rms_norm: x and weight must be bfloat16")
    dim = x.shape[-1]
    if weight.shape != (dim,):
        raise ValueError(f"rms_norm: weight shape {tuple(weight.shape)} != ({dim},)")
    xc = x.contiguous()
    w = weight.contiguous()
    rows = xc.numel() // dim if dim else 0
    return torch.ops.amla.rms_norm(xc.view(rows, dim), w, float(eps)).view(x.shape)


def fp8_block_dequant(weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """inference/ops.py:30-43: fp32 f32(weight) * scale_inv[i//128, j//128], bit-exact."""
    _need(weight, "weight", FP8)
    _need(scale_inv, "scale_inv", torch.float32, weight.device)
    n, k = weight.shape
    if scale_inv.shape != (math.ceil(n / 128), math.ceil(k / 128)):
        raise ValueError(f"scale_inv shape {tuple(scale_inv.shape)} does not match weight {n}x{k}")
    out = torch.empty(n, k, dtype=torch.float32, device=weight.device)
    check(lib().amla_fp8_block_dequant(weight.data_ptr(), scale_inv.data_ptr(), n, k, out.data_ptr(),
                                       _stream_ptr(weight)), "fp8_block_dequant")
    return out


def fp8_linear(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor,
               out_dtype: torch.dtype = BF16) -> torch.Tensor:
    """inference/ops.py:15-44: ( x @ dequant(weight, scale_inv).T ).to(out_dtype), fp32 accumulation.

    bf16 rounds in the kernel's epilogue (``torch.ops.amla.fp8_linear``); any other out_dtype
    takes the fp32 result (``torch.ops.amla.fp8_linear_f32``) cast with ``.to(out_dtype)`` as the
    reference does."""
    _need_cuda(x, "x")
    if x.dtype != BF16:
        raise TypeError(f"fp8_linear: x must be bfloat16 (got {x.dtype})")
    if not isinstance(out_dtype, torch.dtype) or not (out_dtype.is_floating_point or out_dtype.is_complex):
        raise TypeError(f"fp8_linear: out_dtype must be a floating-point dtype (got {out_dtype})")
    _need(weight, "weight", FP8, x.device)
    _need(scale_inv, "scale_inv", torch.float32, x.device)
    n, k = weight.shape
    if x.shape[-1] != k:
        raise ValueError(f"fp8_linear: x has {x.shape[-1]} features, weight expects {k}")
    if scale_inv.shape != (math.ceil(n / 128), math.ceil(k / 128)):
        raise ValueError(f"scale_inv shape {tuple(scale_inv.shape)} does not match weight {n}x{k}")
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    if out_dtype == BF16:
        return torch.ops.amla.fp8_linear(x2, weight, scale_inv).view(*x.shape[:-1], n)
    y = torch.ops.amla.fp8_linear_f32(x2, weight, scale_inv).view(*x.shape[:-1], n)
    return y if out_dtype == torch.float32 else y.to(out_dtype)


# ------------------------------------------------------------------ RoPE

def yarn_get_mscale(scale: float = 1.0, mscale: float = 1.0) -> float:
    """inference/ops.py:47-50 (host scalar)."""
    if scale <= 1.0:
        return 1.0
    return 0.1 * mscale * math.log(scale) + 1.0


def precompute_rope_freqs(config, seq_len: int, device) -> torch.Tensor:
    """inference/ops.py:53-83: YaRN-blended frequencies, complex64 (seq_len, rope/2).

    One-time table set-up (the engine builds it once, inference/engine.py:63):
    computed with fp32 torch ops in the same order as the reference, so the
    table is bit-identical, then moved to ``device``.
    """
    dim = config.qk_rope_head_dim
    base = config.rope_theta
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))

    def edge(beta):
        return dim * math.log(config.original_max_position_embeddings / (beta * 2 * math.pi)) / (2 * math.log(base))

    low = max(math.floor(edge(config.rope_scaling_beta_fast)), 0)
    high = min(math.ceil(edge(config.rope_scaling_beta_slow)), dim // 2 - 1)
    ramp = torch.ones(dim // 2, dtype=torch.float32)
    if high > low:
        ramp = ((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low)).clamp(0.0, 1.0)
    inv = inv * (1.0 - ramp) + (inv / config.rope_scaling_factor) * ramp
    ang = torch.outer(torch.arange(seq_len, dtype=torch.float32), inv)
    return torch.polar(torch.ones_like(ang), ang).to(device)


def apply_rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """inference/ops.py:86-97: x (B, H, S, rope) bf16, freqs (S, rope/2) complex64."""
    _need_cuda(x, "x")
    if x.dtype != BF16:
        raise TypeError("apply_rope: x must be bfloat16")
    if freqs.dtype != torch.complex64 or freqs.device != x.device:
        raise TypeError("apply_rope: freqs must be complex64 on the same device")
    S, dim = x.shape[-2], x.shape[-1]
    if freqs.shape != (S, dim // 2):
        raise ValueError(f"apply_rope: freqs shape {tuple(freqs.shape)} != ({S}, {dim // 2})")
    xc = x.contiguous()
    groups = xc.numel() // (S * dim) if S * dim else 0
    return torch.ops.amla.apply_rope(xc.view(groups, S, dim), freqs.contiguous()).view(x.shape)


# ------------------------------------------------------------------ MLA

def softmax_scale(config) -> float:
    """mscale / sqrt(qk_head_dim), mscale applied once (inference/ops.py:166-167)."""
    return yarn_get_mscale(config.rope_scaling_factor, config.rope_scaling_mscale_all_dim) / math.sqrt(
        config.qk_head_dim)


def _positions(position, B: int, S: int, device, max_context):
    """(int32 device tensor (B,), max position+S or None) from an int, a sequence or a tensor."""
    if isinstance(position, torch.Tensor):
        if position.dtype != torch.int32 or position.device != device or position.shape != (B,):
            raise ValueError("position tensor must be int32 (B,) on the hidden states' device")
        return position, max_context
    if isinstance(position, int):
        if position < 0:
            raise ValueError("position must be >= 0")
        return torch.full((B,), position, dtype=torch.int32, device=device), position + S
    pos = [int(p) for p in position]
    if len(pos) != B or min(pos) < 0:
        raise ValueError("one non-negative position per sequence is required")
    return torch.tensor(pos, dtype=torch.int32, device=device), max(pos) + S


_PROJ = (("q_a_proj", "w_q_a"), ("q_b_proj", "w_q_b"), ("kv_a_proj_with_mqa", "w_kv_a"),
         ("kv_b_proj", "w_kv_b"), ("o_proj", "w_o"))


def _mla_operands(hidden, attn_weights, kv_cache, position, rope_freqs, config, *, input_gamma=None,
                  residual=None, attn_out=None, max_context=None) -> dict:
    """Validates the reference's arguments and unpacks them into the operands of
    ``torch.ops.amla.mla_decode`` / ``mla_prefill`` (raises before any launch)."""
    _need(hidden, "hidden", BF16)
    dev = hidden.device
    if hidden.dim() != 3:
        raise ValueError("hidden must be (B, S, hidden_size)")
    B, S, D = hidden.shape
    if D != config.hidden_size:
        raise ValueError(f"hidden size {D} != config.hidden_size {config.hidden_size}")
    ckv, kpe = kv_cache
    _need(ckv, "compressed_kv_cache", BF16, dev)
    _need(kpe, "k_pe_cache", BF16, dev)
    if ckv.dim() != 3 or kpe.dim() != 3 or ckv.shape[:2] != kpe.shape[:2]:
        raise ValueError("kv caches must be (B_alloc, max_seq, kv_lora) and (B_alloc, max_seq, rope)")
    if ckv.shape[0] < B or ckv.shape[2] != config.kv_lora_rank or kpe.shape[2] != config.qk_rope_head_dim:
        raise ValueError(f"kv cache shapes {tuple(ckv.shape)} / {tuple(kpe.shape)} do not fit batch {B}")
    max_seq = ckv.shape[1]
    if rope_freqs.dtype != torch.complex64 or rope_freqs.device != dev or not rope_freqs.is_contiguous():
        raise TypeError("rope_freqs must be a contiguous complex64 tensor on the same device")
    if rope_freqs.dim() != 2 or rope_freqs.shape[1] != config.qk_rope_head_dim // 2:
        raise ValueError("rope_freqs must have qk_rope_head_dim/2 columns")
    pos_t, mc = _positions(position, B, S, dev, max_context)
    if mc is None:
        mc = min(max_seq, rope_freqs.shape[0])
    if mc > max_seq:
        raise ValueError(f"position + seq_len = {mc} exceeds the cache length {max_seq}")
    if mc > rope_freqs.shape[0]:
        raise ValueError(f"position + seq_len = {mc} exceeds the rope table length {rope_freqs.shape[0]}")
    if mc < S:
        raise ValueError(f"max_context {mc} is below seq_len {S}")
    H = config.num_attention_heads
    shapes = {
        "q_a_proj": (config.q_lora_rank, D),
        "q_b_proj": (H * config.qk_head_dim, config.q_lora_rank),
        "kv_a_proj_with_mqa": (config.kv_lora_rank + config.qk_rope_head_dim, D),
        "kv_b_proj": (H * (config.qk_nope_head_dim + config.v_head_dim), config.kv_lora_rank),
        "o_proj": (D, H * config.v_head_dim),
    }
    ops = {"hidden": hidden}
    for name, field in _PROJ:
        w, sc = attn_weights[name]
        _need(w, f"{name}.weight", FP8, dev)
        _need(sc, f"{name}.weight_scale_inv", torch.float32, dev)
        n, k = shapes[name]
        if tuple(w.shape) != (n, k) or tuple(sc.shape) != (math.ceil(n / 128), math.ceil(k / 128)):
            raise ValueError(f"{name}: weight {tuple(w.shape)} / scale {tuple(sc.shape)} do not match ({n}, {k})")
        ops[field] = w
        ops["s" + field[1:]] = sc
    gq, gkv = attn_weights["q_a_layernorm"], attn_weights["kv_a_layernorm"]
    _need(gq, "q_a_layernorm", BF16, dev)
    _need(gkv, "kv_a_layernorm", BF16, dev)
    if gq.shape != (config.q_lora_rank,) or gkv.shape != (config.kv_lora_rank,):
        raise ValueError("q_a_layernorm / kv_a_layernorm do not match q_lora_rank / kv_lora_rank")
    if input_gamma is not None:
        _need(input_gamma, "input_layernorm", BF16, dev)
        if input_gamma.shape != (D,):
            raise ValueError("input_layernorm must be (hidden_size,)")
    if residual is not None:
        _need(residual, "residual", BF16, dev)
        if residual.shape != hidden.shape:
            raise ValueError("residual must have the hidden states' shape")
    if attn_out is not None:
        _need(attn_out, "attn_out", BF16, dev)
        if tuple(attn_out.shape) != (B, S, H * config.v_head_dim) or attn_out.data_ptr() % 16:
            raise ValueError(f"attn_out must be a 16-byte aligned (B, S, {H * config.v_head_dim}) bf16 tensor")
    ops.update(gamma_q=gq, gamma_kv=gkv, ckv_cache=ckv, kpe_cache=kpe, positions=pos_t, rope_freqs=rope_freqs,
               input_gamma=input_gamma, residual=residual, attn_out=attn_out, max_context=int(mc),
               eps=float(config.rms_norm_eps), softmax_scale=float(softmax_scale(config)), heads=H,
               qk_nope=config.qk_nope_head_dim, v_dim=config.v_head_dim)
    return ops


def _mla(ops: dict) -> torch.Tensor:
    fn = torch.ops.amla.mla_decode if ops["hidden"].shape[1] == 1 else torch.ops.amla.mla_prefill
    return fn(**ops)


def mla_attention(hidden: torch.Tensor, attn_weights: dict, kv_cache: tuple, position, rope_freqs: torch.Tensor,
                  config, *, max_context: int | None = None, attn_out: torch.Tensor | None = None) -> torch.Tensor:
    """inference/ops.py:100-183 on gfx950 (``torch.ops.amla.mla_decode`` / ``mla_prefill``).

    S == 1 runs the absorbed decode; S > 1 the kv_b decompression + causal
    flash prefill.  Writes the raw new rows into ``kv_cache`` at
    [position, position+S) like the reference.  ``max_context`` (largest
    position+S) is only needed when ``position`` is a device tensor.  When
    ``attn_out`` ((B, S, heads * v_head_dim) bf16) is given, the per-head
    attention output before o_proj is written into it.
    """
    return _mla(_mla_operands(hidden, attn_weights, kv_cache, position, rope_freqs, config,
                              max_context=max_context, attn_out=attn_out))


def mla_layer(hidden: torch.Tensor, input_layernorm: torch.Tensor, attn_weights: dict, kv_cache: tuple,
              position, rope_freqs: torch.Tensor, config, *, max_context: int | None = None,
              attn_out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention half of transformer_layer (inference/forward.py:92-94), fused:
    ``hidden + mla_attention(rms_norm(hidden, input_layernorm), ...)`` with the
    norm as the layer's first launch and the bf16 residual add in o_proj's
    epilogue."""
    return _mla(_mla_operands(hidden, attn_weights, kv_cache, position, rope_freqs, config,
                              input_gamma=input_layernorm, residual=hidden, max_context=max_context,
                              attn_out=attn_out))


# ------------------------------------------------------------------ FFN / MoE

def _fp8_pair(w: torch.Tensor, s: torch.Tensor, name: str, shape: tuple, dev) -> None:
    _need(w, name, FP8, dev)
    _need(s, name + " scale", torch.float32, dev)
    if tuple(w.shape) != shape:
        raise ValueError(f"{name}: shape {tuple(w.shape)}, expected {shape}")
    if tuple(s.shape) != (math.ceil(shape[0] / 128), math.ceil(shape[1] / 128)):
        raise ValueError(f"{name} scale: shape {tuple(s.shape)} does not match {shape}")


def swiglu(x: torch.Tensor, gate_proj: torch.Tensor, gate_scale: torch.Tensor, up_proj: torch.Tensor,
           up_scale: torch.Tensor, down_proj: torch.Tensor, down_scale: torch.Tensor) -> torch.Tensor:
    """inference/ops.py:186-192: down_proj(silu(gate_proj(x)) * up_proj(x)), every fp8 linear,
    the silu and the product rounded to bf16 as in the reference."""
    _need_cuda(x, "x")
    if x.dtype != BF16:
        raise TypeError(f"swiglu: x must be bfloat16 (got {x.dtype})")
    if gate_proj.dim() != 2:
        raise ValueError("swiglu: gate_proj must be (intermediate, hidden)")
    n, k = gate_proj.shape
    if x.shape[-1] != k:
        raise ValueError(f"swiglu: x has {x.shape[-1]} features, gate_proj expects {k}")
    _fp8_pair(gate_proj, gate_scale, "gate_proj", (n, k), x.device)
    _fp8_pair(up_proj, up_scale, "up_proj", (n, k), x.device)
    _fp8_pair(down_proj, down_scale, "down_proj", (k, n), x.device)
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    y = torch.ops.amla.swiglu(x2, gate_proj, gate_scale, up_proj, up_scale, down_proj, down_scale)
    return y.view(*x.shape[:-1], k)


def dense_ffn(hidden: torch.Tensor, mlp_weights: dict) -> torch.Tensor:
    """inference/ops.py:195-199."""
    return swiglu(hidden, *mlp_weights["gate_proj"], *mlp_weights["up_proj"], *mlp_weights["down_proj"])


def expert_ffn(hidden: torch.Tensor, expert_weights: dict) -> torch.Tensor:
    """inference/ops.py:202-206."""
    return swiglu(hidden, *expert_weights["gate_proj"], *expert_weights["up_proj"], *expert_weights["down_proj"])


def route(hidden: torch.Tensor, gate_weight: torch.Tensor, config) -> tuple[torch.Tensor, torch.Tensor]:
    """inference/ops.py:209-257: sigmoid scores, group-limited top-k, optional normalisation.

    Returns (indices int64, weights fp32), each (*hidden.shape[:-1], num_experts_per_tok).
    """
    _need_cuda(hidden, "hidden")
    if hidden.dtype != BF16:
        raise TypeError(f"route: hidden must be bfloat16 (got {hidden.dtype})")
    _need(gate_weight, "gate_weight", BF16, hidden.device)
    E, d = gate_weight.shape
    if hidden.shape[-1] != d:
        raise ValueError(f"route: hidden has {hidden.shape[-1]} features, gate_weight expects {d}")
    if E != config.n_routed_experts:
        raise ValueError(f"route: gate_weight has {E} experts, config says {config.n_routed_experts}")
    top_k = config.num_experts_per_tok
    h2 = hidden.reshape(-1, d)
    if not h2.is_contiguous() or h2.data_ptr() % 16:
        h2 = h2.contiguous()
    m = h2.shape[0]
    idx = torch.empty(m, top_k, dtype=torch.int64, device=hidden.device)
    w = torch.empty(m, top_k, dtype=torch.float32, device=hidden.device)
    if m:
        ws = workspace(hidden.device, lib().amla_moe_route_workspace_bytes(m, E))
        check(lib().amla_moe_route(h2.data_ptr(), m, d, gate_weight.data_ptr(), E, config.n_group,
                                   config.topk_group, top_k, int(bool(config.norm_topk_prob)), idx.data_ptr(),
                                   w.data_ptr(), ws.data_ptr(), ws.numel(), _stream_ptr(hidden)), "route")
    shape = (*hidden.shape[:-1], top_k)
    return idx.view(shape), w.view(shape)


_stacked_cache: dict = {}


def _stacked_key(experts: dict, E: int, d: int) -> tuple:
    return tuple((experts[k][0].data_ptr(), experts[k][1].data_ptr(), tuple(experts[k][0].shape),
                  tuple(experts[k][1].shape), experts[k][0].dtype, experts[k][1].dtype, experts[k][0].stride(),
                  experts[k][1].stride(), str(experts[k][0].device)) for k in ("gate_proj", "up_proj", "down_proj")) + (E, d)


def _stacked_expert_tables(experts: dict, E: int, d: int, dev):
    """Pointer tables of stacked expert weights (validated once per set of tensors)."""
    key = _stacked_key(experts, E, d)
    hit = _stacked_cache.get(key)
    if hit is not None:
        return hit[0], hit[1]
    tabs = []
    n_inter = experts["gate_proj"][0].shape[1]
    for key_name, shape in (("gate_proj", (E, n_inter, d)), ("up_proj", (E, n_inter, d)), ("down_proj", (E, d, n_inter))):
        wt, sc = experts[key_name]
        if wt.dtype != FP8 or sc.dtype != torch.float32 or wt.device != dev or sc.device != dev or \
                not (wt.is_contiguous() and sc.is_contiguous()):
            raise ValueError(f"moe_block: stacked {key_name} must be contiguous e4m3fn weights with fp32 scales on {dev}")
        if tuple(wt.shape) != shape or tuple(sc.shape) != (E, math.ceil(shape[1] / 128), math.ceil(shape[2] / 128)):
            raise ValueError(f"moe_block: stacked {key_name} has shape {tuple(wt.shape)} / {tuple(sc.shape)}, "
                             f"expected {shape}")
        for t in (wt, sc):
            step = t[0].numel() * t.element_size()
            tabs.append((ctypes.c_void_p * E)(*[t.data_ptr() + e * step for e in range(E)]))
    if len(_stacked_cache) > 64:
        _stacked_cache.clear()
    # [host tables, n_inter, device table (made on first use)]: one entry per full key
    # (pointers, shapes, strides, dtypes, device, E, d), so a device table is never reused for
    # other tensors that happen to start at the same addresses
    _stacked_cache[key] = [tabs, n_inter, None]
    return tabs, n_inter


def _stacked_device_table(experts: dict, E: int, d: int, dev):
    """Device pointer table [gate_w | gate_s | up_w | up_s | down_w | down_s] x E of stacked
    expert weights (amla_moe_experts_dev), made once per set of tensors and kept with the
    host tables of the same key."""
    tabs, n_inter = _stacked_expert_tables(experts, E, d, dev)
    entry = _stacked_cache[_stacked_key(experts, E, d)]
    if entry[2] is None:
        flat = [int(t[e] or 0) for t in tabs for e in range(E)]
        entry[2] = torch.tensor(flat, dtype=torch.int64).to(dev)
    return entry[2], n_inter


def moe_block(hidden: torch.Tensor, gate_weight: torch.Tensor, shared_weights: dict, experts, config, *,
              layer: int | None = None, routing=None, device_grouping: bool = True) -> torch.Tensor:
    """inference/forward.py:112-153 with the routed experts handed in.

    ``experts`` is one of:

    * a mapping (or a callable) from expert index to its weight dict on the same device;
    * one dict of stacked weights ``{"gate_proj": (w (E, n, k), s (E, ceil(n/128),
      ceil(k/128))), ...}`` (all experts of the layer contiguous: no per-expert host work);
    * an ``amla.experts.ExpertStreamer`` (with ``layer=``): the chosen experts are streamed
      from host memory in waves of at most the pool size, each wave computed before the
      next one is copied, so any batch runs on any pool (gpu_transfer.py:50-89 plus
      forward.py:140-151 without the per-token host synchronisation).

    ``routing=(indices, weights)`` reuses a routing already computed (``route``), so a caller
    that routed to prefetch experts does not route twice.  With stacked weights (and
    ``device_grouping``, the default) the slots are grouped by expert on the device
    (amla_moe_experts_dev): no host copy of the indices and no synchronisation, so the whole
    block can be captured in a HIP graph.  Otherwise, as in the reference, the chosen indices
    come to the host once (one synchronisation) for amla_moe_experts.  Either way each chosen
    expert runs once over all tokens that chose it (the reference loops over (token, k)
    pairs), and the combine keeps the reference's order and bf16 roundings: per token,
    k = 0.. accumulates bf16(bf16(w_k) * expert_k(x)) into a bf16 sum, then shared + sum * 2.5.
    """
    from .experts import ExpertStreamer

    streamed = isinstance(experts, ExpertStreamer)
    if streamed and layer is None:
        raise ValueError("moe_block: an ExpertStreamer needs layer=")
    stacked = not streamed and isinstance(experts, dict) and "gate_proj" in experts and \
        experts["gate_proj"][0].dim() == 3
    get = None if stacked or streamed else (experts if callable(experts) else experts.__getitem__)
    if routing is not None:
        idx, w = routing
    else:
        idx, w = route(hidden, gate_weight, config)
    shared_out = expert_ffn(hidden, shared_weights)
    d = hidden.shape[-1]
    top_k = config.num_experts_per_tok
    E = config.n_routed_experts
    h2 = hidden.reshape(-1, d)
    if not h2.is_contiguous() or h2.data_ptr() % 16:
        h2 = h2.contiguous()
    m = h2.shape[0]
    out = torch.empty_like(hidden)
    if m == 0:
        return out
    dev = hidden.device
    if stacked and device_grouping and E <= MOE_DEV_MAX_EXPERTS:
        table, n_inter = _stacked_device_table(experts, E, d, dev)
        eout = torch.empty(m, top_k, d, dtype=BF16, device=dev)
        _moe_experts_dev_call(h2, idx.reshape(m, top_k).contiguous(), table, n_inter, E, eout)
        return _moe_combine(shared_out, eout, w, m, top_k, d, config, out, hidden)
    idx_host = idx.reshape(m, top_k).cpu().contiguous()
    if streamed:
        eout = _moe_experts_streamed(h2, idx_host, experts, layer, config)
        return _moe_combine(shared_out, eout, w, m, top_k, d, config, out, hidden)
    if stacked:
        tables, n_inter = _stacked_expert_tables(experts, E, d, dev)
        keep = []
        chosen = []
    else:
        tables = [(ctypes.c_void_p * E)() for _ in range(6)]
        n_inter = None
        keep = []
        chosen = torch.unique(idx_host).tolist()
    for e in chosen:
        ew = get(int(e))
        for j, key in enumerate(("gate_proj", "up_proj", "down_proj")):
            wt, sc = ew[key]
            if wt.dtype != FP8 or sc.dtype != torch.float32 or wt.device != dev or sc.device != dev or \
                    not (wt.is_contiguous() and sc.is_contiguous()):
                raise ValueError(f"moe_block: expert {e} {key} must be contiguous e4m3fn weights with fp32 "
                                 f"scales on {dev}")
            tables[2 * j][e] = wt.data_ptr()
            tables[2 * j + 1][e] = sc.data_ptr()
            keep.append((wt, sc))
        ni = ew["gate_proj"][0].shape[0]
        if n_inter is None:
            n_inter = ni
        elif ni != n_inter:
            raise ValueError("moe_block: experts of different intermediate sizes")
        if tuple(ew["gate_proj"][0].shape) != (ni, d) or tuple(ew["up_proj"][0].shape) != (ni, d) or \
                tuple(ew["down_proj"][0].shape) != (d, ni):
            raise ValueError(f"moe_block: expert {e} weights do not match hidden size {d}")
    eout = torch.empty(m, top_k, d, dtype=BF16, device=hidden.device)
    _moe_experts_call(h2, idx_host, tables, n_inter, E, eout)
    del keep
    return _moe_combine(shared_out, eout, w, m, top_k, d, config, out, hidden)


def _moe_experts_call(h2, idx_host, tables, n_inter, E, eout) -> None:
    """amla_moe_experts over the (token, k) slots whose index is >= 0."""
    m, top_k = idx_host.shape
    d = h2.shape[1]
    ws = workspace(h2.device, lib().amla_moe_experts_workspace_bytes(m, d, top_k, n_inter))
    check(lib().amla_moe_experts(h2.data_ptr(), m, d, top_k, idx_host.data_ptr(), n_inter, E,
                                 *[ctypes.cast(t, ctypes.c_void_p) for t in tables], eout.data_ptr(),
                                 ws.data_ptr(), ws.numel(), _stream_ptr(h2)), "moe_experts")


MOE_DEV_MAX_EXPERTS = 512
MOE_DEV_MAX_SLOTS = 65536


def _moe_experts_dev_call(h2, idx_dev, table, n_inter, E, eout) -> None:
    """amla_moe_experts_dev over token chunks of at most 65536 (token, k) slots each."""
    m, top_k = idx_dev.shape
    d = h2.shape[1]
    tpc = max(1, MOE_DEV_MAX_SLOTS // top_k)
    for t0 in range(0, m, tpc):
        mc = min(tpc, m - t0)
        ws = workspace(h2.device, lib().amla_moe_experts_dev_workspace_bytes(mc, d, top_k, n_inter, E))
        check(lib().amla_moe_experts_dev(h2[t0:t0 + mc].data_ptr(), mc, d, top_k, idx_dev[t0:t0 + mc].data_ptr(),
                                         n_inter, E, table.data_ptr(), eout[t0:t0 + mc].data_ptr(), ws.data_ptr(),
                                         ws.numel(), _stream_ptr(h2)), "moe_experts_dev")


def _moe_combine(shared_out, eout, w, m, top_k, d, config, out, hidden):
    sh = shared_out.reshape(m, d).contiguous()
    wc = w.reshape(m, top_k).contiguous()
    check(lib().amla_moe_combine(sh.data_ptr(), eout.data_ptr(), wc.data_ptr(), m, top_k, d,
                                 float(config.routed_scaling_factor), out.data_ptr(), _stream_ptr(hidden)),
          "moe_combine")
    return out


def _moe_experts_streamed(h2, idx_host, streamer, layer, config) -> torch.Tensor:
    """Routed experts streamed in waves of at most ``streamer.slots`` distinct experts: the
    wave's copies (ordered on the device before its compute), then amla_moe_experts over the
    slots of that wave only (the others carry index -1); the next wave's copies reuse slots
    only after this wave's compute (``ExpertStreamer`` releases on the next call)."""
    m, top_k = idx_host.shape
    d = h2.shape[1]
    E = config.n_routed_experts
    chosen = torch.unique(idx_host).tolist()
    eout = torch.empty(m, top_k, d, dtype=BF16, device=h2.device)
    n_inter = None
    for w0 in range(0, len(chosen), streamer.slots):
        wave = chosen[w0:w0 + streamer.slots]
        table = streamer.experts_for(layer, wave)
        tables = [(ctypes.c_void_p * E)() for _ in range(6)]
        for e, ew in table.items():
            for j, key in enumerate(("gate_proj", "up_proj", "down_proj")):
                wt, sc = ew[key]
                tables[2 * j][e] = wt.data_ptr()
                tables[2 * j + 1][e] = sc.data_ptr()
            n_inter = ew["gate_proj"][0].shape[0]
        in_wave = torch.zeros(E, dtype=torch.bool)
        in_wave[wave] = True
        idx_w = torch.where(in_wave[idx_host], idx_host, torch.full_like(idx_host, -1)).contiguous()
        _moe_experts_call(h2, idx_w, tables, n_inter, E, eout)
    streamer.release()
    return eout


# ------------------------------------------------------------------ output head

def lm_head_logits(hidden: torch.Tensor, lm_head_w: torch.Tensor) -> torch.Tensor:
    """inference/forward.py:72: ``hidden.float() @ lm_head_w.float().T`` without the fp32 copy of
    the weight: exact bf16 products summed in fp32.  Returns fp32 (*hidden.shape[:-1], vocab)."""
    _need_cuda(hidden, "hidden")
    if hidden.dtype != BF16:
        raise TypeError(f"lm_head_logits: hidden must be bfloat16 (got {hidden.dtype})")
    _need(lm_head_w, "lm_head_w", BF16, hidden.device)
    n, k = lm_head_w.shape
    if hidden.shape[-1] != k:
        raise ValueError(f"lm_head_logits: hidden has {hidden.shape[-1]} features, lm_head_w expects {k}")
    h2 = hidden.reshape(-1, k)
    if not h2.is_contiguous() or h2.data_ptr() % 16:
        h2 = h2.contiguous()
    m = h2.shape[0]
    out = torch.empty(m, n, dtype=torch.float32, device=hidden.device)
    if m:
        check(lib().amla_bf16_logits(h2.data_ptr(), m, k, lm_head_w.data_ptr(), n, out.data_ptr(), n,
                                     _stream_ptr(hidden)), "lm_head_logits")
    return out.view(*hidden.shape[:-1], n)


def final_logits(hidden: torch.Tensor, final_norm: torch.Tensor, lm_head_w: torch.Tensor, config) -> torch.Tensor:
    """inference/forward.py:67-72: final RMSNorm, then the lm_head projection in fp32."""
    return lm_head_logits(rms_norm(hidden, final_norm, config.rms_norm_eps), lm_head_w)


def sample(logits: torch.Tensor, temperature: float, top_p: float, *, seed: int | None = None) -> torch.Tensor:
    """inference/engine.py:166-186: (B, vocab) fp32 logits -> (B,) int64 token ids.

    temperature 0 is the argmax (ties to the lower index).  Otherwise nucleus
    sampling with the reference's rule (softmax(logits / T), drop a token when the
    mass strictly before it exceeds top_p, renormalise, draw one); the draw uses
    a counter-based generator keyed by ``seed`` (default: drawn from torch's CPU
    generator), so it follows the same distribution as torch.multinomial but not
    its random stream.  Each row is cut into chunks (rows x chunks workgroups); the
    result equals the one-workgroup-per-row kernels' (amla_argmax, amla_sample_top_p).
    """
    _need_cuda(logits, "logits")
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise TypeError("sample: logits must be a (B, vocab) float32 tensor")
    lg = logits if logits.stride(-1) == 1 else logits.contiguous()
    B, n = lg.shape
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    if B == 0:
        return out
    if temperature != 0 and seed is None:
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    ws_bytes = lib().amla_sample_workspace_bytes(B, n)
    ws = workspace(logits.device, ws_bytes)
    check(lib().amla_sample(lg.data_ptr(), B, n, lg.stride(0), float(temperature), float(top_p),
                            int(seed or 0) & (2 ** 64 - 1), out.data_ptr(), ws.data_ptr(), ws_bytes,
                            _stream_ptr(logits)), "sample")
    return out
