"""PyTorch custom operators over libamla.so: the ``torch.ops.amla`` namespace.

Each operator is a ``torch.library.custom_op`` whose CUDA (ROCm) implementation
calls the C ABI of include/amla.h through ctypes, with a fake (meta)
implementation so that FakeTensor tracing, ``torch.compile`` and ``make_fx`` see
the op, its output shape and its in-place writes:

* ``amla::fp8_linear(x, weight, scale_inv)``           inference/ops.py:15-44
* ``amla::fp8_linear_f32(x, weight, scale_inv)``       the same with fp32 output (out_dtype)
* ``amla::swiglu(x, gate, gate_scale, up, up_scale, down, down_scale)``  inference/ops.py:186-192
* ``amla::rms_norm(x, weight, eps)``                   inference/ops.py:10-12
* ``amla::apply_rope(x, freqs)``                       inference/ops.py:86-97
* ``amla::mla_decode(...)`` / ``amla::mla_prefill(...)``  inference/ops.py:100-183;
  both mutate ``ckv_cache`` and ``kpe_cache`` in place (the cache store of
  inference/ops.py:140-141) and, when given, ``attn_out`` (the per-head output
  before o_proj).

Tensors only, no dicts or dataclasses (the op schema cannot carry them): the
shims in amla.ops keep the reference's signatures and unpack ``attn_weights``
and ``config`` into these arguments after validating them.

Scratch memory (split-K partials, queries, latent partials) is taken from
torch's caching allocator on every call, on the calling stream: a call inside a
HIP graph capture allocates from the graph's private pool, so a replay never
sees memory that a later call freed or reused, and calls on different streams
never share scratch.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from ._lib import MlaArgs, check, lib

BF16 = torch.bfloat16


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _scratch(dev: torch.device, nbytes: int) -> Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=dev)


# ------------------------------------------------------------------ fp8_linear

def _rows16(x: Tensor) -> Tensor:
    """x itself when its base is 16-byte aligned, else an aligned copy (the kernels load 16-byte
    chunks); checked here, inside the operator, where the tensor is real."""
    return x if x.data_ptr() % 16 == 0 else x.clone(memory_format=torch.contiguous_format)


def _linear(x: Tensor, weight: Tensor, scale_inv: Tensor, f32: bool) -> Tensor:
    x = _rows16(x)
    m, k = x.shape
    n = weight.shape[0]
    y = torch.empty(m, n, dtype=torch.float32 if f32 else BF16, device=x.device)
    if m == 0:
        return y
    L = lib()
    need = L.amla_fp8_linear_workspace_bytes(m, n, k) if m <= 64 else 0
    ws = _scratch(x.device, need) if need else None
    fn = L.amla_fp8_linear_f32 if f32 else L.amla_fp8_linear
    check(fn(x.data_ptr(), m, k, x.stride(0), weight.data_ptr(), scale_inv.data_ptr(), n, y.data_ptr(), n,
             ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, _stream(x.device)),
          "fp8_linear_f32" if f32 else "fp8_linear")
    return y


@torch.library.custom_op("amla::fp8_linear", mutates_args=(), device_types="cuda")
def fp8_linear(x: Tensor, weight: Tensor, scale_inv: Tensor) -> Tensor:
    """y (M, N) bf16 = bf16(x (M, K) @ dequant(weight, scale_inv).T); x rows with unit stride."""
    return _linear(x, weight, scale_inv, False)


@fp8_linear.register_fake
def _(x, weight, scale_inv):
    return x.new_empty(x.shape[0], weight.shape[0])


@torch.library.custom_op("amla::fp8_linear_f32", mutates_args=(), device_types="cuda")
def fp8_linear_f32(x: Tensor, weight: Tensor, scale_inv: Tensor) -> Tensor:
    """y (M, N) fp32 = x (M, K) @ dequant(weight, scale_inv).T, fp32 accumulation, no rounding."""
    return _linear(x, weight, scale_inv, True)


@fp8_linear_f32.register_fake
def _(x, weight, scale_inv):
    return x.new_empty(x.shape[0], weight.shape[0], dtype=torch.float32)


@torch.library.custom_op("amla::swiglu", mutates_args=(), device_types="cuda")
def swiglu(x: Tensor, gate_proj: Tensor, gate_scale: Tensor, up_proj: Tensor, up_scale: Tensor, down_proj: Tensor,
           down_scale: Tensor) -> Tensor:
    """(M, K) bf16 -> down(silu(gate(x)) * up(x)) (M, K) bf16, every product rounded as in the reference."""
    x = _rows16(x)
    m, k = x.shape
    n = gate_proj.shape[0]
    y = torch.empty(m, k, dtype=BF16, device=x.device)
    if m == 0:
        return y
    L = lib()
    need = L.amla_swiglu_workspace_bytes(m, k, n)
    ws = _scratch(x.device, need)
    check(L.amla_swiglu(x.data_ptr(), m, k, gate_proj.data_ptr(), gate_scale.data_ptr(), up_proj.data_ptr(),
                        up_scale.data_ptr(), n, down_proj.data_ptr(), down_scale.data_ptr(), y.data_ptr(),
                        ws.data_ptr(), ws.numel(), _stream(x.device)), "swiglu")
    return y


@swiglu.register_fake
def _(x, gate_proj, gate_scale, up_proj, up_scale, down_proj, down_scale):
    return torch.empty_like(x)


# ------------------------------------------------------------------ rms_norm / apply_rope

@torch.library.custom_op("amla::rms_norm", mutates_args=(), device_types="cuda")
def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """(rows, dim) bf16 -> bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)."""
    y = torch.empty_like(x)
    rows, dim = x.shape
    check(lib().amla_rms_norm(x.data_ptr(), rows, dim, dim, weight.data_ptr(), float(eps), y.data_ptr(), dim,
                              _stream(x.device)), "rms_norm")
    return y


@rms_norm.register_fake
def _(x, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op("amla::apply_rope", mutates_args=(), device_types="cuda")
def apply_rope(x: Tensor, freqs: Tensor) -> Tensor:
    """x (groups, S, dim) bf16 rotated by freqs (S, dim/2) complex64."""
    y = torch.empty_like(x)
    groups, s, dim = x.shape
    f = torch.view_as_real(freqs)
    check(lib().amla_apply_rope(x.data_ptr(), groups, s, dim, f.data_ptr(), y.data_ptr(), _stream(x.device)),
          "apply_rope")
    return y


@apply_rope.register_fake
def _(x, freqs):
    return torch.empty_like(x)


# ------------------------------------------------------------------ MLA

def fill_mla_args(hidden: Tensor, w_q_a: Tensor, s_q_a: Tensor, w_q_b: Tensor, s_q_b: Tensor, w_kv_a: Tensor,
                  s_kv_a: Tensor, w_kv_b: Tensor, s_kv_b: Tensor, w_o: Tensor, s_o: Tensor, gamma_q: Tensor,
                  gamma_kv: Tensor, ckv_cache: Tensor, kpe_cache: Tensor, positions: Tensor, rope_freqs: Tensor,
                  input_gamma: Optional[Tensor], residual: Optional[Tensor], attn_out: Optional[Tensor],
                  out: Tensor, max_context: int, eps: float, softmax_scale: float, heads: int, qk_nope: int,
                  v_dim: int) -> MlaArgs:
    """amla_mla_args for validated tensors (no workspace yet)."""
    B, S, D = hidden.shape
    a = MlaArgs()
    a.batch, a.seq_len, a.hidden = B, S, D
    a.heads, a.q_lora, a.kv_lora = heads, w_q_a.shape[0], ckv_cache.shape[2]
    a.qk_nope, a.qk_rope, a.v_dim = qk_nope, kpe_cache.shape[2], v_dim
    a.max_seq, a.rope_rows, a.max_context = ckv_cache.shape[1], rope_freqs.shape[0], int(max_context)
    a.eps, a.softmax_scale = float(eps), float(softmax_scale)
    a.positions = positions.data_ptr()
    a.hidden_states, a.out = hidden.data_ptr(), out.data_ptr()
    a.input_gamma = input_gamma.data_ptr() if input_gamma is not None else None
    a.residual = residual.data_ptr() if residual is not None else None
    a.w_q_a, a.s_q_a, a.w_q_b, a.s_q_b = w_q_a.data_ptr(), s_q_a.data_ptr(), w_q_b.data_ptr(), s_q_b.data_ptr()
    a.w_kv_a, a.s_kv_a = w_kv_a.data_ptr(), s_kv_a.data_ptr()
    a.w_kv_b, a.s_kv_b = w_kv_b.data_ptr(), s_kv_b.data_ptr()
    a.w_o, a.s_o = w_o.data_ptr(), s_o.data_ptr()
    a.gamma_q, a.gamma_kv = gamma_q.data_ptr(), gamma_kv.data_ptr()
    a.ckv_cache, a.kpe_cache = ckv_cache.data_ptr(), kpe_cache.data_ptr()
    a.rope_table = rope_freqs.data_ptr()
    a.attn_out = attn_out.data_ptr() if attn_out is not None else None
    return a


def _mla_run(decode: bool, hidden, w_q_a, s_q_a, w_q_b, s_q_b, w_kv_a, s_kv_a, w_kv_b, s_kv_b, w_o, s_o, gamma_q,
             gamma_kv, ckv_cache, kpe_cache, positions, rope_freqs, input_gamma, residual, attn_out, max_context,
             eps, softmax_scale, heads, qk_nope, v_dim) -> Tensor:
    out = torch.empty_like(hidden)
    a = fill_mla_args(hidden, w_q_a, s_q_a, w_q_b, s_q_b, w_kv_a, s_kv_a, w_kv_b, s_kv_b, w_o, s_o, gamma_q,
                      gamma_kv, ckv_cache, kpe_cache, positions, rope_freqs, input_gamma, residual, attn_out, out,
                      max_context, eps, softmax_scale, heads, qk_nope, v_dim)
    L = lib()
    need = (L.amla_mla_decode_workspace_bytes if decode else L.amla_mla_prefill_workspace_bytes)(a)
    ws = _scratch(hidden.device, need)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    rc = (L.amla_mla_decode if decode else L.amla_mla_prefill)(a, _stream(hidden.device))
    check(rc, "mla_decode" if decode else "mla_prefill")
    return out


_MLA_MUTATES = ("ckv_cache", "kpe_cache", "attn_out")


@torch.library.custom_op("amla::mla_decode", mutates_args=_MLA_MUTATES, device_types="cuda")
def mla_decode(hidden: Tensor, w_q_a: Tensor, s_q_a: Tensor, w_q_b: Tensor, s_q_b: Tensor, w_kv_a: Tensor,
               s_kv_a: Tensor, w_kv_b: Tensor, s_kv_b: Tensor, w_o: Tensor, s_o: Tensor, gamma_q: Tensor,
               gamma_kv: Tensor, ckv_cache: Tensor, kpe_cache: Tensor, positions: Tensor, rope_freqs: Tensor,
               input_gamma: Optional[Tensor], residual: Optional[Tensor], attn_out: Optional[Tensor],
               max_context: int, eps: float, softmax_scale: float, heads: int, qk_nope: int,
               v_dim: int) -> Tensor:
    """Absorbed-MLA decode (S == 1): returns (B, 1, hidden) bf16; writes the new cache rows."""
    return _mla_run(True, hidden, w_q_a, s_q_a, w_q_b, s_q_b, w_kv_a, s_kv_a, w_kv_b, s_kv_b, w_o, s_o, gamma_q,
                    gamma_kv, ckv_cache, kpe_cache, positions, rope_freqs, input_gamma, residual, attn_out,
                    max_context, eps, softmax_scale, heads, qk_nope, v_dim)


@torch.library.custom_op("amla::mla_prefill", mutates_args=_MLA_MUTATES, device_types="cuda")
def mla_prefill(hidden: Tensor, w_q_a: Tensor, s_q_a: Tensor, w_q_b: Tensor, s_q_b: Tensor, w_kv_a: Tensor,
                s_kv_a: Tensor, w_kv_b: Tensor, s_kv_b: Tensor, w_o: Tensor, s_o: Tensor, gamma_q: Tensor,
                gamma_kv: Tensor, ckv_cache: Tensor, kpe_cache: Tensor, positions: Tensor, rope_freqs: Tensor,
                input_gamma: Optional[Tensor], residual: Optional[Tensor], attn_out: Optional[Tensor],
                max_context: int, eps: float, softmax_scale: float, heads: int, qk_nope: int,
                v_dim: int) -> Tensor:
    """Causal MLA prefill (S >= 1): returns (B, S, hidden) bf16; writes the new cache rows."""
    return _mla_run(False, hidden, w_q_a, s_q_a, w_q_b, s_q_b, w_kv_a, s_kv_a, w_kv_b, s_kv_b, w_o, s_o, gamma_q,
                    gamma_kv, ckv_cache, kpe_cache, positions, rope_freqs, input_gamma, residual, attn_out,
                    max_context, eps, softmax_scale, heads, qk_nope, v_dim)


def _mla_fake(hidden, *args, **kwargs):
    return torch.empty_like(hidden)


mla_decode.register_fake(_mla_fake)
mla_prefill.register_fake(_mla_fake)
