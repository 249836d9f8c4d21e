"""Float64 statements of the MLA path, for invariants and error budgets.

TEST INFRASTRUCTURE ONLY (see oracle/ref_ops.py for the import rule).

``mla_naive_f64`` is inference/ops.py:100-183 with every intermediate kept in
float64 (no bf16 rounding points); ``mla_decode_absorbed_f64`` is the absorbed
formulation the GPU decode implements:

    r_t    = rsqrt(mean(c_t^2) + eps)
    qt[h]  = gamma * (W_UK[h]^T q_nope[h])                      (512)
    s[h,t] = sigma * ( r_t (qt[h] . c_t) + q_pe_rot[h] . rot(t) k_pe[t] )
    out[h] = W_UV[h] ( gamma * sum_t softmax(s[h])_t r_t c_t )

with W_UK[h] = kv_b rows h*256 .. h*256+127 and W_UV[h] = rows h*256+128 .. +255
(inference/ops.py:149-151).  The two agree to fp64 rounding; a test checks it.
"""
from __future__ import annotations

import math

import torch

from .ref_ops import fp8_block_dequant, yarn_get_mscale


def _rms64(x, gamma, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * gamma.double()


def _rope64(x, freqs):
    """Rotate interleaved pairs of x (..., T, 2P) by complex freqs (T, P) in fp64."""
    xc = torch.view_as_complex(x.reshape(*x.shape[:-1], -1, 2).contiguous())
    f = freqs.to(torch.complex128)
    return torch.view_as_real(xc * f).flatten(-2)


def _w64(pair):
    return fp8_block_dequant(*pair).double()


def project_queries_f64(hidden, aw, position, rope_freqs, cfg):
    """(q_nope (B,H,S,nope), q_pe_rot (B,H,S,rope), kv_a (B,S,lora+rope)) in fp64."""
    B, S, _ = hidden.shape
    H = cfg.num_attention_heads
    x = hidden.double()
    qa = _rms64(x @ _w64(aw["q_a_proj"]).T, aw["q_a_layernorm"], cfg.rms_norm_eps)
    q = (qa @ _w64(aw["q_b_proj"]).T).view(B, S, H, cfg.qk_head_dim).permute(0, 2, 1, 3)
    q_nope, q_pe = q.split([cfg.qk_nope_head_dim, cfg.qk_rope_head_dim], -1)
    q_pe = _rope64(q_pe, rope_freqs[position:position + S])
    kva = x @ _w64(aw["kv_a_proj_with_mqa"]).T
    return q_nope, q_pe, kva


def mla_naive_f64(hidden, aw, ckv_rows, kpe_rows, position, rope_freqs, cfg):
    """Reference math in fp64.  ckv_rows/kpe_rows: (B, T, .) cache contents *after* the new rows."""
    return mla_naive_parts_f64(hidden, aw, ckv_rows, kpe_rows, position, rope_freqs, cfg)[1]


def mla_naive_parts_f64(hidden, aw, ckv_rows, kpe_rows, position, rope_freqs, cfg):
    """mla_naive_f64 returning (per-head output before o_proj (B, S, H*v), output (B, S, hidden))."""
    B, S, _ = hidden.shape
    H, nope, vd = cfg.num_attention_heads, cfg.qk_nope_head_dim, cfg.v_head_dim
    T = position + S
    q_nope, q_pe, _ = project_queries_f64(hidden, aw, position, rope_freqs, cfg)
    c = _rms64(ckv_rows[:, :T].double(), aw["kv_a_layernorm"], cfg.rms_norm_eps)
    kvb = (c @ _w64(aw["kv_b_proj"]).T).view(B, T, H, nope + vd).permute(0, 2, 1, 3)
    k_nope, v = kvb.split([nope, vd], -1)
    kpe = _rope64(kpe_rows[:, :T].double(), rope_freqs[:T])[:, None].expand(-1, H, -1, -1)
    sigma = yarn_get_mscale(cfg.rope_scaling_factor, cfg.rope_scaling_mscale_all_dim) / math.sqrt(cfg.qk_head_dim)
    s = (q_nope @ k_nope.transpose(-1, -2) + q_pe @ kpe.transpose(-1, -2)) * sigma
    if S > 1:
        i = torch.arange(S)[:, None] + position
        j = torch.arange(T)[None, :]
        s = s.masked_fill(j > i, float("-inf"))
    p = torch.softmax(s, -1)
    o = (p @ v).permute(0, 2, 1, 3).reshape(B, S, H * vd)
    return o, o @ _w64(aw["o_proj"]).T


def mla_decode_absorbed_f64(hidden, aw, ckv_rows, kpe_rows, positions, rope_freqs, cfg):
    """Absorbed decode (S = 1), one position per sequence; returns (B, 1, hidden) fp64."""
    return mla_decode_absorbed_parts_f64(hidden, aw, ckv_rows, kpe_rows, positions, rope_freqs, cfg)[1]


def mla_decode_absorbed_parts_f64(hidden, aw, ckv_rows, kpe_rows, positions, rope_freqs, cfg):
    """Absorbed decode in fp64: (per-head output before o_proj (B, 1, H*v), output (B, 1, hidden))."""
    B = hidden.shape[0]
    H, nope, vd, lora = cfg.num_attention_heads, cfg.qk_nope_head_dim, cfg.v_head_dim, cfg.kv_lora_rank
    gamma = aw["kv_a_layernorm"].double()
    wkvb = _w64(aw["kv_b_proj"]).view(H, nope + vd, lora)
    w_uk, w_uv = wkvb[:, :nope], wkvb[:, nope:]
    wo = _w64(aw["o_proj"])
    sigma = yarn_get_mscale(cfg.rope_scaling_factor, cfg.rope_scaling_mscale_all_dim) / math.sqrt(cfg.qk_head_dim)
    heads, outs = [], []
    for b in range(B):
        p = int(positions[b])
        T = p + 1
        q_nope, q_pe, _ = project_queries_f64(hidden[b:b + 1], aw, p, rope_freqs, cfg)
        q_nope, q_pe = q_nope[0, :, 0], q_pe[0, :, 0]                        # (H, nope), (H, rope)
        o = _absorbed_row(q_nope, q_pe, ckv_rows[b, :T], kpe_rows[b, :T], rope_freqs, w_uk, w_uv, gamma, sigma,
                          cfg.rms_norm_eps).reshape(1, H * vd)
        heads.append(o)
        outs.append(o @ wo.T)
    return torch.stack(heads, 0), torch.stack(outs, 0)


def _absorbed_row(q_nope, q_pe, ckv, kpe, rope_freqs, w_uk, w_uv, gamma, sigma, eps):
    """One query (H heads) over the cache rows ckv/kpe (T, .), absorbed form in fp64: (H, v)."""
    T = ckv.shape[0]
    qt = torch.einsum("hd,hdc->hc", q_nope, w_uk) * gamma                    # (H, lora)
    c = ckv.double()
    r = torch.rsqrt(c.pow(2).mean(-1) + eps)                                 # (T,)
    kpe = _rope64(kpe.double(), rope_freqs[:T])                              # (T, rope)
    s = sigma * (r[None] * (qt @ c.T) + q_pe @ kpe.T)                        # (H, T)
    w = torch.softmax(s, -1)
    lat = (w * r[None]) @ c * gamma                                          # (H, lora)
    return torch.einsum("hvc,hc->hv", w_uv, lat)


def mla_prefill_rows_f64(hidden, aw, ckv_rows, kpe_rows, position, rows, rope_freqs, cfg):
    """Exact outputs of chosen query rows of a causal prefill of B = 1 sequence.

    Query row i (position ``position + i``) attends to cache rows
    [0, position + i]; ckv_rows / kpe_rows hold the cache after the new rows
    were written.  Returns (per-head outputs (len(rows), H*v), outputs
    (len(rows), hidden)), fp64.  The absorbed form equals the naive one in exact
    arithmetic (checked by tests/test_oracle.py), and costs O(T) per row.
    """
    H, nope, vd, lora = cfg.num_attention_heads, cfg.qk_nope_head_dim, cfg.v_head_dim, cfg.kv_lora_rank
    gamma = aw["kv_a_layernorm"].double()
    wkvb = _w64(aw["kv_b_proj"]).view(H, nope + vd, lora)
    w_uk, w_uv = wkvb[:, :nope], wkvb[:, nope:]
    wo = _w64(aw["o_proj"])
    sigma = yarn_get_mscale(cfg.rope_scaling_factor, cfg.rope_scaling_mscale_all_dim) / math.sqrt(cfg.qk_head_dim)
    heads = []
    for i in rows:
        i = int(i)
        T = position + i + 1
        # queries are per row: only the chosen rows are projected (at their own positions)
        q_nope, q_pe, _ = project_queries_f64(hidden[:1, i:i + 1], aw, position + i, rope_freqs, cfg)
        heads.append(_absorbed_row(q_nope[0, :, 0], q_pe[0, :, 0], ckv_rows[0, :T], kpe_rows[0, :T], rope_freqs,
                                   w_uk, w_uv, gamma, sigma, cfg.rms_norm_eps).reshape(H * vd))
    h = torch.stack(heads, 0)
    return h, h @ wo.T
