"""Pins the FFN / MoE oracle (oracle/ref_ffn.py) against closed forms and an independent
float64 formulation of the routing.  No GPU.
"""
import math
from types import SimpleNamespace

import numpy as np
import torch

from oracle import ref_ffn as F


def _bf(x: float) -> float:
    return torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).item()


def _onehot_fp8(n: int, k: int, cols) -> tuple[torch.Tensor, torch.Tensor]:
    """(n, k) e4m3fn weight whose row i is the unit vector e_{cols[i]}; scale_inv 1."""
    w = torch.zeros(n, k, dtype=torch.float32)
    w[torch.arange(n), torch.as_tensor(cols)] = 1.0
    return w.to(torch.float8_e4m3fn), torch.ones((n + 127) // 128, (k + 127) // 128)


def test_swiglu_onehot_closed_form():
    torch.manual_seed(0)
    K, N, D = 256, 128, 256
    x = (torch.randn(1, 3, K) * 3).to(torch.bfloat16)
    gc = torch.randperm(K)[:N]
    uc = torch.randperm(K)[:N]
    dc = torch.randint(0, N, (D,))
    out = F.swiglu(x, *_onehot_fp8(N, K, gc), *_onehot_fp8(N, K, uc), *_onehot_fp8(D, N, dc))
    xs = x.double()
    g = xs[..., gc]
    silu = g / (1.0 + torch.exp(-g))                    # float64 closed form
    silu_b = silu.float().to(torch.bfloat16).double()
    h = (silu_b * xs[..., uc]).float().to(torch.bfloat16).double()
    want = h[..., dc]
    # float64 -> fp32 -> bf16 can differ from the fp32 formula by one bf16 ulp at a tie
    ulp = want.abs().clamp_min(2.0 ** -126) * 2.0 ** -7
    assert ((out.double() - want).abs() <= ulp).all()
    assert (out.double() == want).float().mean() > 0.99


def test_silu_special_values():
    x = torch.tensor([0.0, 1.0, -1.0, 20.0, -20.0], dtype=torch.bfloat16)
    got = F.silu_bf16(x).float()
    want = [0.0, _bf(1 / (1 + math.exp(-1))), _bf(-1 / (1 + math.exp(1))), 20.0, _bf(-20 / (1 + math.exp(20)))]
    assert got.tolist() == want


def _route_numpy(scores: np.ndarray, n_group: int, topk_group: int, top_k: int, norm: bool):
    """Independent formulation: rank groups by their maximum, then the experts of the chosen
    groups by score (no masking, no torch.topk)."""
    E = scores.shape[-1]
    gs = E // n_group
    idx_all, w_all = [], []
    for row in scores.reshape(-1, E):
        gmax = row.reshape(n_group, gs).max(axis=1)
        groups = np.argsort(-gmax, kind="stable")[:topk_group]
        cand = np.concatenate([np.arange(g * gs, (g + 1) * gs) for g in groups])
        order = cand[np.argsort(-row[cand], kind="stable")][:top_k]
        w = row[order].astype(np.float64)
        if norm:
            w = w / (w.sum() + 1e-9)
        idx_all.append(order)
        w_all.append(w)
    shp = scores.shape[:-1] + (top_k,)
    return np.array(idx_all).reshape(shp), np.array(w_all).reshape(shp)


def _cfg(E, n_group, topk_group, top_k, norm=True):
    return SimpleNamespace(n_routed_experts=E, n_group=n_group, topk_group=topk_group,
                           num_experts_per_tok=top_k, norm_topk_prob=norm, routed_scaling_factor=2.5)


def test_route_matches_independent_formulation():
    torch.manual_seed(1)
    for (E, G, TG, K, D) in [(256, 8, 4, 8, 512), (64, 8, 3, 6, 96), (16, 4, 2, 4, 128)]:
        cfg = _cfg(E, G, TG, K)
        h = torch.randn(2, 5, D).to(torch.bfloat16)
        gw = (torch.randn(E, D) * 0.05).to(torch.bfloat16)
        idx, w = F.route(h, gw, cfg)
        scores = torch.sigmoid(h.float() @ gw.float().T).numpy()
        want_i, want_w = _route_numpy(scores, G, TG, K, True)
        assert (idx.numpy() == want_i).all()
        np.testing.assert_allclose(w.numpy(), want_w, rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(w.sum(-1).numpy(), 1.0, rtol=1e-5)
        # the logits are an fp32 GEMM of bf16 inputs: float64 agrees to fp32 rounding
        l64 = h.double() @ gw.double().T
        np.testing.assert_allclose((h.float() @ gw.float().T).double().numpy(), l64.numpy(), rtol=1e-4, atol=1e-5)


def test_route_group_limit_changes_the_answer():
    # group 0 holds the single best expert; group 1 holds many good ones.  With
    # topk_group = 1 only group 1 may be chosen if its maximum is larger.
    E, G = 16, 4
    logits = torch.full((1, 1, E), -4.0)
    logits[0, 0, 0] = 3.0                     # group 0: one high expert
    logits[0, 0, 4:8] = torch.tensor([3.5, 2.9, 2.8, 2.7])  # group 1: max 3.5
    gw = torch.eye(E).to(torch.bfloat16)
    hidden = logits.to(torch.bfloat16)        # hidden @ I = logits (exact in bf16 here)
    idx, _ = F.route(hidden, gw, _cfg(E, G, 1, 3))
    assert idx[0, 0].tolist() == [4, 5, 6]    # all from group 1; expert 0 is excluded
    idx2, _ = F.route(hidden, gw, _cfg(E, G, 2, 3))
    assert idx2[0, 0].tolist() == [4, 0, 5]   # groups 1 and 0 allowed


def test_route_without_normalisation_returns_sigmoids():
    torch.manual_seed(2)
    h = torch.randn(1, 2, 64).to(torch.bfloat16)
    gw = (torch.randn(32, 64) * 0.1).to(torch.bfloat16)
    idx, w = F.route(h, gw, _cfg(32, 4, 4, 5, norm=False))
    s = torch.sigmoid(h.float() @ gw.float().T)
    assert torch.equal(w, torch.gather(s, -1, idx))


def _expert(seed, D, I):
    g = torch.Generator().manual_seed(seed)
    def q(n, k):
        w = torch.randn(n, k, generator=g) * 0.05
        s = torch.rand((n + 127) // 128, (k + 127) // 128, generator=g) + 0.5
        return (w / s.repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)[:, :k]).clamp(-448, 448).to(
            torch.float8_e4m3fn), s
    return {"gate_proj": q(I, D), "up_proj": q(I, D), "down_proj": q(D, I)}


def test_moe_zero_routed_experts_leave_shared_output():
    D, I, E = 256, 128, 16
    cfg = _cfg(E, 4, 2, 4)
    torch.manual_seed(3)
    hidden = torch.randn(2, 1, D).to(torch.bfloat16)
    gw = (torch.randn(E, D) * 0.05).to(torch.bfloat16)
    shared = _expert(100, D, I)
    zero = _expert(101, D, I)
    zero["down_proj"] = (torch.zeros(D, I).to(torch.float8_e4m3fn), zero["down_proj"][1])
    out = F.moe_block(hidden, gw, shared, lambda e: zero, cfg)
    assert torch.equal(out, F.expert_ffn(hidden, shared))


def test_moe_single_expert_closed_form():
    D, I, E = 256, 128, 8
    cfg = _cfg(E, 2, 2, 1)
    torch.manual_seed(4)
    hidden = torch.randn(1, 2, D).to(torch.bfloat16)
    gw = (torch.randn(E, D) * 0.05).to(torch.bfloat16)
    shared = _expert(200, D, I)
    table = {e: _expert(300 + e, D, I) for e in range(E)}
    out = F.moe_block(hidden, gw, shared, lambda e: table[e], cfg)
    idx, w = F.route(hidden, gw, cfg)
    assert torch.allclose(w, torch.ones_like(w))        # one expert, normalised weight 1 - 1e-9
    for s in range(2):
        e_out = F.expert_ffn(hidden[:, s:s + 1], table[int(idx[0, s, 0])])[0, 0]
        routed = (w[0, s, 0].to(torch.bfloat16).float() * e_out.float()).to(torch.bfloat16)
        sh = F.expert_ffn(hidden[:, s:s + 1], shared)[0, 0]
        want = (sh.float() + (routed.float() * 2.5).to(torch.bfloat16).float()).to(torch.bfloat16)
        assert torch.equal(out[0, s], want)
