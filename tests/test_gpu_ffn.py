"""GPU parity of the FFN / MoE entry points (swiglu, route, moe combine, moe_block)
against the CPU oracle (oracle/ref_ffn.py)."""
import ctypes
from types import SimpleNamespace

import pytest
import torch

from oracle import ref_ffn as F
from amla import ops, synth
from amla.config import DeepSeekConfig
from _tol import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()


def _q(n, k, tag, std=0.02):
    return synth.quantize_fp8_blocks(synth.randn((n, k), synth.seed_of("ffn", tag, n, k), std))


def _mlp(d, i, tag):
    return {"gate_proj": _q(i, d, tag + "/gate"), "up_proj": _q(i, d, tag + "/up"), "down_proj": _q(d, i, tag + "/down")}


def _dev(w):
    return {k: (a.to(DEV), b.to(DEV)) for k, (a, b) in w.items()}


def _x(shape, tag, std=1.0):
    return synth.randn(shape, synth.seed_of("ffnx", tag, *shape), std).to(torch.bfloat16)


def test_silu_mul_bit_pattern():
    for n in (8 * 1000, 8 * 1000 + 5, 1):
        print(f"[case] silu_mul n={n}", flush=True)
        g = _x((n,), "g", 4.0)
        u = _x((n,), "u")
        gd, ud = g.to(DEV), u.to(DEV)
        out = torch.empty_like(gd)
        ops.check(ops.lib().amla_silu_mul(gd.data_ptr(), ud.data_ptr(), n, out.data_ptr(), ops._stream_ptr(gd)),
                  "silu_mul")
        want = F.silu_bf16(g) * u
        got = out.cpu()
        # device expf and torch's CPU exp may differ in the last fp32 bit, which
        # moves a bf16 rounding only at a tie: allow one bf16 ulp on those
        d = (got.float() - want.float()).abs()
        assert (d <= want.float().abs() * 2.0 ** -7 + 1e-30).all()
        assert (got == want).float().mean() >= 0.999


@pytest.mark.parametrize("M", [1, 8, 70])
def test_swiglu_small(M):
    print(f"[case] swiglu small M={M}", flush=True)
    d, i = 256, 384
    w = _mlp(d, i, "small")
    x = _x((M, d), f"small{M}")
    got = ops.dense_ffn(x.to(DEV), _dev(w))
    torch.cuda.synchronize()
    assert_parity(got, F.dense_ffn(x, w), f"swiglu small M={M}")


@pytest.mark.parametrize("which,M", [("dense", 8), ("dense", 32), ("dense", 64), ("expert", 8), ("expert", 1),
                                     ("expert", 96)])
def test_swiglu_r1_shapes(which, M):
    """Dense at M = 64: down_proj's K = 18432 in 18 parts of 8 blocks (x held in registers)."""
    print(f"[case] swiglu r1 {which} M={M}", flush=True)
    d = R1.hidden_size
    i = R1.intermediate_size if which == "dense" else R1.moe_intermediate_size
    w = _mlp(d, i, which)
    x = _x((1, M, d), f"{which}{M}")
    got = ops.swiglu(x.to(DEV), *_dev(w)["gate_proj"], *_dev(w)["up_proj"], *_dev(w)["down_proj"])
    torch.cuda.synchronize()
    assert got.shape == x.shape
    assert_parity(got, F.swiglu(x, *w["gate_proj"], *w["up_proj"], *w["down_proj"]), f"swiglu {which} M={M}")


def _cfg(E, G, TG, K, norm=True):
    return SimpleNamespace(n_routed_experts=E, n_group=G, topk_group=TG, num_experts_per_tok=K,
                           norm_topk_prob=norm, routed_scaling_factor=2.5)


def _check_route(idx, w, ridx, rw, scores):
    """Indices equal, except where the oracle's own scores tie within fp32 noise."""
    idx, w = idx.cpu(), w.cpu()
    same = (idx == ridx).all(-1)
    for r in (~same).nonzero():
        t = tuple(r.tolist())
        a, b = set(idx[t].tolist()), set(ridx[t].tolist())
        diff = sorted(a ^ b)
        s = scores[t]
        kth = s[ridx[t]].min()
        assert all(abs(float(s[e] - kth)) < 1e-5 for e in diff), (t, diff)
    assert same.float().mean() > 0.9
    m = same
    torch.testing.assert_close(w[m], rw[m], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B,S", [(8, 1), (1, 37), (2, 40)])
def test_route_r1(B, S):
    print(f"[case] route r1 B={B} S={S}", flush=True)
    d, E = R1.hidden_size, R1.n_routed_experts
    h = _x((B, S, d), f"route{B}x{S}")
    gw = synth.randn((E, d), synth.seed_of("router", d), 0.02).to(torch.bfloat16)
    idx, w = ops.route(h.to(DEV), gw.to(DEV), R1)
    torch.cuda.synchronize()
    ridx, rw = F.route(h, gw, R1)
    scores = torch.sigmoid(h.float() @ gw.float().T)
    assert idx.shape == ridx.shape and idx.dtype == torch.int64 and w.dtype == torch.float32
    _check_route(idx, w, ridx, rw, scores)
    torch.testing.assert_close(w.cpu().sum(-1), torch.ones(B, S), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("E,G,TG,K,norm", [(16, 4, 2, 4, True), (64, 8, 3, 6, False), (32, 1, 1, 5, True)])
def test_route_small_configs(E, G, TG, K, norm):
    print(f"[case] route small E={E} G={G} TG={TG} K={K}", flush=True)
    cfg = _cfg(E, G, TG, K, norm)
    h = _x((3, 5, 96), f"rs{E}{G}")
    gw = synth.randn((E, 96), synth.seed_of("router-small", E), 0.1).to(torch.bfloat16)
    idx, w = ops.route(h.to(DEV), gw.to(DEV), cfg)
    ridx, rw = F.route(h, gw, cfg)
    _check_route(idx, w, ridx, rw, torch.sigmoid(h.float() @ gw.float().T))


def test_route_group_limit():
    E, G = 16, 4
    logits = torch.full((1, 1, E), -4.0)
    logits[0, 0, 0] = 3.0
    logits[0, 0, 4:8] = torch.tensor([3.5, 2.9, 2.8, 2.7])
    pad = torch.zeros(1, 1, 32 - E)
    h = torch.cat([logits, pad], -1).to(torch.bfloat16).to(DEV)
    gw = torch.eye(E, 32).to(torch.bfloat16).to(DEV)
    idx, _ = ops.route(h, gw, _cfg(E, G, 1, 3))
    assert idx[0, 0].tolist() == [4, 5, 6]
    idx2, _ = ops.route(h, gw, _cfg(E, G, 2, 3))
    assert idx2[0, 0].tolist() == [4, 0, 5]


def test_moe_combine_bit_exact():
    m, K, d = 6, 8, 1000
    sh = _x((m, d), "sh")
    eo = _x((m, K, d), "eo")
    w = torch.rand(m, K, generator=torch.Generator().manual_seed(5))
    out = torch.empty(m, d, dtype=torch.bfloat16, device=DEV)
    shd, eod, wd = sh.to(DEV), eo.to(DEV), w.to(DEV)
    ops.check(ops.lib().amla_moe_combine(shd.data_ptr(), eod.data_ptr(), wd.data_ptr(), m, K, d, 2.5,
                                         out.data_ptr(), ops._stream_ptr(shd)), "moe_combine")
    routed = torch.zeros(m, d, dtype=torch.bfloat16)
    for t in range(m):
        for k in range(K):
            routed[t] += w[t, k].to(torch.bfloat16) * eo[t, k]
    want = sh + routed * 2.5
    assert torch.equal(out.cpu(), want)


@pytest.mark.parametrize("E,G,TG,K,B,S", [(16, 4, 2, 4, 2, 3), (256, 8, 4, 8, 8, 1)])
def test_moe_block(E, G, TG, K, B, S):
    print(f"[case] moe_block E={E} K={K} B={B} S={S}", flush=True)
    d, i = 256, 256
    cfg = _cfg(E, G, TG, K)
    h = _x((B, S, d), f"moe{E}")
    gw = synth.randn((E, d), synth.seed_of("moe-router", E), 0.1).to(torch.bfloat16)
    shared = _mlp(d, i, "shared")
    table = {e: _mlp(d, i, f"expert{e}") for e in range(E)}
    dev_table = {e: _dev(v) for e, v in table.items()}
    got = ops.moe_block(h.to(DEV), gw.to(DEV), _dev(shared), dev_table, cfg)
    torch.cuda.synchronize()
    idx, _ = ops.route(h.to(DEV), gw.to(DEV), cfg)
    ridx, _ = F.route(h, gw, cfg)
    assert torch.equal(idx.cpu(), ridx), "routing differs from the oracle on this seed"
    want = F.moe_block(h, gw, shared, lambda e: table[e], cfg)
    assert_parity(got, want, f"moe_block E={E}")


@pytest.mark.parametrize("E,K,m", [(2, 1, 300), (6, 3, 150), (256, 8, 8), (16, 8, 200)])
def test_moe_experts_vs_expert_ffn(E, K, m):
    """amla_moe_experts (chunks of 512 slots; large expert groups take the GEMM path) against
    expert_ffn of every (token, k) pair."""
    print(f"[case] moe_experts E={E} K={K} m={m}", flush=True)
    d, i = 256, 256
    h = _x((m, d), f"mx{E}{K}")
    g = torch.Generator().manual_seed(E * 1000 + K)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(m)])   # distinct experts per token
    table = {e: _mlp(d, i, f"mx-expert{e}") for e in range(E)}
    dev_table = {e: _dev(v) for e, v in table.items()}
    ptrs = [(ctypes.c_void_p * E)() for _ in range(6)]
    for e in range(E):
        for j, key in enumerate(("gate_proj", "up_proj", "down_proj")):
            ptrs[2 * j][e] = dev_table[e][key][0].data_ptr()
            ptrs[2 * j + 1][e] = dev_table[e][key][1].data_ptr()
    hd = h.to(DEV)
    eout = torch.empty(m, K, d, dtype=torch.bfloat16, device=DEV)
    need = ops.lib().amla_moe_experts_workspace_bytes(m, d, K, i)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    idx64 = idx.to(torch.int64).contiguous()
    ops.check(ops.lib().amla_moe_experts(hd.data_ptr(), m, d, K, idx64.data_ptr(), i, E,
                                         *[ctypes.cast(t, ctypes.c_void_p) for t in ptrs], eout.data_ptr(),
                                         ws.data_ptr(), need, ops._stream_ptr(hd)), "moe_experts")
    torch.cuda.synchronize()
    want = torch.empty(m, K, d, dtype=torch.bfloat16)
    for e in range(E):
        sel = (idx == e).nonzero()
        if len(sel):
            y = F.expert_ffn(h[sel[:, 0]], table[e])
            want[sel[:, 0], sel[:, 1]] = y
    assert_parity(eout, want, f"moe_experts E={E} K={K} m={m}")


def test_moe_block_stacked_experts():
    print("[case] moe_block stacked", flush=True)
    E, d, i = 32, 256, 256
    cfg = _cfg(E, 4, 2, 4)
    h = _x((3, 2, d), "moe-stacked")
    gw = synth.randn((E, d), synth.seed_of("moe-router-st", E), 0.1).to(torch.bfloat16)
    shared = _mlp(d, i, "shared-st")
    table = {e: _mlp(d, i, f"st-expert{e}") for e in range(E)}
    stacked = {k: (torch.stack([table[e][k][0] for e in range(E)]).to(DEV),
                   torch.stack([table[e][k][1] for e in range(E)]).to(DEV)) for k in ("gate_proj", "up_proj", "down_proj")}
    got = ops.moe_block(h.to(DEV), gw.to(DEV), _dev(shared), stacked, cfg)
    got2 = ops.moe_block(h.to(DEV), gw.to(DEV), _dev(shared), stacked, cfg)    # cached tables
    torch.cuda.synchronize()
    want = F.moe_block(h, gw, shared, lambda e: table[e], cfg)
    assert_parity(got, want, "moe_block stacked")
    assert torch.equal(got, got2)


def test_empty_inputs():
    d, i = 256, 256
    w = _dev(_mlp(d, i, "empty"))
    x = torch.zeros(2, 0, d, dtype=torch.bfloat16, device=DEV)
    assert ops.dense_ffn(x, w).shape == (2, 0, d)
    cfg = _cfg(16, 4, 2, 4)
    gw = torch.zeros(16, d, dtype=torch.bfloat16, device=DEV)
    idx, wt = ops.route(x, gw, cfg)
    assert idx.shape == (2, 0, 4) and wt.shape == (2, 0, 4)
    assert ops.moe_block(x, gw, w, {e: w for e in range(16)}, cfg).shape == (2, 0, d)


def test_moe_experts_duplicate_indices_r1_shape():
    """Every (token, k) slot of 8 tokens on one expert (a token may list an expert more than
    once): one 64-row group at the R1 expert shape, whose K-part sums need the workspace
    sized for 64 rows, not for the 8 tokens."""
    print("[case] moe_experts duplicates m=8 K=8 R1 shape", flush=True)
    E, K, m, d, i = 4, 8, 8, 7168, 2048
    h = _x((m, d), "mxdup")
    idx = torch.full((m, K), 3, dtype=torch.int64)
    idx[0, 0] = 1                                           # one slot elsewhere: two runs
    table = {e: _mlp(d, i, f"mxdup-expert{e}") for e in (1, 3)}
    dev_table = {e: _dev(v) for e, v in table.items()}
    ptrs = [(ctypes.c_void_p * E)() for _ in range(6)]
    for e, v in dev_table.items():
        for j, key in enumerate(("gate_proj", "up_proj", "down_proj")):
            ptrs[2 * j][e] = v[key][0].data_ptr()
            ptrs[2 * j + 1][e] = v[key][1].data_ptr()
    hd = h.to(DEV)
    eout = torch.empty(m, K, d, dtype=torch.bfloat16, device=DEV)
    need = ops.lib().amla_moe_experts_workspace_bytes(m, d, K, i)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ops.check(ops.lib().amla_moe_experts(hd.data_ptr(), m, d, K, idx.data_ptr(), i, E,
                                         *[ctypes.cast(t, ctypes.c_void_p) for t in ptrs], eout.data_ptr(),
                                         ws.data_ptr(), need, ops._stream_ptr(hd)), "moe_experts")
    torch.cuda.synchronize()
    want = torch.empty(m, K, d, dtype=torch.bfloat16)
    for e in (1, 3):
        sel = (idx == e).nonzero()
        want[sel[:, 0], sel[:, 1]] = F.expert_ffn(h[sel[:, 0]], table[e])
    assert_parity(eout, want, "moe_experts duplicate indices")
