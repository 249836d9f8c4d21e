"""GPU parity of the output head (lm_head logits, greedy and nucleus sampling) against the
CPU oracle (oracle/ref_head.py)."""
import pytest
import torch

from oracle import ref_head as H
from amla import ops, synth
from amla.config import DeepSeekConfig

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
R1 = DeepSeekConfig()


def test_lm_head_logits_r1():
    print("[case] lm_head logits r1 B=8", flush=True)
    d, V = R1.hidden_size, R1.vocab_size
    h = synth.randn((8, 1, d), synth.seed_of("head", "h"), 1.0).to(torch.bfloat16)
    g = synth.gamma(d, synth.seed_of("head", "g"))
    w = synth.randn((V, d), synth.seed_of("head", "w"), 0.02).to(torch.bfloat16)
    got = ops.final_logits(h.to(DEV), g.to(DEV), w.to(DEV), R1)
    torch.cuda.synchronize()
    want = H.lm_head_logits(h, g, w, R1.rms_norm_eps)
    assert got.shape == want.shape and got.dtype == torch.float32
    # fp32 sums of the same exact products in another order
    torch.testing.assert_close(got.cpu(), want, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("M,K,N", [(1, 64, 48), (37, 256, 1000), (300, 96, 160)])
def test_bf16_logits_small(M, K, N):
    x = synth.randn((M, K), synth.seed_of("hx", M, K), 1.0).to(torch.bfloat16)
    w = synth.randn((N, K), synth.seed_of("hw", N, K), 0.5).to(torch.bfloat16)
    got = ops.lm_head_logits(x.to(DEV), w.to(DEV)).cpu()
    torch.testing.assert_close(got.double(), x.double() @ w.double().T, rtol=1e-5, atol=1e-5)


def test_argmax_exact_with_ties():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(6, 129280, generator=g)
    logits[1, 500] = logits[1, 70000] = 100.0      # tie: lower index wins
    logits[2] = 0.0                                 # all equal: index 0
    logits[3, -1] = 50.0                            # last position
    got = ops.sample(logits.to(DEV), 0.0, 0.9).cpu()
    assert got.tolist() == H.greedy(logits).tolist()
    assert got[1].item() == 500 and got[2].item() == 0 and got[3].item() == 129279


def test_top_p_draws_from_the_nucleus():
    g = torch.Generator().manual_seed(4)
    for top_p, temp in ((0.0, 1.0), (0.5, 0.7), (0.9, 1.0), (0.99, 1.3)):
        print(f"[case] top_p {top_p} T {temp}", flush=True)
        logits = torch.randn(64, 5000, generator=g) * 2
        kept, _ = H.nucleus(logits, temp, top_p)
        got = ops.sample(logits.to(DEV), temp, top_p, seed=1234).cpu()
        assert kept[torch.arange(64), got].all()
        if top_p == 0.0:
            assert got.tolist() == H.greedy(logits).tolist()


def test_top_p_distribution():
    # one row repeated: every row draws with its own counter, so the rows are independent samples
    logits = torch.tensor([2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -3.0])
    rows = 40000
    lg = logits.repeat(rows, 1)
    got = ops.sample(lg.to(DEV), 0.8, 0.9, seed=99).cpu()
    _, p = H.nucleus(logits[None], 0.8, 0.9)
    freq = torch.bincount(got, minlength=8).double() / rows
    # binomial standard error <= 0.0025 at 40000 draws: 5 sigma
    assert (freq - p[0].double()).abs().max() < 0.0125, (freq, p)
    assert (freq[p[0] == 0] == 0).all()
    # another seed gives another stream
    got2 = ops.sample(lg.to(DEV), 0.8, 0.9, seed=100).cpu()
    assert not torch.equal(got, got2)


def test_empty_inputs():
    w = torch.zeros(48, 64, dtype=torch.bfloat16, device=DEV)
    x = torch.zeros(0, 64, dtype=torch.bfloat16, device=DEV)
    assert ops.lm_head_logits(x, w).shape == (0, 48)
    lg = torch.zeros(0, 48, device=DEV)
    assert ops.sample(lg, 0.0, 0.9).shape == (0,)
    assert ops.sample(lg, 1.0, 0.9).shape == (0,)


def _one_workgroup_per_row(lg, temp, top_p, seed):
    """amla_argmax / amla_sample_top_p (one workgroup per row) through the C-ABI."""
    B, n = lg.shape
    out = torch.empty(B, dtype=torch.int64, device=DEV)
    L, st = ops.lib(), ops._stream_ptr(lg)
    if temp == 0:
        rc = L.amla_argmax(lg.data_ptr(), B, n, lg.stride(0), out.data_ptr(), st)
    else:
        rc = L.amla_sample_top_p(lg.data_ptr(), B, n, lg.stride(0), temp, top_p, seed, out.data_ptr(), st)
    ops.check(rc, "one workgroup per row")
    return out


@pytest.mark.parametrize("rows,n,ld", [(8, 129280, 129280), (1, 129280, 129280), (3, 5000, 5008), (64, 1000, 1000),
                                       (2, 1, 1), (5, 70000, 70001), (600, 3000, 3000)])
def test_chunked_sample_equals_one_workgroup_per_row(rows, n, ld):
    """amla_sample (rows cut into chunks, histograms merged with integer atomics) returns the same
    token as the one-workgroup kernels for every (temperature, top_p, seed), each inside the
    oracle's nucleus.  Half the rows hold logits on a grid of 1/4, so many tokens tie, also at the
    threshold."""
    print(f"[case] chunked sample rows={rows} n={n} ld={ld}", flush=True)
    g = torch.Generator().manual_seed(rows * 1009 + n)
    buf = torch.randn(rows, ld, generator=g) * 2.5
    buf[::2] = torch.round(buf[::2] * 4) / 4
    lg_cpu = buf[:, :n]
    lg = buf.to(DEV)[:, :n]
    got = ops.sample(lg, 0.0, 0.9)
    assert torch.equal(got, _one_workgroup_per_row(lg, 0.0, 0.9, 0)), "temperature 0"
    assert got.cpu().tolist() == H.greedy(lg_cpu).tolist()
    for temp, top_p, seed in ((1.0, 0.9, 11), (0.7, 0.5, 12), (1.3, 0.99, 13), (1.0, 0.0, 14), (1.0, 1.0, 15),
                              (0.9, 5.0, 16), (1.0, 0.9, 2 ** 63 + 17)):
        got = ops.sample(lg, temp, top_p, seed=seed)
        want = _one_workgroup_per_row(lg, temp, top_p, seed)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (temp, top_p, seed)
        kept, _ = H.nucleus(lg_cpu, temp, top_p)
        assert kept[torch.arange(rows), got.cpu()].all(), (temp, top_p, seed)


def test_sample_in_a_hip_graph():
    """ops.sample captured once (workspace from the graph's pool), replayed on new logits with
    eager work between replays: every replay equals the eager call."""
    print("[case] sample graph capture B=8 V=129280", flush=True)
    g = torch.Generator().manual_seed(21)
    inputs = [torch.randn(8, 129280, generator=g) * 2 for _ in range(3)]
    static = inputs[0].to(DEV)
    for temp in (0.0, 0.8):
        ops.sample(static, temp, 0.9, seed=5)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = ops.sample(static, temp, 0.9, seed=5)
        for r, x in enumerate(inputs):
            static.copy_(x.to(DEV))
            eager = ops.sample(x.to(DEV), temp, 0.9, seed=5)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager), (temp, r)


def test_sample_with_masked_tokens():
    """Logits set to -inf (banned tokens) have probability 0: never drawn, by the chunked and the
    one-workgroup kernels alike (the same token), also when top_p >= 1 keeps every token and when
    a single token is left; a near-zero temperature draws the argmax."""
    print("[case] sample with -inf logits", flush=True)
    g = torch.Generator().manual_seed(33)
    rows, n = 8, 129280
    lg_cpu = torch.randn(rows, n, generator=g) * 2
    lg_cpu[torch.rand(rows, n, generator=g) < 0.5] = -float("inf")
    lg_cpu[3, :] = -float("inf")
    lg_cpu[3, 77777] = 1.5                      # one token left
    lg = lg_cpu.to(DEV)
    finite = torch.isfinite(lg_cpu)
    for temp, top_p, seed in ((1.0, 0.9, 1), (1.0, 1.0, 2), (0.7, 5.0, 3), (1.0, 0.0, 4)):
        got = ops.sample(lg, temp, top_p, seed=seed)
        want = _one_workgroup_per_row(lg, temp, top_p, seed)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (temp, top_p)
        got = got.cpu()
        assert finite[torch.arange(rows), got].all(), (temp, top_p)
        assert got[3].item() == 77777
        kept, _ = H.nucleus(lg_cpu, temp, top_p)
        assert kept[torch.arange(rows), got].all(), (temp, top_p)
    cold = ops.sample(lg, 1e-3, 0.9, seed=5).cpu()
    assert cold.tolist() == H.greedy(lg_cpu).tolist()
